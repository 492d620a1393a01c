"""GPU parity of the MoE glue around gather_qmm: routing, sorted dispatch, row take,
SwiGLU, the score-weighted slot reduction and the fused decode entry points. Index work is
bit-exact against the oracle; the bf16 rounding contracts (SwiGLU, down-reduce) are
bit-exact; fused entry points are bit-equal to the split calls they replace."""
import numpy as np
import pytest
import torch

import oracle as O
from helpers import BF16_TOL, bf16_bits, max_err_ratio, to_dev_bf16, to_dev_u32, to_f64, weights
import mi_qmm

pytestmark = pytest.mark.gpu


def _print_case(**kw):
    print("CASE", kw, flush=True)


def _u32(t):
    return t.cpu().numpy().view(np.uint32)


@pytest.mark.parametrize("T,E,k", [(37, 128, 8), (5, 256, 8), (9, 60, 4), (3, 16, 1),
                                   (64, 1000, 16)])
def test_route_topk(dev, T, E, k):
    _print_case(t="route", T=T, E=E, k=k)
    logits = O.randn(T * E, O.seed_for(4, 2)).reshape(T, E)
    logits[0, 3] = logits[0, 7] = logits[0].max() + 1.0   # tie at the top: lower id first
    if T > 1:
        logits[1, :] = 0.5                                  # all equal: ids 0..k-1
    inds, scores = mi_qmm.moe_route_topk(torch.from_numpy(logits).to(dev), k)
    ri, rs = O.route_softmax_topk(logits, k)
    assert np.array_equal(_u32(inds), ri)
    np.testing.assert_allclose(scores.cpu().numpy(), rs, rtol=2e-6, atol=1e-7)
    _, sb = mi_qmm.moe_route_topk(torch.from_numpy(logits).to(dev), k, torch.bfloat16)
    # one bf16 rounding of an fp32 score that matches the oracle's to 2e-6
    d = np.abs(bf16_bits(sb).astype(np.int32) - O.f32_to_bf16(rs).astype(np.int32))
    assert d.max() <= 1


@pytest.mark.parametrize("n,E,k,skew", [(1, 128, 1, False), (8, 128, 8, False),
                                        (1000, 128, 8, False), (4096, 128, 8, True),
                                        (5000, 256, 8, True), (512, 8192, 4, False),
                                        (20000, 4000, 8, True), (3000, 4001, 2, False),
                                        (8192, 64, 8, True), (8193, 64, 8, False),
                                        (8192, 4000, 8, True)])
def test_sort_dispatch(dev, n, E, k, skew):
    _print_case(t="sort", n=n, E=E, k=k, skew=skew)
    rng = np.random.default_rng(n + E)
    flat = rng.integers(0, E, size=n).astype(np.uint32)
    if skew:
        hot = rng.choice(E, 8, replace=False)
        m = rng.random(n) < 0.5
        flat[m] = rng.choice(hot, m.sum())
    order, inv, srt, lhs, seg = mi_qmm.moe_sort_dispatch(to_dev_u32(flat, dev), k, E)
    ro, ri, rsrt, rl = O.sort_dispatch(flat, k)
    assert np.array_equal(_u32(order), ro)
    assert np.array_equal(_u32(inv), ri)
    assert np.array_equal(_u32(srt), rsrt)
    assert np.array_equal(_u32(lhs), rl)
    counts = np.bincount(flat, minlength=E)
    want = np.concatenate([[0], np.cumsum(counts)]).astype(np.uint32)
    assert np.array_equal(_u32(seg), want)


def test_sort_dispatch_out_of_range_ids_sort_last(dev):
    _print_case(t="sort_oob")
    flat = np.array([3, 99, 1, 3, 99, 0], np.uint32)
    order, inv, srt, lhs, seg = mi_qmm.moe_sort_dispatch(to_dev_u32(flat, dev), 2, 4)
    assert _u32(order).tolist() == [5, 2, 0, 3, 1, 4]
    assert _u32(srt).tolist() == [0, 1, 3, 3, 99, 99]
    assert _u32(seg).tolist() == [0, 1, 2, 2, 4]


def test_take_rows(dev):
    _print_case(t="take")
    rng = np.random.default_rng(1)
    x = torch.from_numpy(rng.standard_normal((50, 768)).astype(np.float32)).to(dev).bfloat16()
    idx = rng.integers(0, 50, size=77).astype(np.uint32)
    idx[5] = 1000  # out of range -> zero row
    got = mi_qmm.take_rows(x, to_dev_u32(idx, dev)).cpu()
    ref = x.cpu()[torch.from_numpy(np.minimum(idx, 49).astype(np.int64))]
    ref[5] = 0
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    b = torch.from_numpy(rng.integers(0, 255, size=(9, 3)).astype(np.uint8)).to(dev)
    got = mi_qmm.take_rows(b, to_dev_u32(np.array([8, 0, 4], np.uint32), dev)).cpu()
    assert torch.equal(got, b.cpu()[[8, 0, 4]])


def test_swiglu_exhaustive(dev):
    _print_case(t="swiglu")
    g = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    g = g[~np.isnan(O.bf16_to_f32(g))]
    u = O.f32_to_bf16(np.random.default_rng(2).standard_normal(g.size).astype(np.float32))
    y = mi_qmm.swiglu(to_dev_bf16(g, dev), to_dev_bf16(u, dev))
    assert np.array_equal(bf16_bits(y), O.swiglu_bf16(g, u))
    # a length divisible by 8 takes the 16-byte vector kernel
    g8, u8 = g[: g.size // 8 * 8], u[: g.size // 8 * 8]
    y8 = mi_qmm.swiglu(to_dev_bf16(g8, dev), to_dev_bf16(u8, dev))
    assert np.array_equal(bf16_bits(y8), O.swiglu_bf16(g8, u8))
    # u = 1 and u = 2^-10: the output is bf16(g * sigmoid(g)) (scaled exactly), so a wrong
    # sigmoid rounding shows up unless the product's rounding hides it
    for uv in (0x3F80, 0x3A80):
        u1 = np.full(g.size, uv, dtype=np.uint16)
        y1 = mi_qmm.swiglu(to_dev_bf16(g, dev), to_dev_bf16(u1, dev))
        assert np.array_equal(bf16_bits(y1), O.swiglu_bf16(g, u1))


@pytest.mark.parametrize("N", [2048, 2044])
def test_down_reduce_bit_exact(dev, N):
    _print_case(t="down_reduce", N=N)
    T, k = 6, 8
    rng = np.random.default_rng(3)
    v = O.f32_to_bf16(rng.standard_normal((T, k, N)).astype(np.float32))
    sc = O.f32_to_bf16(rng.random((T, k)).astype(np.float32))
    y = bf16_bits(mi_qmm.moe_down_reduce(to_dev_bf16(v, dev), to_dev_bf16(sc, dev)))
    for t in range(T):
        assert np.array_equal(y[t], O.down_reduce_bf16(v[t], sc[t]))


def _bank(E, N, K, seed, bits=4):
    wq, s, b = weights(E, N, K, bits, 64, seed)
    return wq, s, b


@pytest.mark.parametrize("T,E,k,N,K", [(1, 16, 8, 192, 512), (3, 12, 4, 128, 256),
                                       (2, 8, 4, 256, 2048), (1, 32, 8, 768, 2048),
                                       (4, 24, 6, 512, 1024)])
def test_fused_decode_mlp_matches_split(dev, T, E, k, N, K):
    """gate+up+SwiGLU and down+reduce entry points == split gather_qmm + glue, bit for bit;
    and the split path matches the oracle composition within tolerance."""
    _print_case(t="fused", T=T, E=E, k=k, N=N, K=K)
    rng = np.random.default_rng(T * 100 + E)
    gq, gs_, gb = _bank(E, N, K, 11)
    uq, us, ub = _bank(E, N, K, 12)
    dq, ds, db = _bank(E, K, N, 13)
    x = O.make_x_bf16(T, K, 14)
    inds = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.uint32)
    sc = O.f32_to_bf16(rng.random((T, k)).astype(np.float32))
    D = lambda *a: [to_dev_u32(a[0], dev), to_dev_bf16(a[1], dev), to_dev_bf16(a[2], dev)]  # noqa
    G, U, Dn = D(gq, gs_, gb), D(uq, us, ub), D(dq, ds, db)
    xd, idd, scd = to_dev_bf16(x, dev), to_dev_u32(inds, dev), to_dev_bf16(sc, dev)

    act = mi_qmm.gather_qmv_gate_up_swiglu(xd, *G, *U, idd, group_size=64, bits=4)
    xg = xd.reshape(T, 1, 1, K)
    g_split = mi_qmm.gather_qmm(xg, *G, rhs_indices=idd, group_size=64, bits=4)
    u_split = mi_qmm.gather_qmm(xg, *U, rhs_indices=idd, group_size=64, bits=4)
    act_split = mi_qmm.swiglu(g_split, u_split).reshape(T, k, N)
    assert torch.equal(act.view(torch.int16), act_split.view(torch.int16))

    y = mi_qmm.gather_qmv_down_reduce(act, *Dn, idd, scd, group_size=64, bits=4)
    v_split = mi_qmm.gather_qmm(act.reshape(T * k, 1, N), *Dn, rhs_indices=idd.reshape(-1),
                                group_size=64, bits=4)
    y_split = mi_qmm.moe_down_reduce(v_split.reshape(T, k, K), scd)
    assert torch.equal(y.view(torch.int16), y_split.view(torch.int16))

    # split path against the oracle: gate/up products, then the bf16 glue on GPU values
    tg = O.gather_qmm_f64(x.reshape(T, 1, K), gq, gs_, gb, None, inds.reshape(-1), T * k,
                          lhs_div=k)
    assert max_err_ratio(to_f64(g_split).reshape(T * k, 1, N), tg) <= BF16_TOL
    a_np = bf16_bits(act).reshape(T * k, N)
    assert np.array_equal(a_np, O.swiglu_bf16(bf16_bits(g_split).reshape(T * k, N),
                                              bf16_bits(u_split).reshape(T * k, N)))
    tv = O.gather_qmm_f64(a_np.reshape(T * k, 1, N), dq, ds, db, None, inds.reshape(-1), T * k)
    assert max_err_ratio(to_f64(v_split).reshape(T * k, 1, K), tv) <= BF16_TOL


def test_down_reduce_out_of_range_expert(dev):
    """An expert id >= E gives NaN for its slot (the one-row kernel's rule), so the token's
    row is NaN; the other tokens are unaffected. One-launch and split paths agree bitwise."""
    _print_case(t="down_oob")
    T, E, k, N, K = 3, 16, 8, 768, 2048
    rng = np.random.default_rng(5)
    dq, ds, db = _bank(E, K, N, 31)
    a = O.make_x_bf16(T * k, N, 32)
    inds = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.uint32)
    inds[1, 3] = E + 7
    sc = O.f32_to_bf16(rng.random((T, k)).astype(np.float32))
    Dn = [to_dev_u32(dq, dev), to_dev_bf16(ds, dev), to_dev_bf16(db, dev)]
    ad, idd, scd = to_dev_bf16(a, dev), to_dev_u32(inds, dev), to_dev_bf16(sc, dev)
    y = mi_qmm.gather_qmv_down_reduce(ad.reshape(T, k, N), *Dn, idd, scd, group_size=64, bits=4)
    v_split = mi_qmm.gather_qmm(ad.reshape(T * k, 1, N), *Dn, rhs_indices=idd.reshape(-1),
                                group_size=64, bits=4)
    y_split = mi_qmm.moe_down_reduce(v_split.reshape(T, k, K), scd)
    assert torch.equal(y.view(torch.int16), y_split.view(torch.int16))
    yf = to_f64(y)
    assert np.isnan(yf[1]).all() and not np.isnan(yf[0]).any() and not np.isnan(yf[2]).any()
    ok = inds.copy()
    ok[1, 3] = 0
    tv = O.gather_qmm_f64(a.reshape(T * k, 1, N), dq, ds, db, None, ok.reshape(-1), T * k)
    assert max_err_ratio(to_f64(v_split).reshape(T * k, 1, K)[[0, 1, 2, 16, 17]],
                         tv[[0, 1, 2, 16, 17]]) <= BF16_TOL


def test_sorted_moe_pipeline_end_to_end(dev):
    """Router -> sort -> gather_qmm(sorted, lhs = order//k) -> take_rows(inv) equals the
    unsorted per-(token, slot) products (the reference's sorted prefill path, :14961-15043)."""
    _print_case(t="pipeline")
    T, E, k, N, K = 48, 16, 4, 96, 512
    logits = O.randn(T * E, O.seed_for(4, 2)).reshape(T, E)
    inds, _ = mi_qmm.moe_route_topk(torch.from_numpy(logits).to(dev), k)
    order, inv, srt, lhs, seg = mi_qmm.moe_sort_dispatch(inds.reshape(-1), k, E)
    wq, s, b = _bank(E, N, K, 21)
    x = O.make_x_bf16(T, K, 22)
    xd = to_dev_bf16(x, dev).reshape(T, 1, K)
    W = [to_dev_u32(wq, dev), to_dev_bf16(s, dev), to_dev_bf16(b, dev)]
    ys = mi_qmm.gather_qmm(xd, *W, lhs_indices=lhs, rhs_indices=srt, group_size=64, bits=4,
                           sorted_indices=True)
    y = mi_qmm.take_rows(ys.reshape(T * k, N), inv)
    ri, _ = O.route_softmax_topk(logits, k)
    truth = O.gather_qmm_f64(x.reshape(T, 1, K), wq, s, b, None, ri.reshape(-1), T * k, lhs_div=k)
    assert max_err_ratio(to_f64(y).reshape(T * k, 1, N), truth) <= BF16_TOL


@pytest.mark.parametrize("T,E,k,N,K", [(1, 128, 8, 768, 2048), (1, 256, 8, 2048, 7168),
                                       (3, 60, 4, 256, 1024), (2, 16, 2, 192, 512),
                                       (1, 300, 8, 128, 512)])
def test_route_fused_gate_up_matches_split(dev, T, E, k, N, K):
    """Routing inside the gate+up launch: indices and bf16 scores equal mi_moe_route_topk's,
    and the activations equal the fused gate+up call on those indices, bit for bit (E=300
    takes the two-call path)."""
    _print_case(t="route_fused", T=T, E=E, k=k, N=N, K=K)
    gq, gs_, gb = _bank(E, N, K, 21)
    uq, us, ub = _bank(E, N, K, 22)
    D = lambda *a: [to_dev_u32(a[0], dev), to_dev_bf16(a[1], dev), to_dev_bf16(a[2], dev)]  # noqa
    G, U = D(gq, gs_, gb), D(uq, us, ub)
    x = to_dev_bf16(O.make_x_bf16(T, K, 23), dev)
    logits = torch.from_numpy(O.randn(T * E, 24).reshape(T, E)).to(dev)
    y, inds, sc = mi_qmm.moe_route_gate_up_swiglu(logits, x, *G, *U, k, group_size=64, bits=4)
    ri, rs = mi_qmm.moe_route_topk(logits, k, torch.bfloat16)
    assert torch.equal(inds, ri) and torch.equal(sc.view(torch.int16), rs.view(torch.int16))
    act = mi_qmm.gather_qmv_gate_up_swiglu(x, *G, *U, ri, group_size=64, bits=4)
    assert torch.equal(y.view(torch.int16), act.view(torch.int16))


@pytest.mark.parametrize("E,k,ng,tg", [(512, 8, 8, 4), (256, 8, 8, 4), (64, 4, 4, 2),
                                       (128, 6, 1, 1)])
def test_route_grouped_matches_oracle(dev, E, k, ng, tg):
    """Group-limited routing against the float64 oracle (the reference test's own
    reference, src/transformer.zig:23390): indices exact on 256 rows of the reference
    test's data shape, weights within 1e-5 relative."""
    _print_case(t="route_grouped", E=E, k=k, ng=ng, tg=tg)
    rng = np.random.default_rng(E + ng)
    T = 256
    logits = ((rng.random((T, E)) - 0.5) * 6.0 + (np.arange(T * E) % 7).reshape(T, E) * 0.011)
    logits = logits.astype(np.float32)
    bias = ((rng.random(E) - 0.5) * 0.2).astype(np.float32)
    inds, w = mi_qmm.moe_route_grouped(torch.from_numpy(logits).to(dev),
                                       torch.from_numpy(bias).to(dev), k, ng, tg, True, 2.5)
    ri, rw = O.route_grouped(logits, bias, k, ng, tg, True, 2.5)
    assert np.array_equal(_u32(inds), ri)
    wg = w.cpu().numpy().astype(np.float64)
    assert np.max(np.abs(wg - rw) / np.abs(rw)) <= 1e-5
    if ng > tg:  # the limit must bite on this data: some rows differ from the unmasked top-k
        free, _ = O.route_grouped(logits, bias, k, ng, ng, True, 2.5)
        assert (np.sort(free, axis=1) != np.sort(ri, axis=1)).any()


def _fp_bank(mode, E, N, K, seed):
    m, bits, gs = O.FP_MODES[mode]
    rng = np.random.default_rng(seed)
    q = rng.integers(0, 1 << bits, size=(E * N, K)).astype(np.uint8)
    # scales for weights of a realistic size: random e4m3 codes reach +-480, so mxfp8 takes
    # e8m0 scales 2^-17..2^-14 (|w| <= 0.03) and the fused MLP's activations stay well inside
    # fp32 exp range; the 4-bit modes' codes stop at +-6
    lo, hi = {"nvfp4": (0x20, 0x48), "mxfp4": (118, 126), "mxfp8": (110, 114)}[mode]
    sc = rng.integers(lo, hi, size=(E, N, K // gs)).astype(np.uint8)
    return O.pack(q, bits).reshape(E, N, -1), sc


@pytest.mark.parametrize("mode", ["nvfp4", "mxfp4", "mxfp8"])
@pytest.mark.parametrize("T", [1, 3])
def test_fused_decode_mlp_fp_modes(dev, mode, T):
    """The fused decode MoE entry points at the bias-less modes: gate + up + SwiGLU and
    down + slot sum are bit-equal to the split calls (gather_qmm, swiglu, moe_down_reduce),
    the routed variant equals route + fused, and the whole MLP is within tolerance of fp64."""
    _print_case(t="fused_fp", mode=mode, T=T)
    E, k, N, K = 16, 4, 256, 512
    wg, sg = _fp_bank(mode, E, N, K, 70)
    wu, su = _fp_bank(mode, E, N, K, 71)
    wd, sd = _fp_bank(mode, E, K, N, 72)
    D = lambda a: to_dev_u32(a, dev)
    S = lambda a: torch.from_numpy(a).to(dev)
    x = O.make_x_bf16(T, K, 73)
    logits = torch.from_numpy(O.randn(T * E, 74).reshape(T, E)).to(dev)
    inds, sc = mi_qmm.moe_route_topk(logits, k, torch.bfloat16)
    xd = to_dev_bf16(x, dev)
    act = mi_qmm.gather_qmv_gate_up_swiglu(xd, D(wg), S(sg), None, D(wu), S(su), None, inds,
                                           mode=mode)
    # split: two gathers and SwiGLU
    lhs = to_dev_u32(np.repeat(np.arange(T, dtype=np.uint32), k), dev)
    rhs = inds.reshape(-1)
    g = mi_qmm.gather_qmm(xd.view(T, 1, K), D(wg), S(sg), None, lhs_indices=lhs,
                          rhs_indices=rhs, mode=mode)
    u = mi_qmm.gather_qmm(xd.view(T, 1, K), D(wu), S(su), None, lhs_indices=lhs,
                          rhs_indices=rhs, mode=mode)
    act_split = mi_qmm.swiglu(g, u).view(T, k, N)
    assert np.array_equal(bf16_bits(act), bf16_bits(act_split))
    a2, i2, s2 = mi_qmm.moe_route_gate_up_swiglu(logits, xd, D(wg), S(sg), None, D(wu), S(su),
                                                 None, k, mode=mode)
    assert torch.equal(i2.view(torch.int32), inds.view(torch.int32))
    assert np.array_equal(bf16_bits(a2), bf16_bits(act))
    y = mi_qmm.gather_qmv_down_reduce(act, D(wd), S(sd), None, inds, sc, mode=mode)
    v = mi_qmm.gather_qmm(act.view(T * k, 1, N), D(wd), S(sd), None, rhs_indices=rhs, mode=mode)
    y_split = mi_qmm.moe_down_reduce(v.view(T, k, K), sc)
    assert np.array_equal(bf16_bits(y), bf16_bits(y_split))
    # fp64 truth of the whole routed MLP over the same routing
    ii = inds.view(torch.int32).cpu().numpy()
    scf = sc.float().cpu().numpy().astype(np.float64)
    xf = O.bf16_to_f32(x).astype(np.float64)
    deq = lambda w, s_, e: O.dequantize_fp(w[e], s_[e], mode).astype(np.float64)
    want = np.zeros((T, K))
    for t in range(T):
        for j in range(k):
            e = ii[t, j]
            gg, uu = xf[t] @ deq(wg, sg, e).T, xf[t] @ deq(wu, su, e).T
            h = gg / (1.0 + np.exp(-gg)) * uu
            want[t] += scf[t, j] * (h @ deq(wd, sd, e).T)
    assert max_err_ratio(to_f64(y), want) <= 3 * BF16_TOL


@pytest.mark.parametrize("T,E,k,N,K", [(512, 16, 4, 256, 512), (3, 16, 2, 192, 512),
                                       (64, 128, 8, 768, 2048), (40, 8, 2, 100, 256),
                                       (8, 16, 4, 256, 1024), (16, 64, 8, 512, 7168)])
def test_sorted_up_swiglu_and_unsort_reduce_match_split(dev, T, E, k, N, K):
    """The fused sorted-path entries equal the split calls bit for bit: gather_qmm_swiglu ==
    swiglu(gate, gather_qmm) and gather_qmm_gate_up_swiglu == both (grouped kernel at T=512,
    the one-row kernel at T=3, the few-row kernel at T=8 and 16 (a K split at K=7168), the
    tile kernel at N=100), and moe_down_reduce_rows ==
    moe_down_reduce(take_rows(v, inv))."""
    _print_case(t="sorted_fused", T=T, E=E, k=k, N=N, K=K)
    logits = torch.from_numpy(O.randn(T * E, 31).reshape(T, E)).to(dev)
    inds, sc = mi_qmm.moe_route_topk(logits, k, torch.bfloat16)
    order, inv, srt, lhs, seg = mi_qmm.moe_sort_dispatch(inds.reshape(-1), k, E)
    D = lambda *a: [to_dev_u32(a[0], dev), to_dev_bf16(a[1], dev), to_dev_bf16(a[2], dev)]  # noqa
    G, U = D(*_bank(E, N, K, 32)), D(*_bank(E, N, K, 33))
    x = to_dev_bf16(O.make_x_bf16(T, K, 34), dev).reshape(T, 1, K)
    kw = dict(lhs_indices=lhs, rhs_indices=srt, group_size=64, bits=4, sorted_indices=True)
    g = mi_qmm.gather_qmm(x, *G, **kw)
    u = mi_qmm.gather_qmm(x, *U, **kw)
    split = mi_qmm.swiglu(g, u)
    fused = mi_qmm.gather_qmm_swiglu(g, x, *U, **kw)
    assert torch.equal(fused.view(torch.int16), split.view(torch.int16))
    both = mi_qmm.gather_qmm_gate_up_swiglu(x, *G, *U, **kw)  # one launch on the grouped kernel
    assert torch.equal(both.view(torch.int16), split.view(torch.int16))
    v = to_dev_bf16(O.make_x_bf16(T * k, N, 35), dev)
    ref = mi_qmm.moe_down_reduce(mi_qmm.take_rows(v, inv).view(T, k, N), sc)
    got = mi_qmm.moe_down_reduce_rows(v, inv, sc)
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    bad = inv.clone()
    bad[1] = T * k + 7                      # out of range: a zero row, as take_rows gives
    ref = mi_qmm.moe_down_reduce(mi_qmm.take_rows(v, bad).view(T, k, N), sc)
    got = mi_qmm.moe_down_reduce_rows(v, bad, sc)
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))


@pytest.mark.parametrize("n_pairs,E", [(6, 16), (40, 64)])
def test_gate_up_swiglu_one_row_items_bad_rows(dev, n_pairs, E):
    """Sorted one-row items on the dual one-row launch: an expert id past E and an lhs index
    past the batch give NaN rows, as the split calls do, and every row is bit-equal to them."""
    _print_case(t="gate_up_bad_rows", n_pairs=n_pairs, E=E)
    N, K = 128, 512
    rng = np.random.default_rng(n_pairs)
    rhs = np.sort(rng.choice(E, size=n_pairs, replace=False)).astype(np.uint32)
    rhs[-1] = E + 3                      # unknown expert: sorts last
    lhs = rng.integers(0, n_pairs, size=n_pairs).astype(np.uint32)
    lhs[1] = 10 * n_pairs                # row past the batch
    D = lambda *a: [to_dev_u32(a[0], dev), to_dev_bf16(a[1], dev), to_dev_bf16(a[2], dev)]  # noqa
    G, U = D(*_bank(E, N, K, 41)), D(*_bank(E, N, K, 42))
    x = to_dev_bf16(O.make_x_bf16(n_pairs, K, 43), dev).reshape(n_pairs, 1, K)
    kw = dict(lhs_indices=to_dev_u32(lhs, dev), rhs_indices=to_dev_u32(rhs, dev), group_size=64,
              bits=4, sorted_indices=True)
    g = mi_qmm.gather_qmm(x, *G, **kw)
    split = mi_qmm.gather_qmm_swiglu(g, x, *U, **kw)
    both = mi_qmm.gather_qmm_gate_up_swiglu(x, *G, *U, **kw)
    assert torch.equal(both.view(torch.int16), split.view(torch.int16))
    bf = to_f64(both).reshape(n_pairs, N)
    assert np.isnan(bf[1]).all() and np.isnan(bf[-1]).all()
    assert not np.isnan(np.delete(bf, [1, n_pairs - 1], axis=0)).any()


def test_gather_qmm_swiglu_unsorted_tile_kernel(dev):
    """Unsorted 16-row pairs run on the tile kernels, which write the product and then apply
    SwiGLU in place: still bit-equal to the two calls."""
    _print_case(t="swiglu_tile")
    E, N, K, n = 6, 256, 512, 5
    W = [to_dev_u32(a, dev) if i == 0 else to_dev_bf16(a, dev)
         for i, a in enumerate(_bank(E, N, K, 36))]
    x = to_dev_bf16(O.make_x_bf16(n * 16, K, 37), dev).reshape(n, 16, K)
    rhs = torch.tensor([3, 0, 5, 3, 1], dtype=torch.int32, device=dev)
    gate = to_dev_bf16(O.make_x_bf16(n * 16, N, 38), dev).reshape(n, 16, N)
    up = mi_qmm.gather_qmm(x, *W, rhs_indices=rhs, group_size=64, bits=4)
    fused = mi_qmm.gather_qmm_swiglu(gate, x, *W, rhs_indices=rhs, group_size=64, bits=4)
    assert torch.equal(fused.view(torch.int16), mi_qmm.swiglu(gate, up).view(torch.int16))
