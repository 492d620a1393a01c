"""GPU parity of libmi_qmm.so against the CPU oracle (calls go through the C ABI via
mi_qmm's ctypes binding). Tolerances: bf16 output max-abs-err <= 1e-2*||y||inf,
fp32 output <= 1e-3*||y||inf, both against fp64 truth on exactly dequantized
weights; dequantize/quantize/indices are bit-exact."""
import numpy as np
import pytest
import torch

import oracle as O
from helpers import (BF16_TOL, F32_TOL, bf16_bits, max_err_ratio, to_dev_bf16, to_dev_u32,
                     to_f64, weights)
import mi_qmm

pytestmark = pytest.mark.gpu


def _print_case(**kw):
    print("CASE", kw, flush=True)


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
def test_dequantize_bit_exact(dev, bits, gs):
    _print_case(t="dequant", bits=bits, gs=gs)
    wq, s, b = weights(1, 96, 512, bits, gs, 11)
    wq, s, b = wq[0], s[0], b[0]
    W, S, B = to_dev_u32(wq, dev), to_dev_bf16(s, dev), to_dev_bf16(b, dev)
    f32 = mi_qmm.dequantize(W, S, B, gs, bits, dtype=torch.float32).cpu().numpy()
    assert np.array_equal(f32.view(np.uint32),
                          O.dequantize(wq, s, b, gs, bits, O.DQ_F32).view(np.uint32))
    for rounding, kind in ((1, O.DQ_BF16_OPWISE), (0, O.DQ_BF16_FUSED)):
        got = bf16_bits(mi_qmm.dequantize(W, S, B, gs, bits, dtype=torch.bfloat16,
                                          rounding=rounding))
        assert np.array_equal(got, O.dequantize(wq, s, b, gs, bits, kind))


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
def test_quantize_bit_exact(dev, bits, gs):
    _print_case(t="quant", bits=bits, gs=gs)
    w = O.f32_to_bf16(O.randn(64 * 512, 21, 0.0, 0.02).reshape(64, 512))
    # a few adversarial groups: constant, all-zero, one outlier, exact grid
    w[0, :gs] = O.f32_to_bf16(np.full(gs, 0.5, np.float32))
    w[1, :gs] = 0
    w[2, :gs] = O.f32_to_bf16(np.r_[np.zeros(gs - 1), [3.0]].astype(np.float32))
    w[3, :gs] = O.f32_to_bf16((np.arange(gs) % 16 - 5).astype(np.float32) * 0.125)
    wq, s, b = mi_qmm.quantize(to_dev_bf16(w, dev), gs, bits)
    rq, rs, rb = O.quantize(w, gs, bits)
    assert np.array_equal(wq.cpu().numpy().view(np.uint32), rq)
    assert np.array_equal(bf16_bits(s), rs)
    assert np.array_equal(bf16_bits(b), rb)


QMM_CASES = [(1, 4096, 512), (1, 100, 1024), (2, 64, 256), (3, 48, 512), (4, 80, 256),
             (5, 32, 384), (8, 64, 512), (16, 64, 256), (17, 40, 256), (32, 96, 512),
             (33, 64, 256), (64, 48, 256), (1, 1024, 4096), (3, 512, 8192), (16, 256, 4096),
             (1, 320, 14336), (5, 48, 2560), (1, 64, 2176), (1, 200, 3200), (1, 8, 256),
             (32, 256, 8192), (12, 320, 14336), (7, 4096, 1024), (48, 320, 8192),
             (64, 512, 2048), (40, 200, 3200)]


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("M,N,K", QMM_CASES)
def test_qmm_bf16(dev, M, N, K, bits, gs):
    if K % gs:
        pytest.skip("K not a multiple of gs")
    _print_case(t="qmm_bf16", M=M, N=N, K=K, bits=bits, gs=gs)
    wq, s, b = weights(1, N, K, bits, gs, 1000 + M)
    x = O.make_x_bf16(M, K, 2000 + N)
    y = mi_qmm.quantized_matmul(to_dev_bf16(x, dev), to_dev_u32(wq[0], dev),
                                to_dev_bf16(s[0], dev), to_dev_bf16(b[0], dev), True, gs, bits)
    truth = O.qmm_f64(x, wq[0], s[0], b[0], gs, bits)
    assert y.shape == (M, N) and y.dtype == torch.bfloat16
    assert max_err_ratio(to_f64(y), truth) <= BF16_TOL


@pytest.mark.parametrize("bits", [2, 3, 5, 6])
@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("M,N,K", [(1, 256, 1024), (7, 96, 512), (8, 100, 2048), (2, 50, 256),
                                   (300, 64, 384)])
def test_qmm_other_widths(dev, M, N, K, bits, gs):
    """2/3/5/6-bit weights: up to 8 rows read the packed bitstream directly (qmv_any),
    more rows dequantize to bf16 and run the bf16 GEMM."""
    _print_case(t="qmm_width", M=M, N=N, K=K, bits=bits, gs=gs)
    wq, s, b = weights(1, N, K, bits, gs, 3000 + bits)
    x = O.make_x_bf16(M, K, 4000 + M)
    y = mi_qmm.quantized_matmul(to_dev_bf16(x, dev), to_dev_u32(wq[0], dev),
                                to_dev_bf16(s[0], dev), to_dev_bf16(b[0], dev), True, gs, bits)
    truth = O.qmm_f64(x, wq[0], s[0], b[0], gs, bits)
    assert y.shape == (M, N) and y.dtype == torch.bfloat16
    assert max_err_ratio(to_f64(y), truth) <= BF16_TOL


@pytest.mark.parametrize("bits", [2, 3, 5, 6, 8])
@pytest.mark.parametrize("N,K", [(320, 14336), (64, 2176), (4096, 1024), (100, 4096)])
def test_qmm_other_widths_one_row(dev, bits, N, K):
    """One row of 2/3/5/6/8-bit gs 64 on the one-row streaming kernel's other-width instances
    (K = 2176: 17 chunks, a K-split plan and the fixed-order reduce)."""
    _print_case(t="qmm_odd_one_row", bits=bits, N=N, K=K)
    wq, s, b = weights(1, N, K, bits, 64, 4000 + bits)
    x = O.make_x_bf16(1, K, 4100 + N)
    y = mi_qmm.quantized_matmul(to_dev_bf16(x, dev), to_dev_u32(wq[0], dev),
                                to_dev_bf16(s[0], dev), to_dev_bf16(b[0], dev), True, 64, bits)
    truth = O.qmm_f64(x, wq[0], s[0], b[0], 64, bits)
    assert max_err_ratio(to_f64(y), truth) <= BF16_TOL


@pytest.mark.parametrize("bits", [3, 5, 6])
def test_gather_other_widths(dev, bits):
    """2/3/5/6-bit gathers: one token broadcast over its slots, one slot out of range
    (NaN row); truth is the oracle's fp64 gather."""
    _print_case(t="gather_width", bits=bits)
    E, N, K, T, k = 4, 48, 256, 3, 2
    wq, s, b = weights(E, N, K, bits, 64, 5 + bits)
    x = O.make_x_bf16(T, K, 6)
    inds = np.array([[1, 3], [0, E + 2], [2, 2]], np.uint32)
    y = mi_qmm.gather_qmm(to_dev_bf16(x, dev).reshape(T, 1, 1, K), to_dev_u32(wq, dev),
                          to_dev_bf16(s, dev), to_dev_bf16(b, dev),
                          rhs_indices=to_dev_u32(inds, dev), group_size=64, bits=bits)
    yf = to_f64(y).reshape(T * k, 1, N)
    assert np.isnan(yf[3]).all()
    ok = inds.reshape(-1).copy()
    ok[3] = 0
    truth = O.gather_qmm_f64(x.reshape(T, 1, K), wq, s, b, None, ok, T * k, lhs_div=k,
                             group_size=64, bits=bits)
    keep = [0, 1, 2, 4, 5]
    assert max_err_ratio(yf[keep], truth[keep]) <= BF16_TOL


@pytest.mark.parametrize("mode", ["nvfp4", "mxfp4", "mxfp8"])
def test_gather_fp_modes(dev, mode):
    _print_case(t="gather_fp", mode=mode)
    E, N, K, T = 3, 40, 512, 4
    banks = [_fp_weight(mode, N, K, 30 + e) for e in range(E)]
    wq = np.stack([bk[0] for bk in banks])
    sc = np.stack([bk[1] for bk in banks])
    x = O.make_x_bf16(T * 2, K, 31).reshape(T, 2, K)  # 2 rows per pair
    rhs = np.array([2, 0, 1, 2], np.uint32)
    y = mi_qmm.gather_qmm(to_dev_bf16(x, dev), to_dev_u32(wq, dev), torch.from_numpy(sc).to(dev),
                          None, lhs_indices=to_dev_u32(np.arange(T, dtype=np.uint32), dev),
                          rhs_indices=to_dev_u32(rhs, dev), mode=mode)
    xf = O.bf16_to_f32(x).astype(np.float64)
    truth = np.stack([xf[i] @ O.dequantize_fp(wq[rhs[i]], sc[rhs[i]], mode).astype(np.float64).T
                      for i in range(T)])
    assert max_err_ratio(to_f64(y).reshape(T, 2, N), truth) <= BF16_TOL


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("M,N,K", [(1, 256, 1024), (3, 64, 512), (20, 48, 256)])
def test_qmm_f32(dev, M, N, K, bits):
    _print_case(t="qmm_f32", M=M, N=N, K=K, bits=bits)
    wq, s, b = weights(1, N, K, bits, 64, 3000 + M)
    x = O.randn(M * K, 4000 + N).reshape(M, K)
    y = mi_qmm.quantized_matmul(torch.from_numpy(x).to(dev), to_dev_u32(wq[0], dev),
                                to_dev_bf16(s[0], dev), to_dev_bf16(b[0], dev), True, 64, bits)
    truth = O.qmm_f64(x, wq[0], s[0], b[0], 64, bits)
    assert y.dtype == torch.float32
    assert max_err_ratio(y.cpu().numpy().astype(np.float64), truth) <= F32_TOL


def test_qmm_special_cases(dev):
    """One-hot x reads out one dequantized column; scale 1 / bias 0 integer weights
    give an exact integer matmul."""
    _print_case(t="special")
    N, K = 64, 256
    q = (np.arange(N * K) * 7 % 16).astype(np.uint8).reshape(N, K)
    wq = O.pack(q, 4)
    one = O.f32_to_bf16(np.ones((N, K // 64), np.float32))
    zero = np.zeros((N, K // 64), np.uint16)
    x = np.zeros((4, K), np.float32)
    x[0, 5] = 1.0
    x[1, :] = 1.0
    x[2, ::3] = 2.0
    x[3] = (np.arange(K) % 5).astype(np.float32)
    xb = O.f32_to_bf16(x)
    y = mi_qmm.quantized_matmul(to_dev_bf16(xb, dev), to_dev_u32(wq, dev), to_dev_bf16(one, dev),
                                to_dev_bf16(zero, dev), True, 64, 4)
    exact = x.astype(np.float64) @ q.T.astype(np.float64)
    got = to_f64(y)
    # bf16 output holds integers up to 256 exactly; compare after bf16 rounding
    assert np.array_equal(got, O.bf16_to_f32(O.f32_to_bf16(exact.astype(np.float32))))
    assert np.array_equal(got[0], q[:, 5].astype(np.float64))


def test_gather_decode_broadcast(dev):
    """Reference decode call: x [B,S,1,1,D] with inds [B,S,K], no lhs (lhs = i / K)."""
    _print_case(t="gather_decode")
    E, N, K, topk = 16, 96, 512, 4
    wq, s, b = weights(E, N, K, 4, 64, 55)
    x = O.make_x_bf16(2, K, 56)  # B*S = 2 tokens
    inds = np.array([[3, 0, 15, 7], [7, 7, 2, 9]], np.uint32)
    xd = to_dev_bf16(x, dev).reshape(1, 2, 1, 1, K)
    y = mi_qmm.gather_qmm(xd, to_dev_u32(wq, dev), to_dev_bf16(s, dev), to_dev_bf16(b, dev),
                          rhs_indices=to_dev_u32(inds.reshape(1, 2, topk), dev), group_size=64,
                          bits=4)
    assert y.shape == (1, 2, topk, 1, N)
    truth = O.gather_qmm_f64(x.reshape(2, 1, K), wq, s, b, None, inds.reshape(-1), 2 * topk,
                             lhs_div=topk)
    assert max_err_ratio(to_f64(y).reshape(2 * topk, 1, N), truth) <= BF16_TOL


@pytest.mark.parametrize("M,K,E,T,topk", [(1, 256, 8, 40, 3), (3, 256, 8, 40, 3),
                                          (1, 1024, 8, 40, 3), (2, 2048, 8, 40, 3),
                                          (1, 512, 64, 20, 2), (1, 512, 40, 30, 2),
                                          (1, 1024, 32, 40, 3), (2, 512, 16, 24, 2),
                                          (1, 512, 4, 64, 4), (1, 8192, 4, 64, 4),
                                          (1, 256, 16, 3000, 4), (2, 256, 300, 2600, 2),
                                          (1, 768, 6, 120, 4)])
def test_gather_sorted_matches_unsorted(dev, M, K, E, T, topk):
    """Sorted (grouped) path and unsorted path both match truth; the shapes cover work
    items of 1 row (one-row kernel), 2..32 rows (few-row MFMA kernel, K split across
    blocks for K=8192) and the older 16/32-row-tile kernels; 12000 and 5200 pairs take
    several passes of the work-item builder."""
    _print_case(t="gather_sorted", M=M, K=K, E=E, T=T, topk=topk)
    N = 64
    wq, s, b = weights(E, N, K, 4, 64, 77)
    rng = np.random.default_rng(5)
    flat = rng.integers(0, E, size=T * topk).astype(np.uint32)
    order, inv, srt, lhs = O.sort_dispatch(flat, topk)
    x = O.make_x_bf16(T * M, K, 78).reshape(T, M, K)
    Wd, Sd, Bd = to_dev_u32(wq, dev), to_dev_bf16(s, dev), to_dev_bf16(b, dev)
    xd = to_dev_bf16(x, dev)
    ys = mi_qmm.gather_qmm(xd, Wd, Sd, Bd, lhs_indices=to_dev_u32(lhs, dev),
                           rhs_indices=to_dev_u32(srt, dev), group_size=64, bits=4,
                           sorted_indices=True)
    yu = mi_qmm.gather_qmm(xd, Wd, Sd, Bd, lhs_indices=to_dev_u32(lhs, dev),
                           rhs_indices=to_dev_u32(srt, dev), group_size=64, bits=4,
                           sorted_indices=False)
    truth = O.gather_qmm_f64(x, wq, s, b, lhs, srt, T * topk)
    assert max_err_ratio(to_f64(ys), truth) <= BF16_TOL
    assert max_err_ratio(to_f64(yu), truth) <= BF16_TOL
    # permuting back gives the per-(token, slot) result
    back = to_f64(ys)[inv]
    t2 = O.gather_qmm_f64(x, wq, s, b, None, flat, T * topk, lhs_div=topk)
    assert max_err_ratio(back, t2) <= BF16_TOL


@pytest.mark.parametrize("N,K,E,T,topk,skew", [(200, 256, 8, 64, 4, False),
                                                 (1536, 2048, 16, 96, 4, True),
                                                 (260, 768, 4, 100, 2, True)])
def test_gather_sorted_grouped_kernel(dev, N, K, E, T, topk, skew):
    """Sorted gathers that average several rows per expert run the grouped kernel (one
    block per work item x 128-row weight tile): widths that end in a partial tile, items of
    32 and 64 rows, and skewed routings whose hot experts are cut into several items."""
    _print_case(t="gather_grouped", N=N, K=K, E=E, T=T, topk=topk, skew=skew)
    wq, s, b = weights(E, N, K, 4, 64, 210 + N)
    rng = np.random.default_rng(N + K)
    p = np.ones(E) / E
    if skew:
        p = np.ones(E)
        p[: max(1, E // 8)] = 4.0 * E / max(1, E // 8)
        p /= p.sum()
    flat = rng.choice(E, size=T * topk, p=p).astype(np.uint32)
    order, inv, srt, lhs = O.sort_dispatch(flat, topk)
    x = O.make_x_bf16(T, K, 211 + K).reshape(T, 1, K)
    y = mi_qmm.gather_qmm(to_dev_bf16(x, dev), to_dev_u32(wq, dev), to_dev_bf16(s, dev),
                          to_dev_bf16(b, dev), lhs_indices=to_dev_u32(lhs, dev),
                          rhs_indices=to_dev_u32(srt, dev), group_size=64, bits=4,
                          sorted_indices=True)
    truth = O.gather_qmm_f64(x, wq, s, b, lhs, srt, T * topk)
    assert max_err_ratio(to_f64(y), truth) <= BF16_TOL


@pytest.mark.parametrize("N,K,E,T,topk,skew", [(512, 7168, 16, 8, 4, False),
                                                 (2048, 2048, 16, 4, 8, True),
                                                 (200, 1024, 32, 16, 4, True),
                                                 (64, 4096, 8, 6, 2, False)])
def test_gather_sorted_rows_kernel(dev, N, K, E, T, topk, skew):
    """Sorted gathers of a few rows per expert (configs[4]-like: ~2.3 rows a distinct
    expert) on the few-row kernel's work items; skewed routings put runs longer than one
    item on hot experts (cut into several items); K = 7168 and 4096 take K splits."""
    _print_case(t="gather_rows", N=N, K=K, E=E, T=T, topk=topk, skew=skew)
    wq, s, b = weights(E, N, K, 4, 64, 230 + E)
    rng = np.random.default_rng(N + K + E)
    p = np.ones(E) / E
    if skew:
        p = np.ones(E)
        p[:2] = E
        p /= p.sum()
    flat = np.stack([rng.choice(E, size=topk, replace=False, p=p) for _ in range(T)])
    flat = flat.reshape(-1).astype(np.uint32)
    order, inv, srt, lhs = O.sort_dispatch(flat, topk)
    x = O.make_x_bf16(T, K, 231 + K).reshape(T, 1, K)
    y = mi_qmm.gather_qmm(to_dev_bf16(x, dev), to_dev_u32(wq, dev), to_dev_bf16(s, dev),
                          to_dev_bf16(b, dev), lhs_indices=to_dev_u32(lhs, dev),
                          rhs_indices=to_dev_u32(srt, dev), group_size=64, bits=4,
                          sorted_indices=True)
    truth = O.gather_qmm_f64(x, wq, s, b, lhs, srt, T * topk)
    assert max_err_ratio(to_f64(y), truth) <= BF16_TOL


def test_gather_out_of_range_is_nan(dev):
    _print_case(t="gather_oob")
    E, N, K = 4, 32, 128
    wq, s, b = weights(E, N, K, 4, 64, 90)
    x = O.make_x_bf16(3, K, 91).reshape(3, 1, K)
    rhs = np.array([0, 9, 2], np.uint32)
    lhs = np.array([0, 1, 7], np.uint32)
    y = mi_qmm.gather_qmm(to_dev_bf16(x, dev), to_dev_u32(wq, dev), to_dev_bf16(s, dev),
                          to_dev_bf16(b, dev), lhs_indices=to_dev_u32(lhs, dev),
                          rhs_indices=to_dev_u32(rhs, dev), group_size=64, bits=4)
    yf = to_f64(y)
    assert np.isnan(yf[1]).all() and np.isnan(yf[2]).all()
    truth = O.gather_qmm_f64(x, wq, s, b, lhs[:1], rhs[:1], 1)
    assert max_err_ratio(yf[:1], truth) <= BF16_TOL


def test_gather_sorted_multirow_nan_rows(dev):
    """Sorted runs of several rows: a run on an unknown expert and a row whose lhs index
    is out of range come out NaN; the other rows of the same runs are exact."""
    _print_case(t="gather_sorted_nan")
    E, N, K = 4, 64, 256
    wq, s, b = weights(E, N, K, 4, 64, 92)
    x = O.make_x_bf16(6, K, 93).reshape(6, 1, K)
    rhs = np.array([0, 0, 0, 1, 1, 9, 9], np.uint32)
    lhs = np.array([0, 1, 7, 2, 3, 4, 5], np.uint32)
    y = mi_qmm.gather_qmm(to_dev_bf16(x, dev), to_dev_u32(wq, dev), to_dev_bf16(s, dev),
                          to_dev_bf16(b, dev), lhs_indices=to_dev_u32(lhs, dev),
                          rhs_indices=to_dev_u32(rhs, dev), group_size=64, bits=4,
                          sorted_indices=True)
    yf = to_f64(y)
    for r in (2, 5, 6):
        assert np.isnan(yf[r]).all()
    ok = np.array([0, 1, 3, 4])
    truth = O.gather_qmm_f64(x, wq, s, b, lhs[ok], rhs[ok], len(ok))
    assert max_err_ratio(yf[ok], truth) <= BF16_TOL


def test_gather_sorted_long_runs(dev):
    """Sorted runs longer than one work item (32 rows), at a configs[3]-like width: a run of
    50 rows (one lhs out of range -> NaN row), a run of 70 (three items), a run on an unknown
    expert (NaN rows); every other row against the oracle."""
    _print_case(t="gather_sorted_long")
    E, N, K = 3, 768, 768
    wq, s, b = weights(E, N, K, 4, 64, 94)
    n0, n1, n9 = 50, 70, 10
    x = O.make_x_bf16(n0 + n1 + n9, K, 95).reshape(-1, 1, K)
    rhs = np.array([0] * n0 + [1] * n1 + [9] * n9, np.uint32)
    lhs = np.arange(n0 + n1 + n9, dtype=np.uint32)
    lhs[7] = 100000
    y = mi_qmm.gather_qmm(to_dev_bf16(x, dev), to_dev_u32(wq, dev), to_dev_bf16(s, dev),
                          to_dev_bf16(b, dev), lhs_indices=to_dev_u32(lhs, dev),
                          rhs_indices=to_dev_u32(rhs, dev), group_size=64, bits=4,
                          sorted_indices=True)
    yf = to_f64(y).reshape(len(rhs), N)
    bad = np.zeros(len(rhs), bool)
    bad[7] = True
    bad[n0 + n1:] = True
    assert np.isnan(yf[bad]).all()
    ok = np.nonzero(~bad)[0]
    truth = O.gather_qmm_f64(x, wq, s, b, lhs[ok], rhs[ok], len(ok)).reshape(len(ok), N)
    assert max_err_ratio(yf[ok], truth) <= BF16_TOL


def test_deterministic(dev):
    _print_case(t="determinism")
    wq, s, b = weights(1, 512, 4096, 4, 64, 99)
    x = to_dev_bf16(O.make_x_bf16(1, 4096, 98), dev)
    args = (to_dev_u32(wq[0], dev), to_dev_bf16(s[0], dev), to_dev_bf16(b[0], dev))
    y0 = bf16_bits(mi_qmm.quantized_matmul(x, *args))
    for _ in range(3):
        assert np.array_equal(bf16_bits(mi_qmm.quantized_matmul(x, *args)), y0)


def test_fill_randn_matches_oracle_stream(dev):
    _print_case(t="randn")
    t = torch.empty(4097, dtype=torch.float32, device=dev)
    mi_qmm.fill_randn(t, 1234, 0.0, 1.0)
    ref = O.randn(4097, 1234)
    got = t.cpu().numpy()
    assert np.max(np.abs(got - ref)) <= 1e-6


PREFILL_CASES = [(33, 64, 256), (128, 256, 512), (257, 300, 1024), (512, 520, 2048), (300, 200, 768),
                 (640, 256, 4096), (1024, 256, 512), (200, 512, 4096)]


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("M,N,K", PREFILL_CASES)
def test_prefill_qmm(dev, M, N, K, bits, gs):
    """Large-M paths: the fused MFMA GEMM (M < 256) and dequantize + hipBLASLt (M >= 256)."""
    _print_case(t="prefill", M=M, N=N, K=K, bits=bits, gs=gs)
    wq, s, b = weights(1, N, K, bits, gs, 5000 + M)
    x = O.make_x_bf16(M, K, 6000 + N)
    y = mi_qmm.quantized_matmul(to_dev_bf16(x, dev), to_dev_u32(wq[0], dev),
                                to_dev_bf16(s[0], dev), to_dev_bf16(b[0], dev), True, gs, bits)
    truth = O.qmm_f64(x, wq[0], s[0], b[0], gs, bits)
    assert max_err_ratio(to_f64(y), truth) <= BF16_TOL


@pytest.mark.parametrize("M,N,K,gs", [(256, 260, 960, 64), (300, 300, 1152, 128)])
@pytest.mark.parametrize("bits", [4, 8])
def test_prefill_odd_group_count(dev, M, N, K, gs, bits):
    """Odd group counts per row (K/gs = 15, 9): a row's scales then do not start on a
    dword, so the 4-bit prefill kernel hands these shapes to another route."""
    _print_case(t="prefill_odd_g", M=M, N=N, K=K, bits=bits, gs=gs)
    wq, s, b = weights(1, N, K, bits, gs, 5100 + M)
    x = O.make_x_bf16(M, K, 6100 + N)
    y = mi_qmm.quantized_matmul(to_dev_bf16(x, dev), to_dev_u32(wq[0], dev),
                                to_dev_bf16(s[0], dev), to_dev_bf16(b[0], dev), True, gs, bits)
    truth = O.qmm_f64(x, wq[0], s[0], b[0], gs, bits)
    assert max_err_ratio(to_f64(y), truth) <= BF16_TOL


@pytest.mark.parametrize("N,K", [(14336, 4096), (4096, 14336)])
def test_prefill_full_size_sampled_rows(dev, N, K):
    """configs[2] shapes at M=2048: 48 sampled output rows against the oracle, and the
    whole output against a torch fp32 GEMM on the exactly dequantized weight."""
    _print_case(t="prefill_full", N=N, K=K)
    M = 2048
    wq, s, b = weights(1, N, K, 4, 64, 7000 + N)
    x = O.make_x_bf16(M, K, 7100 + N)
    W, S, B = to_dev_u32(wq[0], dev), to_dev_bf16(s[0], dev), to_dev_bf16(b[0], dev)
    xd = to_dev_bf16(x, dev)
    y = mi_qmm.quantized_matmul(xd, W, S, B, True, 64, 4)
    rows = np.random.default_rng(N).choice(M, 48, replace=False)
    truth = O.qmm_f64(x[rows], wq[0], s[0], b[0], 64, 4)
    assert max_err_ratio(to_f64(y)[rows], truth) <= BF16_TOL
    wf = mi_qmm.dequantize(W, S, B, 64, 4, dtype=torch.float32)
    ref = xd.float() @ wf.t()
    err = (y.float() - ref).abs().max().item() / ref.abs().max().item()
    assert err <= BF16_TOL


def _fp_weight(mode, N, K, seed):
    m, bits, gs = O.FP_MODES[mode]
    rng = np.random.default_rng(seed)
    q = rng.integers(0, 1 << bits, size=(N, K)).astype(np.uint8)
    if mode == "mxfp8":  # a few 0x7F / 0xFF codes: +-480 in the reference's decoder
        q[(q & 0x7F) == 0x7F] = 0x3F
        q[0, 3], q[1, 40], q[N - 1, K - 1] = 0x7F, 0xFF, 0x7F
    # e8m0 scales near 1; nvfp4's e4m3 scales positive, 2^-3 .. 2^1
    lo, hi = (0x20, 0x48) if mode == "nvfp4" else (118, 126)
    sc = rng.integers(lo, hi, size=(N, K // gs)).astype(np.uint8)
    return O.pack(q, bits), sc


@pytest.mark.parametrize("mode", ["nvfp4", "mxfp4", "mxfp8"])
def test_dequantize_fp_modes_bit_exact(dev, mode):
    _print_case(t="dequant_fp", mode=mode)
    wq, sc = _fp_weight(mode, 96, 512, 7)
    W, S = to_dev_u32(wq, dev), torch.from_numpy(sc).to(dev)
    f32 = mi_qmm.dequantize(W, S, None, mode=mode, dtype=torch.float32).cpu().numpy()
    assert np.array_equal(f32.view(np.uint32), O.dequantize_fp(wq, sc, mode).view(np.uint32))
    bf = bf16_bits(mi_qmm.dequantize(W, S, None, mode=mode))
    assert np.array_equal(bf, O.dequantize_fp(wq, sc, mode, out_bf16=True))


@pytest.mark.parametrize("fmt", ["b2", "b3", "b5", "b6", "nvfp4", "mxfp4", "mxfp8"])
@pytest.mark.parametrize("M", [64, 512])
def test_large_m_other_formats_own_gemm(dev, fmt, M):
    """Above the few-row kernels, 2/3/5/6-bit and nvfp4 / mxfp4 / mxfp8 weights dequantize
    to bf16 and run the prefill kernel's bf16-weight instance: results against the oracle,
    and the vendor GEMM never runs (its call counter does not move)."""
    _print_case(t="large_m_format", fmt=fmt, M=M)
    N, K = 300, 1024
    before = mi_qmm.library_gemm_calls()
    x = O.make_x_bf16(M, K, 900 + M)
    if fmt.startswith("b"):
        bits = int(fmt[1:])
        wq, s, b = weights(1, N, K, bits, 64, 910 + bits)
        y = mi_qmm.quantized_matmul(to_dev_bf16(x, dev), to_dev_u32(wq[0], dev),
                                    to_dev_bf16(s[0], dev), to_dev_bf16(b[0], dev), True, 64, bits)
        truth = O.qmm_f64(x, wq[0], s[0], b[0], 64, bits)
    else:
        wq, sc = _fp_weight(fmt, N, K, 920 + M)
        y = mi_qmm.quantized_matmul(to_dev_bf16(x, dev), to_dev_u32(wq, dev),
                                    torch.from_numpy(sc).to(dev), None, True, mode=fmt)
        truth = O.bf16_to_f32(x).astype(np.float64) @ O.dequantize_fp(wq, sc, fmt).astype(np.float64).T
    torch.cuda.synchronize()
    assert max_err_ratio(to_f64(y), truth) <= BF16_TOL
    assert mi_qmm.library_gemm_calls() == before


@pytest.mark.parametrize("mode", ["nvfp4", "mxfp4", "mxfp8"])
@pytest.mark.parametrize("M,N,K", [(1, 256, 1024), (5, 96, 512), (300, 64, 384)])
def test_qmm_fp_modes(dev, mode, M, N, K):
    """Bias-less modes: dequantize (exact in bf16) + bf16 GEMM; truth is fp64 over the
    oracle's exactly dequantized weight."""
    _print_case(t="qmm_fp", mode=mode, M=M, N=N, K=K)
    wq, sc = _fp_weight(mode, N, K, 11 + M)
    x = O.make_x_bf16(M, K, 12 + N)
    y = mi_qmm.quantized_matmul(to_dev_bf16(x, dev), to_dev_u32(wq, dev),
                                torch.from_numpy(sc).to(dev), None, True, mode=mode)
    wd = O.dequantize_fp(wq, sc, mode).astype(np.float64)
    truth = O.bf16_to_f32(x).astype(np.float64) @ wd.T
    assert y.shape == (M, N) and y.dtype == torch.bfloat16
    assert max_err_ratio(to_f64(y), truth) <= BF16_TOL


@pytest.mark.parametrize("mode", ["nvfp4", "mxfp4", "mxfp8"])
@pytest.mark.parametrize("M,N,K", [(2, 100, 2048), (7, 64, 512), (16, 256, 4096), (17, 48, 7168),
                                   (32, 512, 14336), (24, 80, 384)])
def test_qmm_fp4_mfma(dev, mode, M, N, K):
    """Bias-less modes at 2..32 rows (the few-row MFMA kernel: code x scale converted to bf16,
    exact, per 8-code run; mxfp8's 0x7F / 0xFF codes take the exact per-code route; K = 14336
    at 32 rows takes the K split)."""
    _print_case(t="qmm_fp4_mfma", mode=mode, M=M, N=N, K=K)
    wq, sc = _fp_weight(mode, N, K, 50 + M)
    x = O.make_x_bf16(M, K, 51 + N)
    y = mi_qmm.quantized_matmul(to_dev_bf16(x, dev), to_dev_u32(wq, dev),
                                torch.from_numpy(sc).to(dev), None, True, mode=mode)
    truth = O.bf16_to_f32(x).astype(np.float64) @ O.dequantize_fp(wq, sc, mode).astype(np.float64).T
    assert max_err_ratio(to_f64(y), truth) <= BF16_TOL


@pytest.mark.parametrize("mode", ["nvfp4", "mxfp4", "mxfp8"])
@pytest.mark.parametrize("M,N,K", [(1, 320, 14336), (1, 64, 2176), (1, 4096, 1024),
                                   (1, 100, 4096)])
def test_qmm_fp4_one_row(dev, mode, M, N, K):
    """One row of nvfp4 / mxfp4 / mxfp8 on the one-row streaming kernel's fp instances
    (K = 2176: 17 chunks, a K-split plan and the fixed-order reduce; mxfp8's 0x7F / 0xFF
    codes patched to +-480 x scale)."""
    _print_case(t="qmm_fp4_one_row", mode=mode, N=N, K=K)
    wq, sc = _fp_weight(mode, N, K, 90 + N)
    x = O.make_x_bf16(M, K, 91 + K)
    y = mi_qmm.quantized_matmul(to_dev_bf16(x, dev), to_dev_u32(wq, dev),
                                torch.from_numpy(sc).to(dev), None, True, mode=mode)
    truth = O.bf16_to_f32(x).astype(np.float64) @ O.dequantize_fp(wq, sc, mode).astype(np.float64).T
    assert y.shape == (M, N)
    assert max_err_ratio(to_f64(y), truth) <= BF16_TOL


@pytest.mark.parametrize("mode", ["nvfp4", "mxfp4", "mxfp8"])
@pytest.mark.parametrize("M", [1, 8])
def test_qmm_fp4_mfma_scale_edges(dev, mode, M):
    """Scale bytes at the ends of their formats: e4m3 0x7F (480 in the reference's
    reading) and 0x01 (2^-9), e8m0 0 (2^-127), 1 and 140 groups mixed with ordinary ones;
    for mxfp8 also dense runs of the codes 0x7F / 0xFF (+-480, which the hardware
    conversion reads as NaN) in those groups (one row: the one-row kernel or, for mxfp8,
    the few-row MFMA kernel; eight: the few-row MFMA kernel)."""
    _print_case(t="qmm_fp4_edges", mode=mode, M=M)
    N, K = 64, 512
    wq, sc = _fp_weight(mode, N, K, 77)
    if mode == "nvfp4":
        sc[0, :] = 0x7F
        sc[1, 2] = 0x01
        sc[2, 5] = 0x80 | 0x30  # a negative scale
    else:
        sc[0, 1] = 1
        sc[1, :] = 140  # 2^13
    if mode == "mxfp8":
        sc[2, :] = 0  # 2^-127
        b = wq.view(np.uint8).reshape(N, K)
        b[2, ::5] = 0x7F
        b[2, 1::7] = 0xFF
        b[1, 3::11] = 0xFF
        b[4, ::2] = 0x7F
        b[4, 1::2] = 0xFF
        b[5, 64:96] = 0x7E  # the largest finite code of the hardware's reading
    x = O.make_x_bf16(M, K, 78)
    y = mi_qmm.quantized_matmul(to_dev_bf16(x, dev), to_dev_u32(wq, dev),
                                torch.from_numpy(sc).to(dev), None, True, mode=mode)
    truth = O.bf16_to_f32(x).astype(np.float64) @ O.dequantize_fp(wq, sc, mode).astype(np.float64).T
    yf = to_f64(y)
    for n in range(N):  # per output column: the scales differ by orders of magnitude
        assert max_err_ratio(yf[:, n:n + 1], truth[:, n:n + 1]) <= BF16_TOL, n


@pytest.mark.parametrize("mode", ["nvfp4", "mxfp4", "mxfp8"])
def test_gather_fp4_sorted(dev, mode):
    """Sorted fp4 gather of a skewed MoE routing (T = 64, k = 8, 16 experts): runs of
    several rows per expert become work items of the MFMA kernel."""
    _print_case(t="gather_fp4_sorted", mode=mode)
    E, N, K, T, k = 16, 96, 1024, 64, 8
    banks = [_fp_weight(mode, N, K, 60 + e) for e in range(E)]
    wq = np.stack([bk[0] for bk in banks])
    sc = np.stack([bk[1] for bk in banks])
    rng = np.random.default_rng(61)
    inds = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.uint32)
    flat = inds.reshape(-1)
    order = np.argsort(flat, kind="stable").astype(np.uint32)
    srt = flat[order]
    lhs = (order // k).astype(np.uint32)
    x = O.make_x_bf16(T, K, 62)
    y = mi_qmm.gather_qmm(to_dev_bf16(x, dev).reshape(T, 1, K), to_dev_u32(wq, dev),
                          torch.from_numpy(sc).to(dev), None, lhs_indices=to_dev_u32(lhs, dev),
                          rhs_indices=to_dev_u32(srt, dev), mode=mode, sorted_indices=True)
    xf = O.bf16_to_f32(x).astype(np.float64)
    wd = [O.dequantize_fp(wq[e], sc[e], mode).astype(np.float64) for e in range(E)]
    truth = np.stack([xf[lhs[i]] @ wd[srt[i]].T for i in range(T * k)])
    assert max_err_ratio(to_f64(y).reshape(T * k, N), truth) <= BF16_TOL


@pytest.mark.parametrize("bits", [2, 3, 5, 6])
@pytest.mark.parametrize("M,N,K", [(1, 200, 4096), (5, 64, 512), (16, 96, 2048), (32, 256, 14336),
                                   (24, 40, 384)])
def test_qmm_odd_mfma(dev, bits, M, N, K):
    """Affine 2/3/5/6 bits, gs 64, 1..32 rows on the few-row MFMA kernel (8 codes per lane
    from one 8-byte load of the row's bitstream; K = 14336 at 32 rows takes the K split)."""
    _print_case(t="qmm_odd_mfma", M=M, N=N, K=K, bits=bits)
    wq, s, b = weights(1, N, K, bits, 64, 90 + bits + M)
    x = O.make_x_bf16(M, K, 91 + N)
    y = mi_qmm.quantized_matmul(to_dev_bf16(x, dev), to_dev_u32(wq[0], dev),
                                to_dev_bf16(s[0], dev), to_dev_bf16(b[0], dev), True, 64, bits)
    truth = O.qmm_f64(x, wq[0], s[0], b[0], 64, bits)
    assert max_err_ratio(to_f64(y), truth) <= BF16_TOL


@pytest.mark.parametrize("bits", [2, 3, 5, 6])
def test_gather_odd_sorted(dev, bits):
    """Sorted odd-width gather (T = 64, k = 8, 16 experts): multi-row work items of the MFMA
    kernel, against the oracle."""
    _print_case(t="gather_odd_sorted", bits=bits)
    E, N, K, T, k = 16, 96, 1024, 64, 8
    wq, s, b = weights(E, N, K, bits, 64, 95 + bits)
    rng = np.random.default_rng(96)
    inds = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.uint32)
    flat = inds.reshape(-1)
    order = np.argsort(flat, kind="stable").astype(np.uint32)
    srt = flat[order]
    lhs = (order // k).astype(np.uint32)
    x = O.make_x_bf16(T, K, 97)
    y = mi_qmm.gather_qmm(to_dev_bf16(x, dev).reshape(T, 1, K), to_dev_u32(wq, dev),
                          to_dev_bf16(s, dev), to_dev_bf16(b, dev), lhs_indices=to_dev_u32(lhs, dev),
                          rhs_indices=to_dev_u32(srt, dev), group_size=64, bits=bits,
                          sorted_indices=True)
    truth = O.gather_qmm_f64(x.reshape(T, 1, K), wq, s, b, lhs, srt, T * k, group_size=64,
                             bits=bits)
    assert max_err_ratio(to_f64(y).reshape(T * k, 1, N), truth) <= BF16_TOL


@pytest.mark.parametrize("mode", ["nvfp4", "mxfp4", "mxfp8"])
@pytest.mark.parametrize("sorted_", [False, True])
def test_gather_fp_out_of_range_is_nan(dev, mode, sorted_):
    """An expert id past the bank gives a NaN row on the fp-mode MFMA path too (sorted work
    items and unsorted pairs); every other row matches the oracle."""
    _print_case(t="gather_fp_oob", mode=mode, sorted=sorted_)
    E, N, K, T, k = 6, 64, 512, 8, 2
    banks = [_fp_weight(mode, N, K, 110 + e) for e in range(E)]
    wq = np.stack([bk[0] for bk in banks])
    sc = np.stack([bk[1] for bk in banks])
    rng = np.random.default_rng(111)
    flat = rng.integers(0, E, size=T * k).astype(np.uint32)
    flat[5] = E + 3
    if sorted_:
        order = np.argsort(flat, kind="stable").astype(np.uint32)
        rhs, lhs = flat[order], (order // k).astype(np.uint32)
    else:
        rhs, lhs = flat, (np.arange(T * k) // k).astype(np.uint32)
    x = O.make_x_bf16(T, K, 112)
    y = mi_qmm.gather_qmm(to_dev_bf16(x, dev).reshape(T, 1, K), to_dev_u32(wq, dev),
                          torch.from_numpy(sc).to(dev), None, lhs_indices=to_dev_u32(lhs, dev),
                          rhs_indices=to_dev_u32(rhs, dev), mode=mode, sorted_indices=sorted_)
    yf = to_f64(y).reshape(T * k, N)
    xf = O.bf16_to_f32(x).astype(np.float64)
    for i in range(T * k):
        if rhs[i] >= E:
            assert np.isnan(yf[i]).all(), i
        else:
            truth = xf[lhs[i]] @ O.dequantize_fp(wq[rhs[i]], sc[rhs[i]], mode).astype(np.float64).T
            assert max_err_ratio(yf[i:i + 1], truth[None]) <= BF16_TOL, i


def test_graph_replay_after_workspace_growth(dev):
    """A sorted gather captured in a HIP graph keeps its workspace address; a later,
    larger uncaptured call grows the workspace, and every replay of the old graph must
    still match the eager result (the outgrown buffer stays allocated until
    mi_workspace_release)."""
    _print_case(t="ws_growth")
    E, N, K, T, topk = 8, 64, 8192, 64, 4
    wq, s, b = weights(E, N, K, 4, 64, 401)
    flat = np.random.default_rng(402).integers(0, E, size=T * topk).astype(np.uint32)
    _, _, srt, lhs = O.sort_dispatch(flat, topk)
    x = to_dev_bf16(O.make_x_bf16(T, K, 403).reshape(T, 1, K), dev)
    args = (to_dev_u32(wq, dev), to_dev_bf16(s, dev), to_dev_bf16(b, dev))
    kw = dict(lhs_indices=to_dev_u32(lhs, dev), rhs_indices=to_dev_u32(srt, dev), group_size=64,
              bits=4, sorted_indices=True)
    eager = bf16_bits(mi_qmm.gather_qmm(x, *args, **kw))
    out = torch.empty(T * topk, 1, N, dtype=torch.bfloat16, device=dev)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        mi_qmm.gather_qmm(x, *args, out=out, **kw)
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        mi_qmm.gather_qmm(x, *args, out=out, **kw)
    # grow the workspace past anything earlier tests needed
    mi_qmm.workspace_reserve(1 << 30)
    for _ in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(bf16_bits(out), eager)
    del g
    torch.cuda.synchronize()
    mi_qmm._lib.check(mi_qmm._lib.lib().mi_workspace_release(None))
    assert np.array_equal(bf16_bits(mi_qmm.gather_qmm(x, *args, **kw)), eager)


@pytest.mark.parametrize("g", [0.25, 1.0 / 3.0, 7.5])
def test_dequantize_nvfp4_global_scale(dev, g):
    """mlx_dequantize's global_scale (nvfp4): bit-exact against the oracle in fp32 and bf16;
    other modes and mi_quantize refuse a global scale."""
    _print_case(t="nvfp4_gscale", g=g)
    wq, sc = _fp_weight("nvfp4", 64, 256, 41)
    W, S = to_dev_u32(wq, dev), torch.from_numpy(sc).to(dev)
    gs_t = torch.tensor([g], dtype=torch.float32, device=dev)
    f32 = mi_qmm.dequantize(W, S, None, mode="nvfp4", dtype=torch.float32, global_scale=gs_t)
    ref = O.dequantize_fp(wq, sc, "nvfp4", global_scale=float(np.float32(g)))
    assert np.array_equal(f32.cpu().numpy().view(np.uint32), ref.view(np.uint32))
    bf = bf16_bits(mi_qmm.dequantize(W, S, None, mode="nvfp4", global_scale=gs_t))
    assert np.array_equal(bf, O.dequantize_fp(wq, sc, "nvfp4", out_bf16=True,
                                              global_scale=float(np.float32(g))))
    wq2, sc2 = _fp_weight("mxfp4", 64, 256, 42)
    with pytest.raises(mi_qmm.MiError):
        mi_qmm.dequantize(to_dev_u32(wq2, dev), torch.from_numpy(sc2).to(dev), None,
                          mode="mxfp4", global_scale=gs_t)
    w = torch.zeros(4, 64, dtype=torch.bfloat16, device=dev)
    out = [torch.empty(4, 8, dtype=torch.int32, device=dev),
           torch.empty(4, 1, dtype=torch.bfloat16, device=dev),
           torch.empty(4, 1, dtype=torch.bfloat16, device=dev)]
    from mi_qmm._lib import opt
    rc = mi_qmm._lib.lib().mi_quantize(out[0].data_ptr(), out[1].data_ptr(), out[2].data_ptr(),
                                      w.data_ptr(), 4, 64, opt(64), opt(4), b"affine",
                                      gs_t.data_ptr(), 12, None)
    assert rc == 1  # MI_ERR_UNSUPPORTED
