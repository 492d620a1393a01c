"""Pins the CPU oracle (oracle/mi_oracle.c) before it is trusted as the checker.

Each check comes from somewhere other than the oracle's own formula: published
constants (SplitMix64), torch's bf16 arithmetic, numpy float64 matmuls, hand-worked
groups, closed forms, brute force on tiny inputs, and the reference's own test
expectations (tests/golden/geometry_cases.json, from src/transformer.zig:22930).
"""
import json
import os

import numpy as np
import pytest
import torch

import oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


# ------------------------------------------------------------------ bf16 --
def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(0)
    f = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 20000),
        np.array([0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, 3.0e38, 1e-40, -1e-42], np.float32),
        # exact ties at bf16 precision: round to even
        (np.arange(1, 2000, dtype=np.uint32) << 16 | 0x8000).view(np.float32),
    ]).astype(np.float32)
    ours = O.f32_to_bf16(f)
    theirs = torch.from_numpy(f).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, theirs)
    assert np.array_equal(O.bf16_to_f32(ours), torch.from_numpy(ours.view(np.int16))
                          .view(torch.bfloat16).float().numpy())


def test_bf16_nan_stays_nan():
    f = np.array([np.nan, -np.nan], np.float32)
    assert np.isnan(O.bf16_to_f32(O.f32_to_bf16(f))).all()


# ------------------------------------------------------------- generator --
def test_splitmix64_known_answers():
    # SplitMix64 (Steele, Lea, Flood 2014) seeded with 0: its published first outputs.
    L = O.lib()
    assert L.mo_splitmix64(0, 0) == 0xE220A8397B1DCDAF
    assert L.mo_splitmix64(0, 1) == 0x6E789E6AA1B965F4
    assert L.mo_splitmix64(0, 2) == 0x06C45D188009454F


def test_randn_moments_and_determinism():
    a = O.randn(1 << 20, O.seed_for(1, 1))
    assert abs(a.mean()) < 5e-3 and abs(a.std() - 1.0) < 5e-3
    assert np.array_equal(a[:1000], O.randn(1000, O.seed_for(1, 1)))
    b = O.randn(1 << 16, 7, 0.0, 0.02)
    assert abs(b.std() - 0.02) < 5e-4
    u = O.uniform(1 << 16, 3)
    assert u.min() >= 0.0 and u.max() < 1.0 and abs(u.mean() - 0.5) < 5e-3


# --------------------------------------------------------------- packing --
def test_pack_known_words():
    # LSB-first: value j of a word sits at bits [j*bits, (j+1)*bits)
    # (src/transformer.zig:20098-20108 nibbles, :522-525 bytes).
    q4 = np.array([[0, 1, 2, 3, 4, 5, 6, 7, 15, 14, 13, 12, 11, 10, 9, 8]], np.uint8)
    assert O.pack(q4, 4).tolist() == [[0x76543210, 0x89ABCDEF]]
    q8 = np.array([[1, 2, 3, 4, 255, 0, 128, 7]], np.uint8)
    assert O.pack(q8, 8).tolist() == [[0x04030201, 0x078000FF]]


ALL_BITS = [2, 3, 4, 5, 6, 8]


def _bitstream_unpack(wq, K, bits):
    # a row is one LSB-first bitstream over its little-endian bytes: code j = bits
    # [j*bits, (j+1)*bits)
    rows = wq.reshape(-1, wq.shape[-1])
    bitv = np.unpackbits(rows.view(np.uint8), axis=1, bitorder="little")
    bitv = bitv[:, : K * bits].reshape(rows.shape[0], K, bits).astype(np.uint32)
    return (bitv << np.arange(bits, dtype=np.uint32)).sum(axis=2).astype(np.uint8)


@pytest.mark.parametrize("bits", ALL_BITS)
def test_pack_round_trip(bits):
    rng = np.random.default_rng(bits)
    q = rng.integers(0, 1 << bits, size=(7, 256)).astype(np.uint8)
    wq = O.pack(q, bits)
    assert wq.shape == (7, 256 * bits // 32)
    assert np.array_equal(O.unpack(wq, 256, bits), q)
    assert np.array_equal(_bitstream_unpack(wq, 256, bits), q)  # independent unpack
    if 32 % bits == 0:  # whole codes per word: value j of a word at bits j*bits
        shifts = np.arange(32 // bits, dtype=np.uint32) * bits
        nq = ((wq[..., None] >> shifts) & ((1 << bits) - 1)).reshape(7, 256)
        assert np.array_equal(nq, q)


def test_pack_5_and_6_bit_follow_the_reference_byte_reads():
    # src/transformer.zig:516-578: a pack of 8 codes is `bits` bytes at pack*bits. 5-bit:
    # a 40-bit little-endian r from 5 bytes, code ki = (r >> 5ki) & 31. 6-bit: three
    # little-endian u16 h0..h2, a0 = h0 | (h1 & 0xFF) << 16, a1 = h1 >> 8 | h2 << 8, codes
    # (a0 >> 6ki) & 63 then (a1 >> 6ki) & 63.
    rng = np.random.default_rng(56)
    q5 = rng.integers(0, 32, size=(3, 64)).astype(np.uint8)
    b5 = O.pack(q5, 5).view(np.uint8).reshape(3, -1)
    for r in range(3):
        for p in range(8):
            by = b5[r, 5 * p:5 * p + 5].astype(np.uint64)
            rr = int(sum(int(by[i]) << (8 * i) for i in range(5)))
            assert [(rr >> (5 * ki)) & 31 for ki in range(8)] == q5[r, 8 * p:8 * p + 8].tolist()
    q6 = rng.integers(0, 64, size=(3, 64)).astype(np.uint8)
    b6 = O.pack(q6, 6).view(np.uint8).reshape(3, -1)
    for r in range(3):
        for p in range(8):
            h = [int(b6[r, 6 * p + 2 * i]) | int(b6[r, 6 * p + 2 * i + 1]) << 8 for i in range(3)]
            a0 = h[0] | (h[1] & 0xFF) << 16
            a1 = (h[1] >> 8) | (h[2] << 8)
            got = [(a0 >> (6 * ki)) & 63 for ki in range(4)] + [(a1 >> (6 * ki)) & 63 for ki in range(4)]
            assert got == q6[r, 8 * p:8 * p + 8].tolist()
    # 3-bit: 8 codes in 3 bytes, hand-packed: codes 1..7, 0 -> 0b000_111_110_101_100_011_010_001
    q3 = np.array([[1, 2, 3, 4, 5, 6, 7, 0] * 4], np.uint8)
    w3 = O.pack(q3, 3).view(np.uint8).reshape(-1)
    assert w3[:3].tolist() == list((0b000111110101100011010001).to_bytes(3, "little"))


# -------------------------------------------------------------- quantize --
def test_quantize_hand_worked_group():
    # group min -1, max 0.5: |min| > |max| so scale = 1.5/15 = 0.1 > 0, edge = min = -1,
    # q0 = rint(-1/0.1) = -10, scale = -1/-10 = 0.1, bias = -1; 0.5 -> q 15, 0 -> q 10.
    g = np.zeros(64, np.float32)
    g[0], g[1] = -1.0, 0.5
    w = O.f32_to_bf16(g[None, :])
    wq, s, b = O.quantize(w, 64, 4)
    q = O.unpack(wq, 64, 4)[0]
    assert q[0] == 0 and q[1] == 15 and (q[2:] == 10).all()
    assert s[0, 0] == O.f32_to_bf16(np.float32(0.1)) and b[0, 0] == 0xBF80


def _bits_le(wq_row, K, bits):
    """Independent bitstream unpack: code j = bits [j*bits, (j+1)*bits) of the row's
    little-endian byte string (numpy bit operations, no oracle code)."""
    by = np.ascontiguousarray(wq_row, dtype=np.uint32).view(np.uint8)
    bitv = np.unpackbits(by, bitorder="little")
    return np.array([int("".join(str(b) for b in bitv[j * bits:(j + 1) * bits][::-1]), 2)
                     for j in range(K)])


def test_quantize_code_ties_round_to_even():
    """(w - bias)/scale landing exactly on k + 0.5 rounds to the even code (rint), not
    away from zero. Group {15/16, 6.5/16, 0}: span 15/16, scale -1/16 (|min| <= |max|),
    edge = max, q0 = -15, scale stays -1/16, bias 15/16; code(w) = 15 - 16 w, so
    w = 6.5/16 gives 8.5 -> 8 (half-away-from-zero would give 9), and 0 gives 15."""
    g = np.zeros(64, np.float32)
    g[0], g[1] = 15 / 16, 6.5 / 16
    wq, s, b = O.quantize(O.f32_to_bf16(g[None, :]), 64, 4)
    q = _bits_le(wq[0], 64, 4)
    assert q[0] == 0 and q[1] == 8 and (q[2:] == 15).all()
    assert O.bf16_to_f32(s)[0, 0] == -1 / 16 and O.bf16_to_f32(b)[0, 0] == 15 / 16


def test_quantize_edge_tie_rounds_to_even_then_refits():
    """edge/scale exactly -12.5 (max 12.5/8, min -2.5/8, span 15/8 so scale -1/8): q0 =
    rint(-12.5) = -12 (not -13), the scale is refit to edge/q0 = -0.13020833 and the
    bias is the edge, 1.5625. The max then decodes exactly and the min to code
    rint((-0.3125 - 1.5625)/s) = rint(14.4) = 14."""
    g = np.zeros(32, np.float32)
    g[0], g[1] = 12.5 / 8, -2.5 / 8
    wq, s, b = O.quantize(O.f32_to_bf16(g[None, :]), 32, 4)
    scale = np.float32(np.float32(1.5625) / np.float32(-12.0))
    assert s[0, 0] == O.f32_to_bf16(np.array([scale], np.float32))[0]
    assert O.bf16_to_f32(b)[0, 0] == 1.5625
    q = _bits_le(wq[0], 32, 4)
    assert q[0] == 0 and q[1] == 14
    assert (q[2:] == 12).all()  # 0.0 -> rint(-1.5625 / -0.1302) = rint(12.0) = 12


def test_quantize_negative_edge_group():
    """|min| > |max|: the scale is positive and the bias is the (negative) minimum.
    Values in [-15/8, 0]: scale 1/8, q0 = -15, bias -1.875, code = 15 + 8 w."""
    g = np.array([-1.875, 0.0, -1.0, -0.5, -1.125] + [-0.25] * 27, np.float32)
    wq, s, b = O.quantize(O.f32_to_bf16(g[None, :]), 32, 4)
    assert O.bf16_to_f32(s)[0, 0] == 0.125 and O.bf16_to_f32(b)[0, 0] == -1.875
    q = _bits_le(wq[0], 32, 4)
    assert list(q[:5]) == [0, 15, 7, 11, 6] and (q[5:] == 13).all()


def test_quantize_zero_q0_branch_keeps_eps_scale():
    """A group far below the 1e-7 scale floor: (max-min)/15 < eps so the scale is -1e-7
    (|min| <= |max|), q0 = rint(max/-1e-7) = 0, so the refit is skipped: bias 0, scale
    stays -1e-7 and every code clamps to 0."""
    g = np.full(64, 2.0 ** -26, np.float32)
    g[3] = 2.0 ** -25
    wq, s, b = O.quantize(O.f32_to_bf16(g[None, :]), 64, 4)
    assert b[0, 0] == 0
    assert s[0, 0] == O.f32_to_bf16(np.array([-1e-7], np.float32))[0]
    assert (_bits_le(wq[0], 64, 4) == 0).all()


@pytest.mark.parametrize("bits", [2, 3, 5, 6])
def test_quantize_codes_straddle_words(bits):
    """Grid-exact groups at the odd widths: codes c_j = j mod 2^bits on value
    bias + scale*c (scale 1/4, positive-edge groups); the codes crossing 32-bit word
    boundaries come back exact from an independent bitstream read."""
    gs = 32
    nb = (1 << bits) - 1
    c = np.arange(2 * gs) % (nb + 1)
    c[0], c[gs] = 0, 0
    c[1], c[gs + 1] = nb, nb
    vals = (nb - c).astype(np.float32) * 0.25  # max nb/4 = edge (code 0), min 0 (code nb)
    wq, s, b = O.quantize(O.f32_to_bf16(vals[None, :]), gs, bits)
    assert (O.bf16_to_f32(s) == -0.25).all() and (O.bf16_to_f32(b) == nb * 0.25).all()
    assert np.array_equal(_bits_le(wq[0], 2 * gs, bits), c)


@pytest.mark.parametrize("bits", ALL_BITS)
@pytest.mark.parametrize("gs", [32, 64, 128])
def test_quantize_invariants(bits, gs):
    w = O.f32_to_bf16(O.randn(32 * 512, 9, 0.0, 0.02).reshape(32, 512))
    w[0, :gs] = O.f32_to_bf16(np.full(gs, 0.375, np.float32))  # constant group
    w[1, :gs] = 0                                                # zero group
    # on a 0.25 grid spanning codes 0 .. 2^bits-1 (every value fits bf16 exactly)
    codes = np.random.default_rng(bits).integers(0, 1 << bits, gs)
    codes[0], codes[1] = 0, (1 << bits) - 1
    w[2, :gs] = O.f32_to_bf16(codes.astype(np.float32) * 0.25 - 1.0)
    wq, s, b = O.quantize(w, gs, bits)
    deq = O.dequantize(wq, s, b, gs, bits, O.DQ_F32)
    wf = O.bf16_to_f32(w)
    sf = np.repeat(O.bf16_to_f32(s), gs, axis=1)
    bf = np.repeat(O.bf16_to_f32(b), gs, axis=1)
    # At most one step: the edge refit scale = edge/rint(edge/scale) can stretch the
    # far end of the group past the top code, where it clamps (worst case q0 = 2^(bits-1)).
    # Plus the bf16 rounding of the scale (times q <= 2^bits-1) and of the bias.
    bound = np.abs(sf) * (1.0 + (1 << bits) * 2.0 ** -8) + np.abs(bf) * 2.0 ** -8 + 1e-12
    assert (np.abs(deq - wf) <= bound).all()
    assert np.array_equal(deq[0, :gs], wf[0, :gs])
    assert np.array_equal(deq[1, :gs], wf[1, :gs])
    assert np.array_equal(deq[2, :gs], wf[2, :gs])
    # the edge element of every group (the larger-magnitude end, max on a tie) is
    # reproduced exactly: it becomes the bias and code 0
    G = 512 // gs
    for r in range(32):
        for g in range(G):
            seg = wf[r, g * gs:(g + 1) * gs]
            e = int(np.argmin(seg)) if abs(seg.min()) > abs(seg.max()) else int(np.argmax(seg))
            assert deq[r, g * gs + e] == seg[e]


# ------------------------------------------------------------ dequantize --
@pytest.mark.parametrize("bits", ALL_BITS)
def test_dequantize_closed_forms(bits):
    rng = np.random.default_rng(1)
    N, K, gs = 16, 256, 64
    q = rng.integers(0, 1 << bits, size=(N, K)).astype(np.uint8)
    s = O.f32_to_bf16(rng.standard_normal((N, K // gs)).astype(np.float32) * 0.01)
    b = O.f32_to_bf16(rng.standard_normal((N, K // gs)).astype(np.float32) * 0.1)
    wq = O.pack(q, bits)
    sf = np.repeat(O.bf16_to_f32(s), gs, axis=1).astype(np.float64)
    bf = np.repeat(O.bf16_to_f32(b), gs, axis=1).astype(np.float64)
    exact = sf * q + bf   # exact in float64: 8-bit significands times <= 8-bit integers
    f32 = O.dequantize(wq, s, b, gs, bits, O.DQ_F32)
    assert np.array_equal(f32, exact.astype(np.float32))
    fused = O.dequantize(wq, s, b, gs, bits, O.DQ_BF16_FUSED)
    assert np.array_equal(fused, O.f32_to_bf16(exact.astype(np.float32)))
    # op-by-op bf16: torch's bf16 multiply, then bf16 add
    tq = torch.from_numpy(q.astype(np.float32)).to(torch.bfloat16)
    ts = torch.from_numpy(np.repeat(s, gs, axis=1).view(np.int16)).view(torch.bfloat16)
    tb = torch.from_numpy(np.repeat(b, gs, axis=1).view(np.int16)).view(torch.bfloat16)
    opw = (ts * tq + tb).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.dequantize(wq, s, b, gs, bits, O.DQ_BF16_OPWISE), opw)


# ------------------------------------------------------------------- qmm --
def _dense(wq, s, b, gs, bits):
    return O.dequantize(wq, s, b, gs, bits, O.DQ_F32).astype(np.float64)


@pytest.mark.parametrize("bits", ALL_BITS)
def test_qmm_f64_matches_numpy(bits):
    wq, s, b = O.make_weight(48, 512, 5, bits)
    x = O.make_x_bf16(3, 512, 6)
    truth = O.bf16_to_f32(x).astype(np.float64) @ _dense(wq, s, b, 64, bits).T
    assert np.allclose(O.qmm_f64(x, wq, s, b, 64, bits), truth, rtol=1e-12, atol=1e-12)
    xf = O.randn(2 * 512, 8).reshape(2, 512)
    assert np.allclose(O.qmm_f64(xf, wq, s, b, 64, bits),
                       xf.astype(np.float64) @ _dense(wq, s, b, 64, bits).T, rtol=1e-12,
                       atol=1e-12)
    y32 = O.qmm_f32(x, wq, s, b, 64, bits, 2)
    assert np.max(np.abs(y32 - truth)) <= 1e-5 * np.max(np.abs(truth))


def test_qmm_special_cases():
    N, K = 32, 128
    q = (np.arange(N * K) * 5 % 16).astype(np.uint8).reshape(N, K)
    wq = O.pack(q, 4)
    one = O.f32_to_bf16(np.ones((N, 2), np.float32))
    zero = np.zeros((N, 2), np.uint16)
    x = np.zeros((3, K), np.float32)
    x[0, 9] = 1.0
    x[1] = 1.0
    x[2] = np.arange(K) % 3
    y = O.qmm_f64(x, wq, one, zero, 64, 4)
    assert np.array_equal(y[0], q[:, 9].astype(np.float64))
    assert np.array_equal(y[1], q.sum(axis=1).astype(np.float64))
    assert np.array_equal(y[2], (q * (np.arange(K) % 3)).sum(axis=1).astype(np.float64))


def test_gather_qmm_per_index_and_broadcast():
    E, N, K = 5, 24, 256
    wq, s, b = O.make_weight(E * N, K, 12)
    wq, s, b = wq.reshape(E, N, -1), s.reshape(E, N, -1), b.reshape(E, N, -1)
    x = O.make_x_bf16(4 * 2, K, 13).reshape(4, 2, K)
    lhs = np.array([3, 0, 0, 2, 1, 3], np.uint32)
    rhs = np.array([4, 4, 0, 1, 2, 3], np.uint32)
    y = O.gather_qmm_f64(x, wq, s, b, lhs, rhs, 6)
    for i in range(6):
        t = O.bf16_to_f32(x[lhs[i]]).astype(np.float64) @ _dense(wq[rhs[i]], s[rhs[i]], b[rhs[i]],
                                                                 64, 4).T
        assert np.allclose(y[i], t, rtol=1e-12, atol=1e-12)
    # lhs absent: lhs(i) = i // lhs_div
    y2 = O.gather_qmm_f64(x, wq, s, b, None, rhs[:4], 4, lhs_div=2)
    y3 = O.gather_qmm_f64(x, wq, s, b, np.array([0, 0, 1, 1], np.uint32), rhs[:4], 4)
    assert np.array_equal(y2, y3)
    # out-of-range indices are refused (the GPU path writes NaN rows for them)
    with pytest.raises(ValueError):
        O.gather_qmm_f64(x, wq, s, b, np.array([9], np.uint32), np.array([0], np.uint32), 1)


# --------------------------------------------------------------- routing --
def test_route_softmax_topk_matches_numpy():
    rng = np.random.default_rng(2)
    T, E, k = 17, 128, 8
    logits = rng.standard_normal((T, E)).astype(np.float32)
    logits[0, 5] = logits[0, 9] = 4.0   # tie: the lower expert id comes first
    inds, scores = O.route_softmax_topk(logits, k)
    p = np.exp(logits.astype(np.float64) - logits.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    order = np.lexsort((np.tile(np.arange(E), (T, 1)), -logits), axis=1)[:, :k]
    assert np.array_equal(inds, order.astype(np.uint32))
    top = np.take_along_axis(p, order, 1)
    assert np.allclose(scores, top / top.sum(1, keepdims=True), rtol=1e-5, atol=1e-7)
    assert inds[0, 0] == 5 and inds[0, 1] == 9


def test_sort_dispatch_matches_argsort():
    rng = np.random.default_rng(3)
    k = 8
    flat = rng.integers(0, 128, size=64 * k).astype(np.uint32)
    order, inv, srt, lhs = O.sort_dispatch(flat, k)
    ref = np.argsort(flat, kind="stable")
    assert np.array_equal(order, ref)
    assert np.array_equal(inv[order], np.arange(flat.size))
    assert np.array_equal(srt, flat[ref]) and (np.diff(srt.astype(np.int64)) >= 0).all()
    assert np.array_equal(lhs, ref // k)
    assert np.array_equal(srt[inv], flat)


# ---------------------------------------------------- fused tail contracts --
def test_sigmoid_table_exhaustive():
    # every bf16 pattern: numpy's float64 sigmoid, rounded to fp32 then to bf16
    t = O.sigmoid_table_bf16()
    v = O.bf16_to_f32(np.arange(65536, dtype=np.uint32).astype(np.uint16)).astype(np.float64)
    ok = ~np.isnan(v)
    with np.errstate(over="ignore"):
        sig = 1.0 / (1.0 + np.exp(-v[ok]))
    assert np.array_equal(t[ok], O.f32_to_bf16(sig.astype(np.float32)))
    assert np.isnan(O.bf16_to_f32(t[~ok])).all()


def test_swiglu_and_down_reduce_compositions():
    rng = np.random.default_rng(4)
    g = O.f32_to_bf16(rng.standard_normal(4096).astype(np.float32))
    u = O.f32_to_bf16(rng.standard_normal(4096).astype(np.float32))
    tg = torch.from_numpy(g.view(np.int16)).view(torch.bfloat16)
    tu = torch.from_numpy(u.view(np.int16)).view(torch.bfloat16)
    sig = torch.from_numpy(O.sigmoid_table_bf16()[g].view(np.int16)).view(torch.bfloat16)
    want = ((tg * sig) * tu).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.swiglu_bf16(g, u), want)
    v = O.f32_to_bf16(rng.standard_normal((8, 300)).astype(np.float32))
    sc = O.f32_to_bf16(rng.random(8).astype(np.float32))
    tv = torch.from_numpy(v.view(np.int16)).view(torch.bfloat16)
    ts = torch.from_numpy(sc.view(np.int16)).view(torch.bfloat16)
    acc = torch.zeros(300, dtype=torch.bfloat16)
    for j in range(8):
        acc = acc + tv[j] * ts[j]
    assert np.array_equal(O.down_reduce_bf16(v, sc), acc.view(torch.int16).numpy().view(np.uint16))


# -------------------------------------------------------- geometry solve --
def test_geometry_cases_from_reference_tests():
    cases = json.load(open(os.path.join(GOLDEN, "geometry_cases.json")))["cases"]
    for c in cases:
        got = O.affine_params_from_geometry(c["w_cols"], c["s_cols"], c["in_dim"])
        want = None if c["bits"] is None else (c["bits"], c["group_size"])
        assert got == want, c["name"]
    assert O.affine_params_from_geometry(512, 64, 4096) == (4, 64)
    assert O.affine_params_from_geometry(1024, 64, 4096) == (8, 64)


# --------------------------------------------------- microscaling fp modes --
def test_fp_element_decoders_match_the_format_tables():
    # OCP MX v1.0 element tables: e2m1 magnitudes 0, .5, 1, 1.5, 2, 3, 4, 6 (sign bit 3);
    # e4m3 1.0 = 0x38, max normal 0x7E = 448, min subnormal 0x01 = 2^-9, and 0x7F decodes
    # to 480 (no NaN code, as the reference's bit construction); e8m0 2^(b-127), b=0 2^-127.
    assert [O.fp_element(c, "e2m1") for c in range(8)] == [0, .5, 1, 1.5, 2, 3, 4, 6]
    assert [O.fp_element(c | 8, "e2m1") for c in range(1, 8)] == [-.5, -1, -1.5, -2, -3, -4, -6]
    assert O.fp_element(0x38, "e4m3") == 1.0 and O.fp_element(0xB8, "e4m3") == -1.0
    assert O.fp_element(0x7E, "e4m3") == 448.0 and O.fp_element(0x7F, "e4m3") == 480.0
    assert O.fp_element(0x01, "e4m3") == 2.0 ** -9 and O.fp_element(0x08, "e4m3") == 2.0 ** -6
    assert O.fp_element(0x80, "e4m3") == 0.0
    assert O.fp_element(127, "e8m0") == 1.0 and O.fp_element(130, "e8m0") == 8.0
    assert O.fp_element(0, "e8m0") == 2.0 ** -127 and O.fp_element(254, "e8m0") == 2.0 ** 127
    # every e4m3 byte against the bit-level definition via a float16 view: the byte's low
    # 7 bits shifted left by 7 are a float16 of value/256 (the reference's construction)
    for b in range(256):
        h = np.array([((b & 0x7F) << 7) | ((b & 0x80) << 8)], np.uint16).view(np.float16)
        assert O.fp_element(b, "e4m3") == float(h[0]) * 256.0
    for c in range(16):
        h = np.array([((c & 7) << 9) | ((c & 8) << 12)], np.uint16).view(np.float16)
        assert O.fp_element(c, "e2m1") == float(h[0]) * 2.0 ** 14


@pytest.mark.parametrize("mode", ["nvfp4", "mxfp4", "mxfp8"])
def test_dequantize_fp_closed_form(mode):
    m, bits, gs = O.FP_MODES[mode]
    rng = np.random.default_rng(m)
    N, K = 8, 128
    q = rng.integers(0, 1 << bits, size=(N, K)).astype(np.uint8)
    sc = rng.integers(100, 140, size=(N, K // gs)).astype(np.uint8)
    wq = O.pack(q, bits)
    el = "e4m3" if mode == "mxfp8" else "e2m1"
    sf = "e4m3" if mode == "nvfp4" else "e8m0"
    tab_el = np.array([O.fp_element(c, el) for c in range(1 << bits)], np.float64)
    tab_sc = np.array([O.fp_element(c, sf) for c in range(256)], np.float64)
    exact = tab_el[q] * np.repeat(tab_sc[sc], gs, axis=1)
    f32 = O.dequantize_fp(wq, sc, mode)
    assert np.array_equal(f32.astype(np.float64), exact)  # exact in fp32
    assert np.array_equal(O.dequantize_fp(wq, sc, mode, out_bf16=True),
                          O.f32_to_bf16(exact.astype(np.float32)))
    assert np.array_equal(O.bf16_to_f32(O.dequantize_fp(wq, sc, mode, out_bf16=True)), f32)


def _sigmoid_topk_np(logits, bias, k):
    """Plain descending top-k of sigmoid(logits) + bias, ties to the lower id (numpy)."""
    keys = 1.0 / (1.0 + np.exp(-logits.astype(np.float64))) + bias.astype(np.float64)
    E = keys.shape[-1]
    return np.stack([np.lexsort((np.arange(E), -row))[:k] for row in keys])


def test_route_grouped_reduces_to_plain_topk():
    """One group, or every group surviving, leaves nothing masked: the selection is the
    plain top-k of sigmoid + bias, and the weights are the unbiased sigmoids normalized
    over the selected (then scaled)."""
    rng = np.random.default_rng(3)
    T, E, k = 40, 64, 6
    logits = ((rng.random((T, E)) - 0.5) * 6).astype(np.float32)
    bias = ((rng.random(E) - 0.5) * 0.2).astype(np.float32)
    want = _sigmoid_topk_np(logits, bias, k)
    for ng, tg in ((1, 1), (8, 8), (4, 4)):
        inds, w = O.route_grouped(logits, bias, k, ng, tg, True, 2.5)
        assert np.array_equal(inds, want)
        sig = 1.0 / (1.0 + np.exp(-logits.astype(np.float64)))
        sel = np.take_along_axis(sig, want.astype(np.int64), axis=1)
        assert np.allclose(w, 2.5 * sel / (sel.sum(1, keepdims=True) + 1e-20), rtol=1e-12)
    # route_norm off and k == 1: raw sigmoid times the scale
    inds, w = O.route_grouped(logits, bias, 1, 1, 1, True, 1.0)
    sig = 1.0 / (1.0 + np.exp(-logits.astype(np.float64)))
    assert np.allclose(w[:, 0], sig[np.arange(T), inds[:, 0]], rtol=1e-12)


def test_route_grouped_masks_losing_groups():
    """Two groups of four, one kept: expert 0 has the single largest key but its group's
    top-two sum loses, so every selected expert comes from group 1."""
    logits = np.full((1, 8), -5.0, np.float32)
    logits[0, 0] = 5.0                      # best single expert, group 0
    logits[0, 4:7] = [3.0, 2.9, 2.8]        # group 1: larger top-two sum
    bias = np.zeros(8, np.float32)
    inds, _ = O.route_grouped(logits, bias, 2, 2, 1, True, 1.0)
    assert list(inds[0]) == [4, 5]
    inds, _ = O.route_grouped(logits, bias, 2, 2, 2, True, 1.0)  # no limit
    assert list(inds[0]) == [0, 4]


def test_route_grouped_shipped_geometry_numpy():
    """The reference test's geometry (src/transformer.zig:23390: E=512, 8 groups, 4 kept,
    k=8, route_scale 2.5, 256 rows, logits (u-0.5)*6 + (i%7)*0.011, bias (u-0.5)*0.2)
    against an independent numpy statement: group scores from a sort, groups and experts
    chosen by lexsort (ties to the lower id)."""
    rng = np.random.default_rng(0x116C0DE)
    R, E, k, NG, TG, scale = 256, 512, 8, 8, 4, 2.5
    logits = ((rng.random((R, E)) - 0.5) * 6.0 +
              (np.arange(R * E) % 7).reshape(R, E) * 0.011).astype(np.float32)
    bias = ((rng.random(E) - 0.5) * 0.2).astype(np.float32)
    inds, w = O.route_grouped(logits, bias, k, NG, TG, True, scale)
    sig = 1.0 / (1.0 + np.exp(-logits.astype(np.float64)))
    keys = sig + bias.astype(np.float64)
    gsz = E // NG
    gs = np.sort(keys.reshape(R, NG, gsz), axis=2)[:, :, -2:].sum(2)
    dropped = 0
    for r in range(R):
        keep = np.lexsort((np.arange(NG), -gs[r]))[:TG]
        allowed = np.zeros(E, bool)
        for g in keep:
            allowed[g * gsz:(g + 1) * gsz] = True
        masked = np.where(allowed, keys[r], -1e4)
        want = np.lexsort((np.arange(E), -masked))[:k]
        assert list(inds[r]) == list(want), r
        sel = sig[r, want]
        assert np.allclose(w[r], scale * sel / (sel.sum() + 1e-20), rtol=1e-12)
        dropped += int(np.any(np.lexsort((np.arange(E), -keys[r]))[:k] != want))
    assert dropped > 0  # the group limit changed some rows' selection


def test_dequantize_fp_global_scale():
    """nvfp4's global scale: 1.0 changes nothing; a power of two scales every value
    exactly (fp32 and bf16 alike); other modes refuse it."""
    rng = np.random.default_rng(8)
    q = rng.integers(0, 16, size=(4, 64)).astype(np.uint8)
    wq = O.pack(q, 4)
    sc = rng.integers(0x20, 0x48, size=(4, 4)).astype(np.uint8)
    base = O.dequantize_fp(wq, sc, "nvfp4")
    assert np.array_equal(O.dequantize_fp(wq, sc, "nvfp4", global_scale=1.0).view(np.uint32),
                          base.view(np.uint32))
    for p2 in (0.25, 8.0):
        assert np.array_equal(O.dequantize_fp(wq, sc, "nvfp4", global_scale=p2), base * p2)
        assert np.array_equal(O.dequantize_fp(wq, sc, "nvfp4", out_bf16=True, global_scale=p2),
                              O.f32_to_bf16(base * np.float32(p2)))
    # a general scale: the exact element*scale product times g, rounded once in fp32
    g = np.float32(1 / 3)
    assert np.array_equal(O.dequantize_fp(wq, sc, "nvfp4", global_scale=float(g)), base * g)
    with pytest.raises(ValueError):
        O.dequantize_fp(O.pack(q, 4), rng.integers(118, 126, (4, 2)).astype(np.uint8), "mxfp4",
                        global_scale=2.0)
