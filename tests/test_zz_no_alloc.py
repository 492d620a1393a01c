"""mi_gather_qmm_noalloc (fixed per-device scratch, no allocation inside the library)
against mi_gather_qmm through the C ABI: bit-equal outputs on two calls in a row, the
second smaller, covering work items (sorted runs) and K-split partials; calls whose
scratch need exceeds the fixed maximum are refused."""
import numpy as np
import pytest
import torch

import oracle as O
from helpers import bf16_bits, to_dev_bf16, to_dev_u32, weights
import mi_qmm
from mi_qmm._lib import opt

pytestmark = pytest.mark.gpu

MI_ERR_WORKSPACE = 4


def _case(**kw):
    print("CASE", kw, flush=True)


def _run_pair(dev, E, N, K, T, topk, seed):
    """Sorted gather through both entry points; returns (noalloc bits, regular bits)."""
    wq, s, b = weights(E, N, K, 4, 64, seed)
    rng = np.random.default_rng(seed)
    flat = rng.integers(0, E, size=T * topk).astype(np.uint32)
    _, _, srt, lhs = O.sort_dispatch(flat, topk)
    x = to_dev_bf16(O.make_x_bf16(T, K, seed + 1).reshape(T, 1, K), dev)
    W, S, B = to_dev_u32(wq, dev), to_dev_bf16(s, dev), to_dev_bf16(b, dev)
    L, R = to_dev_u32(lhs, dev), to_dev_u32(srt, dev)
    kw = dict(lhs_indices=L, rhs_indices=R, group_size=64, bits=4, sorted_indices=True)
    y0 = mi_qmm.gather_qmm(x, W, S, B, noalloc=True, **kw)
    y1 = mi_qmm.gather_qmm(x, W, S, B, **kw)
    torch.cuda.synchronize()
    return bf16_bits(y0), bf16_bits(y1)


@pytest.mark.parametrize("first,second", [
    # (E, N, K, T, topk): sorted runs of the few-row kernel, K split over 4 ranges at 8192
    ((8, 64, 8192, 64, 4), (4, 64, 8192, 16, 4)),
    # configs[3]-like gate bank at T=512 (many work items), then T=32
    ((128, 768, 2048, 512, 8), (128, 768, 2048, 32, 8)),
    # one-row items (decode-like), then fewer pairs
    ((64, 512, 4096, 4, 8), (64, 512, 4096, 1, 8)),
])
def test_noalloc_matches_gather(dev, first, second):
    for i, case in enumerate((first, second)):
        _case(t="noalloc", call=i, case=case)
        a, b = _run_pair(dev, *case, seed=300 + 10 * i)
        assert a.shape == b.shape
        assert np.array_equal(a, b)


@pytest.mark.parametrize("mode", ["nvfp4", "mxfp4", "mxfp8"])
def test_noalloc_matches_gather_fp4(dev, mode):
    """fp4 sorted gathers (work items in scratch) through both entry points, two calls in a
    row, the second smaller."""
    for i, (E, N, K, T, topk) in enumerate(((16, 96, 4096, 64, 8), (8, 64, 1024, 16, 4))):
        _case(t="noalloc_fp4", mode=mode, call=i)
        m, bits, gs = O.FP_MODES[mode]
        rng = np.random.default_rng(400 + i)
        q = rng.integers(0, 1 << bits, size=(E * N, K)).astype(np.uint8)
        wq = O.pack(q, bits).reshape(E, N, -1)
        lo, hi = (0x20, 0x48) if mode == "nvfp4" else (118, 126)
        sc = rng.integers(lo, hi, size=(E, N, K // gs)).astype(np.uint8)
        flat = np.concatenate([rng.permutation(E)[:topk] for _ in range(T)]).astype(np.uint32)
        _, _, srt, lhs = O.sort_dispatch(flat, topk)
        x = to_dev_bf16(O.make_x_bf16(T, K, 401 + i).reshape(T, 1, K), dev)
        W, S = to_dev_u32(wq, dev), torch.from_numpy(sc).to(dev)
        kw = dict(lhs_indices=to_dev_u32(lhs, dev), rhs_indices=to_dev_u32(srt, dev),
                  mode=mode, sorted_indices=True)
        y0 = mi_qmm.gather_qmm(x, W, S, None, noalloc=True, **kw)
        y1 = mi_qmm.gather_qmm(x, W, S, None, **kw)
        torch.cuda.synchronize()
        assert np.array_equal(bf16_bits(y0), bf16_bits(y1))


def test_noalloc_allocates_no_device_memory(dev):
    """Device free memory is unchanged across no-alloc calls that need scratch (a sorted
    gather with many work items and a K-split gather), after one warm-up call so the runtime's
    own first-use allocations are out of the picture. A library that grew its workspace or
    called hipMalloc would lower it by at least its 1 MiB minimum generation."""
    _case(t="noalloc_free_memory")
    cases = [(128, 768, 2048, 512, 8), (8, 64, 8192, 64, 4)]
    prepared = []
    for i, (E, N, K, T, topk) in enumerate(cases):
        wq, s, b = weights(E, N, K, 4, 64, 500 + i)
        rng = np.random.default_rng(500 + i)
        flat = rng.integers(0, E, size=T * topk).astype(np.uint32)
        _, _, srt, lhs = O.sort_dispatch(flat, topk)
        x = to_dev_bf16(O.make_x_bf16(T, K, 501 + i).reshape(T, 1, K), dev)
        W, S, B = to_dev_u32(wq, dev), to_dev_bf16(s, dev), to_dev_bf16(b, dev)
        kw = dict(lhs_indices=to_dev_u32(lhs, dev), rhs_indices=to_dev_u32(srt, dev),
                  group_size=64, bits=4, sorted_indices=True, noalloc=True)
        out = torch.empty(T * topk, 1, N, dtype=torch.bfloat16, device=dev)
        prepared.append((x, W, S, B, kw, out))
    for (x, W, S, B, kw, out) in prepared:  # warm-up
        mi_qmm.gather_qmm(x, W, S, B, out=out, **kw)
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info()
    for (x, W, S, B, kw, out) in prepared:
        mi_qmm.gather_qmm(x, W, S, B, out=out, **kw)
    torch.cuda.synchronize()
    free1, _ = torch.cuda.mem_get_info()
    assert free1 == free0


def test_noalloc_rejects_oversized_scratch_fp_mode(dev):
    """The fp-mode path's size guard: an nvfp4 sorted gather of 4.2M pairs on one expert needs
    4.2M + 131K work items (69 MB) of scratch: refused before any launch."""
    _case(t="noalloc_oversize_fp")
    n = 4_200_000
    K, N, E = 1024, 64, 1
    m, bits, gs = O.FP_MODES["nvfp4"]
    rng = np.random.default_rng(11)
    q = rng.integers(0, 1 << bits, size=(E * N, K)).astype(np.uint8)
    wq = O.pack(q, bits).reshape(E, N, -1)
    sc = rng.integers(0x20, 0x48, size=(E, N, K // gs)).astype(np.uint8)
    x = torch.zeros(1, 1, K, dtype=torch.bfloat16, device=dev)
    rhs = torch.zeros(n, dtype=torch.int32, device=dev)
    W, S = to_dev_u32(wq, dev), torch.from_numpy(sc).to(dev)
    y = torch.empty(n, 1, N, dtype=torch.bfloat16, device=dev)
    rc = mi_qmm._lib.lib().mi_gather_qmm_noalloc(
        y.data_ptr(), x.data_ptr(), W.data_ptr(), S.data_ptr(), None, None,
        rhs.data_ptr(), n, n, 1, 1, N, K, E, True, opt(None), opt(None), b"nvfp4", True, 12, 1,
        None)
    assert rc == MI_ERR_WORKSPACE
    assert "scratch" in mi_qmm._lib.last_error()


def test_noalloc_rejects_oversized_scratch(dev):
    """4M one-row pairs need 128 MiB of work items: refused before any launch."""
    _case(t="noalloc_oversize")
    n = 1 << 22
    K, N = 128, 16
    wq, s, b = weights(1, N, K, 4, 64, 9)
    x = torch.zeros(1, 1, K, dtype=torch.bfloat16, device=dev)
    rhs = torch.zeros(n, dtype=torch.int32, device=dev)
    W, S, B = to_dev_u32(wq, dev), to_dev_bf16(s, dev), to_dev_bf16(b, dev)
    y = torch.empty(n, 1, N, dtype=torch.bfloat16, device=dev)
    rc = mi_qmm._lib.lib().mi_gather_qmm_noalloc(
        y.data_ptr(), x.data_ptr(), W.data_ptr(), S.data_ptr(), B.data_ptr(), None,
        rhs.data_ptr(), n, n, 1, 1, N, K, 1, True, opt(64), opt(4), b"affine", True, 12, 12,
        None)
    assert rc == MI_ERR_WORKSPACE
    assert "scratch" in mi_qmm._lib.last_error()
