"""Shared test helpers: move oracle (numpy) inputs to the GPU and compare."""
import numpy as np
import torch

import oracle as O


def to_dev_bf16(a, dev):
    """uint16 bf16 bits (numpy) -> torch bf16 on dev."""
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).to(dev)


def to_dev_u32(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int32)).to(dev)


def bf16_bits(t):
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


def to_f64(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def max_err_ratio(y, truth):
    """max|y - truth| / max|truth| (the north-star tolerance form)."""
    denom = np.max(np.abs(truth))
    return float(np.max(np.abs(y - truth)) / (denom if denom > 0 else 1.0))


BF16_TOL = 1e-2   # max-abs-err <= 1e-2 * ||y||_inf for bf16 output
F32_TOL = 1e-3    # max-abs-err <= 1e-3 * ||y||_inf for fp32 output


def weights(E, N, K, bits, gs, seed, std=0.02):
    w = O.f32_to_bf16(O.randn(E * N * K, seed, 0.0, std).reshape(E * N, K))
    wq, s, b = O.quantize(w, gs, bits)
    return (wq.reshape(E, N, -1), s.reshape(E, N, -1), b.reshape(E, N, -1))
