"""ctypes/numpy front end of the CPU oracle (oracle/mi_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker. The product (libmi_qmm.so
and the mi_qmm package) never imports it.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

DQ_F32, DQ_BF16_FUSED, DQ_BF16_OPWISE = 0, 1, 2


def build():
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        L = _lib
        P = ctypes.c_void_p
        i64, i32, u64, f64 = ctypes.c_int64, ctypes.c_int, ctypes.c_uint64, ctypes.c_double
        L.mo_randn_f32.argtypes = [P, i64, u64, f64, f64]
        L.mo_uniform_f64.argtypes = [P, i64, u64]
        L.mo_splitmix64.argtypes = [u64, u64]
        L.mo_splitmix64.restype = u64
        L.mo_f32_to_bf16_array.argtypes = [P, P, i64]
        L.mo_bf16_to_f32_array.argtypes = [P, P, i64]
        L.mo_pack.argtypes = [P, i64, i64, i32, P]
        L.mo_unpack.argtypes = [P, i64, i64, i32, P]
        L.mo_quantize_bf16.argtypes = [P, i64, i64, i32, i32, P, P, P]
        L.mo_dequantize.argtypes = [P, P, P, i64, i64, i32, i32, i32, P]
        L.mo_dequantize_fp.argtypes = [P, P, i64, i64, i32, i32, P]
        L.mo_dequantize_fp_gs.argtypes = [P, P, i64, i64, i32, i32, i32, ctypes.c_float, P]
        for f in (L.mo_e2m1, L.mo_e4m3, L.mo_e8m0):
            f.argtypes = [ctypes.c_uint32]
            f.restype = ctypes.c_float
        L.mo_qmm_f64.argtypes = [P, i32, P, P, P, i64, i64, i64, i32, i32, P]
        L.mo_qmm_f32.argtypes = [P, P, P, P, i64, i64, i64, i32, i32, P, i32]
        L.mo_gather_qmm_f64.argtypes = [P, i32, P, P, P, P, P, i64, i64, i64, i64, i64,
                                        i64, i64, i32, i32, P]
        L.mo_route_softmax_topk.argtypes = [P, i64, i64, i32, P, P]
        L.mo_sort_dispatch.argtypes = [P, i64, i32, P, P, P, P]
        L.mo_route_grouped_f64.argtypes = [P, P, i64, i64, i32, i32, i32, i32, f64, P, P]
        L.mo_sigmoid_table_bf16.argtypes = [P]
        L.mo_swiglu_bf16.argtypes = [P, P, i64, P]
        L.mo_down_reduce_bf16.argtypes = [P, P, i64, i64, P]
        L.mo_affine_params_from_geometry.argtypes = [i64, i64, i64, ctypes.POINTER(i32),
                                                     ctypes.POINTER(i32)]
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _check(rc, what):
    if rc != 0:
        raise ValueError(f"oracle {what} failed rc={rc}")


# ---------------------------------------------------------------- helpers --
def bf16_to_f32(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    return (h.astype(np.uint32) << 16).view(np.float32).reshape(h.shape)


def f32_to_bf16(f):
    f = np.ascontiguousarray(f, dtype=np.float32)
    out = np.empty(f.shape, dtype=np.uint16)
    lib().mo_f32_to_bf16_array(_p(f), _p(out), f.size)
    return out


def randn(n, seed, mean=0.0, std=1.0):
    out = np.empty(n, dtype=np.float32)
    lib().mo_randn_f32(_p(out), n, seed, mean, std)
    return out


def uniform(n, seed):
    out = np.empty(n, dtype=np.float64)
    lib().mo_uniform_f64(_p(out), n, seed)
    return out


def seed_for(cfg, stream):
    """Seed convention: 0x4D493335_00000000 + 16*cfg + stream."""
    return 0x4D49333500000000 + 16 * cfg + stream


# --------------------------------------------------------------- packing --
def pack(q, bits):
    q = np.ascontiguousarray(q, dtype=np.uint8)
    rows, K = q.shape
    out = np.empty((rows, K * bits // 32), dtype=np.uint32)
    _check(lib().mo_pack(_p(q), rows, K, bits, _p(out)), "pack")
    return out


def unpack(wq, K, bits):
    wq = np.ascontiguousarray(wq, dtype=np.uint32)
    rows = wq.size // (K * bits // 32)
    out = np.empty((rows, K), dtype=np.uint8)
    _check(lib().mo_unpack(_p(wq), rows, K, bits, _p(out)), "unpack")
    return out


def quantize(w_bf16, group_size=64, bits=4):
    """w bf16 bits (uint16) [..., K] -> (wq u32, scales bf16, biases bf16)."""
    w = np.ascontiguousarray(w_bf16, dtype=np.uint16)
    K = w.shape[-1]
    rows = w.size // K
    lead = w.shape[:-1]
    wq = np.empty(lead + (K * bits // 32,), dtype=np.uint32)
    s = np.empty(lead + (K // group_size,), dtype=np.uint16)
    b = np.empty(lead + (K // group_size,), dtype=np.uint16)
    _check(lib().mo_quantize_bf16(_p(w), rows, K, group_size, bits, _p(wq), _p(s), _p(b)),
           "quantize")
    return wq, s, b


FP_MODES = {"nvfp4": (0, 4, 16), "mxfp4": (1, 4, 32), "mxfp8": (2, 8, 32)}


def fp_element(code, fmt):
    """One decoded e2m1 / e4m3 / e8m0 value (float)."""
    return float({"e2m1": lib().mo_e2m1, "e4m3": lib().mo_e4m3, "e8m0": lib().mo_e8m0}[fmt](code))


def dequantize_fp(wq, scales_u8, mode, out_bf16=False, global_scale=None):
    """Bias-less microscaling modes: wq [..., K*bits/32] u32, scales [..., K/gs] uint8."""
    m, bits, gs = FP_MODES[mode]
    wq = np.ascontiguousarray(wq, dtype=np.uint32)
    sc = np.ascontiguousarray(scales_u8, dtype=np.uint8)
    K = wq.shape[-1] * 32 // bits
    rows = wq.size // wq.shape[-1]
    out = np.empty(tuple(wq.shape[:-1]) + (K,), dtype=np.uint16 if out_bf16 else np.float32)
    _check(lib().mo_dequantize_fp_gs(_p(wq), _p(sc), rows, K, m, int(out_bf16),
                                     int(global_scale is not None),
                                     float(1.0 if global_scale is None else global_scale),
                                     _p(out)),
           "dequantize_fp")
    return out


def dequantize(wq, scales, biases, group_size=64, bits=4, kind=DQ_F32):
    wq = np.ascontiguousarray(wq, dtype=np.uint32)
    scales = np.ascontiguousarray(scales, dtype=np.uint16)
    biases = np.ascontiguousarray(biases, dtype=np.uint16)
    K = wq.shape[-1] * 32 // bits
    rows = wq.size // wq.shape[-1]
    shape = wq.shape[:-1] + (K,)
    out = np.empty(shape, dtype=np.float32 if kind == DQ_F32 else np.uint16)
    _check(lib().mo_dequantize(_p(wq), _p(scales), _p(biases), rows, K, group_size, bits,
                               kind, _p(out)), "dequantize")
    return out


def qmm_f64(x, wq, scales, biases, group_size=64, bits=4):
    """x: float32 array or uint16 (bf16 bits) [M, K]."""
    x = np.ascontiguousarray(x)
    x_f32 = 1 if x.dtype == np.float32 else 0
    K = x.shape[-1]
    M = x.size // K
    N = wq.shape[-2] if wq.ndim >= 2 else 1
    y = np.empty((M, N), dtype=np.float64)
    _check(lib().mo_qmm_f64(_p(x), x_f32, _p(np.ascontiguousarray(wq)),
                            _p(np.ascontiguousarray(scales)), _p(np.ascontiguousarray(biases)),
                            M, N, K, group_size, bits, _p(y)), "qmm_f64")
    return y


def qmm_f32(x_bf16, wq, scales, biases, group_size=64, bits=4, threads=0):
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    K = x.shape[-1]
    M = x.size // K
    N = wq.shape[-2]
    y = np.empty((M, N), dtype=np.float32)
    _check(lib().mo_qmm_f32(_p(x), _p(wq), _p(scales), _p(biases), M, N, K, group_size, bits,
                            _p(y), threads), "qmm_f32")
    return y


def gather_qmm_f64(x, wq, scales, biases, lhs, rhs, n_idx, lhs_div=1, group_size=64, bits=4):
    """x [x_batch, M, K]; wq [E, N, K*bits/32]; returns [n_idx, M, N] float64."""
    x = np.ascontiguousarray(x)
    x_f32 = 1 if x.dtype == np.float32 else 0
    x_batch, M, K = x.shape
    E, N = wq.shape[0], wq.shape[1]
    lhs_a = None if lhs is None else np.ascontiguousarray(lhs, dtype=np.uint32)
    rhs_a = None if rhs is None else np.ascontiguousarray(rhs, dtype=np.uint32)
    out = np.empty((n_idx, M, N), dtype=np.float64)
    _check(lib().mo_gather_qmm_f64(_p(x), x_f32, _p(np.ascontiguousarray(wq)),
                                   _p(np.ascontiguousarray(scales)),
                                   _p(np.ascontiguousarray(biases)), _p(lhs_a), _p(rhs_a),
                                   n_idx, lhs_div, M, N, K, x_batch, E, group_size, bits,
                                   _p(out)), "gather_qmm_f64")
    return out


def route_softmax_topk(logits, k):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    T, E = logits.shape
    inds = np.empty((T, k), dtype=np.uint32)
    scores = np.empty((T, k), dtype=np.float32)
    _check(lib().mo_route_softmax_topk(_p(logits), T, E, k, _p(inds), _p(scores)), "route")
    return inds, scores


def route_grouped(logits, bias, k, n_group, topk_group, route_norm=True, route_scale=1.0):
    """Group-limited routing in float64 -> (inds uint32 [T, k], weights float64 [T, k])."""
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    bias = np.ascontiguousarray(bias, dtype=np.float32)
    T, E = logits.shape
    inds = np.empty((T, k), dtype=np.uint32)
    w = np.empty((T, k), dtype=np.float64)
    _check(lib().mo_route_grouped_f64(_p(logits), _p(bias), T, E, k, n_group, topk_group,
                                      int(route_norm), float(route_scale), _p(inds), _p(w)),
           "route_grouped")
    return inds, w


def sort_dispatch(flat, k):
    flat = np.ascontiguousarray(flat, dtype=np.uint32).reshape(-1)
    n = flat.size
    order, inv, srt, lhs = (np.empty(n, dtype=np.uint32) for _ in range(4))
    _check(lib().mo_sort_dispatch(_p(flat), n, k, _p(order), _p(inv), _p(srt), _p(lhs)), "sort")
    return order, inv, srt, lhs


def sigmoid_table_bf16():
    t = np.empty(65536, dtype=np.uint16)
    lib().mo_sigmoid_table_bf16(_p(t))
    return t


def swiglu_bf16(g, u):
    g = np.ascontiguousarray(g, dtype=np.uint16)
    u = np.ascontiguousarray(u, dtype=np.uint16)
    y = np.empty_like(g)
    lib().mo_swiglu_bf16(_p(g), _p(u), g.size, _p(y))
    return y


def down_reduce_bf16(v, scores):
    v = np.ascontiguousarray(v, dtype=np.uint16)
    scores = np.ascontiguousarray(scores, dtype=np.uint16)
    topk, N = v.shape
    y = np.empty(N, dtype=np.uint16)
    lib().mo_down_reduce_bf16(_p(v), _p(scores), topk, N, _p(y))
    return y


def affine_params_from_geometry(w_cols, s_cols, in_dim):
    b, g = ctypes.c_int(0), ctypes.c_int(0)
    rc = lib().mo_affine_params_from_geometry(w_cols, s_cols, in_dim, ctypes.byref(b),
                                              ctypes.byref(g))
    return None if rc != 0 else (b.value, g.value)


# ------------------------------------------------------- input generation --
def make_weight(N, K, seed, bits=4, group_size=64, std=0.02):
    """W ~ N(0, std) fp32 -> bf16 -> affine quantize (the reference tests cast to bf16
    before quantizing, src/transformer.zig:24853-24858)."""
    w = f32_to_bf16(randn(N * K, seed, 0.0, std).reshape(N, K))
    return quantize(w, group_size, bits)


def make_x_bf16(M, K, seed):
    return f32_to_bf16(randn(M * K, seed).reshape(M, K))
