"""MLX-shaped ops over torch device tensors, each one call into libmi_qmm.so.

Argument names, defaults and shape rules follow the mlx-c functions that
ddalcu/mlx-serve binds in src/mlx.zig:262-275 (MLX's Python API has the same
signatures): transpose=True, group_size 64 and bits 4 by default, mode "affine".
torch is used only for device memory and the current HIP stream.
"""
import ctypes
import math

import torch

from ._lib import (DT_BFLOAT16, DT_FLOAT32, DT_UINT8, MI_ERR_INVALID, MiError, check, lib, opt)

_DT = {torch.bfloat16: DT_BFLOAT16, torch.float32: DT_FLOAT32, torch.uint8: DT_UINT8}
# bias-less microscaling modes: (group_size, bits) each one defines
_FP_MODES = {"nvfp4": (16, 4), "mxfp4": (32, 4), "mxfp8": (32, 8)}


def _stream(t):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _dtype_code(t, what):
    if t.dtype not in _DT:
        raise MiError(MI_ERR_INVALID, f"{what} dtype {t.dtype} not supported")
    return _DT[t.dtype]


def _packed(w):
    if w.dtype not in (torch.int32, torch.uint32):
        raise MiError(MI_ERR_INVALID, f"packed weights must be 32-bit, got {w.dtype}")
    return w


def _require(cond, msg):
    if not cond:
        raise MiError(MI_ERR_INVALID, msg)


def _defaults(mode):
    return _FP_MODES.get(mode, (64, 4))


def _resolve(w, scales, group_size, bits, K, mode="affine"):
    """MLX defaults ((64, 4) for affine, the mode's own otherwise); validate against the
    packed geometry."""
    dgs, dnb = _defaults(mode)
    gs = dgs if group_size is None else int(group_size)
    nb = dnb if bits is None else int(bits)
    _require(w.shape[-1] * 32 == K * nb,
             f"packed width {w.shape[-1]} does not match K={K} at bits={nb}")
    _require(scales.shape[-1] * gs == K,
             f"scales width {scales.shape[-1]} does not match K={K} at group_size={gs}")
    return gs, nb


def _contig(*ts):
    for t in ts:
        if t is not None:
            _require(t.is_contiguous(), "tensors must be row-contiguous")
            _require(t.is_cuda, "tensors must be on the GPU")


def quantized_matmul(x, w, scales, biases, transpose=True, group_size=None, bits=None,
                     mode="affine"):
    """y = x @ dequantize(w).T (mlx_quantized_matmul, src/mlx.zig:262). x [..., K]."""
    _contig(x, w, scales, biases)
    K = x.shape[-1]
    gs, nb = _resolve(_packed(w), scales, group_size, bits, K, mode)
    _require(w.dim() == 2, "w must be [N, K*bits/32]")
    N = w.shape[0]
    M = x.numel() // K if K else 0
    y = torch.empty(x.shape[:-1] + (N,), dtype=x.dtype, device=x.device)
    check(lib().mi_quantized_matmul(_ptr(y), _ptr(x), _ptr(w), _ptr(scales), _ptr(biases), M, N,
                                    K, bool(transpose), opt(gs), opt(nb),
                                    mode.encode() if mode else None, _dtype_code(x, "x"),
                                    _dtype_code(scales, "scales"), _stream(x)))
    return y


def _broadcast_indices(x, w, lhs_indices, rhs_indices):
    """MLX gather_qmm index rules: defaults are aranges over the batch dims of x and
    w, both broadcast together. Returns (lhs or None, lhs_div, rhs or None, shape)."""
    xb = tuple(x.shape[:-2])
    wb = tuple(w.shape[:-2])
    dev = x.device
    lhs_shape = tuple(lhs_indices.shape) if lhs_indices is not None else xb
    rhs_shape = tuple(rhs_indices.shape) if rhs_indices is not None else wb
    shape = torch.broadcast_shapes(lhs_shape, rhs_shape)
    n = math.prod(shape)

    def as_u32(t):
        t = t.to(dev)
        if t.dtype not in (torch.int32, torch.uint32):
            t = t.to(torch.int32)
        return t.contiguous()

    wb_full = (1,) * (len(shape) - len(wb)) + wb
    if rhs_indices is None:
        rhs = None if wb_full == shape else as_u32(
            torch.arange(math.prod(wb), device=dev, dtype=torch.int32).reshape(wb_full)
            .expand(shape))
    else:
        rhs = as_u32(rhs_indices.expand(shape) if tuple(rhs_indices.shape) != shape
                     else rhs_indices)

    if lhs_indices is not None:
        lhs = lhs_indices
        lhs = as_u32(lhs.expand(shape) if tuple(lhs.shape) != shape else lhs)
        return lhs, 1, rhs, shape
    # Default lhs = arange over x's batch dims. Common patterns need no index array:
    # x batch == shape (one row per pair) or x batch == shape[:-1] + (1,) (one token
    # broadcast over the trailing top-k axis).
    xb_full = (1,) * (len(shape) - len(xb)) + xb
    if xb_full == shape:
        return None, 1, rhs, shape
    if len(shape) >= 1 and xb_full[:-1] == shape[:-1] and xb_full[-1] == 1:
        return None, shape[-1], rhs, shape
    lhs = torch.arange(math.prod(xb), device=dev, dtype=torch.int32).reshape(xb_full)
    return as_u32(lhs.expand(shape)), 1, rhs, shape


def gather_qmm(x, w, scales, biases, lhs_indices=None, rhs_indices=None, transpose=True,
               group_size=None, bits=None, mode="affine", sorted_indices=False, out=None,
               noalloc=False):
    """out[i] = x[lhs[i]] @ dequantize(w[rhs[i]]).T (mlx_gather_qmm, src/mlx.zig:265).
    x [..., M, K], w [..., N, K*bits/32]; out shape = broadcast(lhs, rhs) + [M, N].
    noalloc=True calls mi_gather_qmm_noalloc (fixed library scratch, no device
    allocation inside the library); `out` may supply the result tensor."""
    _contig(x, w, scales, biases)
    _require(x.dim() >= 2 and w.dim() >= 2, "x and w need at least 2 dims")
    K = x.shape[-1]
    M = x.shape[-2]
    gs, nb = _resolve(_packed(w), scales, group_size, bits, K, mode)
    N = w.shape[-2]
    lhs, lhs_div, rhs, shape = _broadcast_indices(x, w, lhs_indices, rhs_indices)
    n_idx = math.prod(shape)
    x_batch = x.numel() // (M * K) if M * K else 0
    n_exp = w.numel() // (N * w.shape[-1]) if N * w.shape[-1] else 0
    y = torch.empty(tuple(shape) + (M, N), dtype=x.dtype, device=x.device) if out is None else out
    _require(tuple(y.shape) == tuple(shape) + (M, N) and y.dtype == x.dtype and y.is_contiguous(),
             "out has the wrong shape, dtype or layout")
    fn = lib().mi_gather_qmm_noalloc if noalloc else lib().mi_gather_qmm
    check(fn(_ptr(y), _ptr(x), _ptr(w), _ptr(scales), _ptr(biases), _ptr(lhs), _ptr(rhs), n_idx,
             lhs_div, x_batch, M, N, K, n_exp, bool(transpose), opt(gs), opt(nb),
             mode.encode() if mode else None, bool(sorted_indices), _dtype_code(x, "x"),
             _dtype_code(scales, "scales"), _stream(x)))
    return y


def gather_qmm_swiglu(gate, x, w, scales, biases, lhs_indices=None, rhs_indices=None,
                      transpose=True, group_size=None, bits=None, mode="affine",
                      sorted_indices=False):
    """swiglu(gate, gather_qmm(x, w, ...)) in one call (the sorted MoE up projection and
    its activation, src/transformer.zig:15009-15023); gate has the product's shape."""
    _contig(gate, x, w, scales, biases)
    _require(x.dim() >= 2 and w.dim() >= 2, "x and w need at least 2 dims")
    K = x.shape[-1]
    M = x.shape[-2]
    gs, nb = _resolve(_packed(w), scales, group_size, bits, K, mode)
    N = w.shape[-2]
    lhs, lhs_div, rhs, shape = _broadcast_indices(x, w, lhs_indices, rhs_indices)
    n_idx = math.prod(shape)
    x_batch = x.numel() // (M * K) if M * K else 0
    n_exp = w.numel() // (N * w.shape[-1]) if N * w.shape[-1] else 0
    y = torch.empty(tuple(shape) + (M, N), dtype=x.dtype, device=x.device)
    _require(gate.numel() == y.numel() and gate.dtype == x.dtype, "gate must match the product")
    check(lib().mi_gather_qmm_swiglu(_ptr(y), _ptr(gate), _ptr(x), _ptr(w), _ptr(scales),
                                     _ptr(biases), _ptr(lhs), _ptr(rhs), n_idx, lhs_div, x_batch,
                                     M, N, K, n_exp, bool(transpose), opt(gs), opt(nb),
                                     mode.encode() if mode else None, bool(sorted_indices),
                                     _dtype_code(x, "x"), _dtype_code(scales, "scales"),
                                     _stream(x)))
    return y


def gather_qmm_gate_up_swiglu(x, wg, sg, bg, wu, su, bu, lhs_indices=None, rhs_indices=None,
                              transpose=True, group_size=None, bits=None, mode="affine",
                              sorted_indices=False):
    """swiglu(gather_qmm(x, wg, ...), gather_qmm(x, wu, ...)) in one call (the sorted MoE
    path's two projections and activation, src/transformer.zig:15009-15023)."""
    _contig(x, wg, sg, bg, wu, su, bu)
    _require(x.dim() >= 2 and wg.dim() >= 2, "x and w need at least 2 dims")
    _require(wg.shape == wu.shape and sg.shape == su.shape, "gate and up banks differ in shape")
    K = x.shape[-1]
    M = x.shape[-2]
    gs, nb = _resolve(_packed(wg), sg, group_size, bits, K, mode)
    N = wg.shape[-2]
    lhs, lhs_div, rhs, shape = _broadcast_indices(x, wg, lhs_indices, rhs_indices)
    n_idx = math.prod(shape)
    x_batch = x.numel() // (M * K) if M * K else 0
    n_exp = wg.numel() // (N * wg.shape[-1]) if N * wg.shape[-1] else 0
    y = torch.empty(tuple(shape) + (M, N), dtype=x.dtype, device=x.device)
    check(lib().mi_gather_qmm_gate_up_swiglu(
        _ptr(y), _ptr(x), _ptr(wg), _ptr(sg), _ptr(bg), _ptr(wu), _ptr(su), _ptr(bu), _ptr(lhs),
        _ptr(rhs), n_idx, lhs_div, x_batch, M, N, K, n_exp, bool(transpose), opt(gs), opt(nb),
        mode.encode() if mode else None, bool(sorted_indices), _dtype_code(x, "x"),
        _dtype_code(sg, "scales"), _stream(x)))
    return y


def dequantize(w, scales, biases, group_size=None, bits=None, mode="affine", dtype=None,
               rounding=None, global_scale=None):
    """mlx_dequantize (src/mlx.zig:271). dtype defaults to the scales dtype.
    rounding (bf16 output only): None/1 = op-by-op bf16, 0 = single rounding.
    global_scale: nvfp4 only, a one-element fp32 device tensor."""
    _contig(w, scales, biases, global_scale)
    K = w.shape[-1] * 32 // (_defaults(mode)[1] if bits is None else int(bits))
    gs, nb = _resolve(_packed(w), scales, group_size, bits, K, mode)
    dtype = (torch.bfloat16 if scales.dtype == torch.uint8 else scales.dtype) if dtype is None else dtype
    rows = w.numel() // w.shape[-1] if w.shape[-1] else 0
    out = torch.empty(tuple(w.shape[:-1]) + (K,), dtype=dtype, device=w.device)
    check(lib().mi_dequantize_rounding(_ptr(out), _ptr(w), _ptr(scales), _ptr(biases), rows, K,
                                       opt(gs), opt(nb), mode.encode() if mode else None,
                                       _ptr(global_scale),
                                       _dtype_code(scales, "scales"), _dtype_code(out, "out"),
                                       1 if rounding is None else int(rounding), _stream(w)))
    return out


def quantize(w, group_size=None, bits=None, mode="affine"):
    """mlx_quantize (src/mlx.zig:275): returns (wq int32-bits, scales, biases)."""
    _contig(w)
    gs = 64 if group_size is None else int(group_size)
    nb = 4 if bits is None else int(bits)
    K = w.shape[-1]
    _require(K % gs == 0, f"K={K} not a multiple of group_size={gs}")
    rows = w.numel() // K if K else 0
    lead = tuple(w.shape[:-1])
    wq = torch.empty(lead + (K * nb // 32,), dtype=torch.int32, device=w.device)
    sdt = torch.bfloat16
    s = torch.empty(lead + (K // gs,), dtype=sdt, device=w.device)
    b = torch.empty(lead + (K // gs,), dtype=sdt, device=w.device)
    check(lib().mi_quantize(_ptr(wq), _ptr(s), _ptr(b), _ptr(w), rows, K, opt(gs), opt(nb),
                            mode.encode() if mode else None, None, _dtype_code(w, "w"),
                            _stream(w)))
    return wq, s, b


def fill_randn(t, seed, mean=0.0, std=1.0):
    """Fill a bf16/f32 device tensor from the library's counter-based normal stream."""
    _contig(t)
    check(lib().mi_fill_randn(_ptr(t), t.numel(), int(seed) & ((1 << 64) - 1), float(mean),
                              float(std), _dtype_code(t, "t"), _stream(t)))
    return t


def affine_params_from_geometry(w_cols, s_cols, in_dim):
    """(bits, group_size) from packed geometry, or None (src/transformer.zig:16763)."""
    b, g = ctypes.c_int(0), ctypes.c_int(0)
    rc = lib().mi_affine_params_from_geometry(int(w_cols), int(s_cols), int(in_dim),
                                              ctypes.byref(b), ctypes.byref(g))
    return None if rc != 0 else (b.value, g.value)


# ---------------------------------------------------------------- MoE glue --
def moe_route_topk(logits, k, scores_dtype=torch.float32):
    """Softmax top-k routing (moeRoutingChain, src/transformer.zig:17022-17072).
    logits fp32 [..., E] -> (inds uint32-as-int32 [..., k], scores [..., k])."""
    _contig(logits)
    _require(logits.dtype == torch.float32, "logits must be float32")
    E = logits.shape[-1]
    T = logits.numel() // E if E else 0
    inds = torch.empty(logits.shape[:-1] + (k,), dtype=torch.int32, device=logits.device)
    scores = torch.empty(logits.shape[:-1] + (k,), dtype=scores_dtype, device=logits.device)
    check(lib().mi_moe_route_topk(_ptr(inds), _ptr(scores), _ptr(logits), T, E, int(k),
                                  _dtype_code(scores, "scores"), _stream(logits)))
    return inds, scores


def moe_route_grouped(logits, bias, k, n_group, topk_group, route_norm=True, route_scale=1.0):
    """Group-limited sigmoid routing (groupLimitedRouting, src/transformer.zig:17242-17347):
    logits fp32 [..., E], bias fp32 [E] -> (inds int32 [..., k], weights fp32 [..., k])."""
    _contig(logits, bias)
    _require(logits.dtype == torch.float32 and bias.dtype == torch.float32, "fp32 inputs")
    E = logits.shape[-1]
    T = logits.numel() // E if E else 0
    inds = torch.empty(logits.shape[:-1] + (k,), dtype=torch.int32, device=logits.device)
    w = torch.empty(logits.shape[:-1] + (k,), dtype=torch.float32, device=logits.device)
    check(lib().mi_moe_route_grouped(_ptr(inds), _ptr(w), _ptr(logits), _ptr(bias), T, E, int(k),
                                     int(n_group), int(topk_group), bool(route_norm),
                                     float(route_scale), _stream(logits)))
    return inds, w


def moe_sort_dispatch(flat, k, n_experts):
    """Sorted MoE dispatch (src/transformer.zig:14965-14993): returns (order, inv, sorted,
    lhs, seg_offsets) with order = stable argsort(flat), inv = argsort(order),
    sorted = flat[order], lhs = order // k, seg_offsets [n_experts + 1]."""
    _contig(flat)
    flat = flat.reshape(-1)
    n = flat.numel()
    mk = lambda m: torch.empty(m, dtype=torch.int32, device=flat.device)  # noqa: E731
    order, inv, srt, lhs, seg = mk(n), mk(n), mk(n), mk(n), mk(n_experts + 1)
    check(lib().mi_moe_sort_dispatch(_ptr(order), _ptr(inv), _ptr(srt), _ptr(lhs), _ptr(seg),
                                     _ptr(flat), n, int(k), int(n_experts), _stream(flat)))
    return order, inv, srt, lhs, seg


def take_rows(x, indices):
    """x[indices] along axis 0 (mlx_take_axis 0 on row-major rows)."""
    _contig(x, indices)
    idx = indices.reshape(-1)
    out = torch.empty((idx.numel(),) + tuple(x.shape[1:]), dtype=x.dtype, device=x.device)
    row_bytes = x[0].numel() * x.element_size() if x.shape[0] else 0
    check(lib().mi_take_rows(_ptr(out), _ptr(x), _ptr(idx), idx.numel(), x.shape[0], row_bytes,
                             _stream(x)))
    return out


def swiglu(gate, up):
    """bf16(bf16(g * sigmoid(g)) * u) (fusedSwiGLU, src/transformer.zig:19846-19884)."""
    _contig(gate, up)
    _require(gate.shape == up.shape, "gate/up shapes differ")
    y = torch.empty_like(gate)
    check(lib().mi_swiglu(_ptr(y), _ptr(gate), _ptr(up), gate.numel(), _dtype_code(gate, "gate"),
                          _stream(gate)))
    return y


def moe_down_reduce(v, scores):
    """Score-weighted slot sum in bf16: v [T, k, N], scores [T, k] -> [T, N]."""
    _contig(v, scores)
    T, k, N = v.shape
    y = torch.empty((T, N), dtype=v.dtype, device=v.device)
    check(lib().mi_moe_down_reduce(_ptr(y), _ptr(v), _ptr(scores), T, k, N,
                                   _dtype_code(v, "v"), _stream(v)))
    return y


def moe_down_reduce_rows(v, rows, scores):
    """moe_down_reduce(take_rows(v, rows).view(T, k, N), scores) in one pass: v [R, N],
    rows [T*k] (the inverse permutation of the sorted dispatch), scores [T, k] -> [T, N]."""
    _contig(v, rows, scores)
    T, k = scores.shape
    N = v.shape[-1]
    _require(rows.numel() == T * k, "rows must hold T*k entries")
    y = torch.empty((T, N), dtype=v.dtype, device=v.device)
    check(lib().mi_moe_down_reduce_rows(_ptr(y), _ptr(v), _ptr(scores), _ptr(rows),
                                        v.numel() // N if N else 0, T, int(k), N,
                                        _dtype_code(v, "v"), _stream(v)))
    return y


def gather_qmv_gate_up_swiglu(x, wg, sg, bg, wu, su, bu, inds, group_size=None, bits=None,
                              mode="affine"):
    """gatherQmvGateUp (src/transformer.zig:20303-20396): x [T, K], inds [T, k] ->
    [T, k, N] = swiglu(x @ Wg[e]^T, x @ Wu[e]^T), each product rounded to bf16 first."""
    _contig(x, wg, sg, bg, wu, su, bu, inds)
    T, K = x.shape
    k = inds.shape[-1]
    gs, nb = _resolve(_packed(wg), sg, group_size, bits, K, mode)
    E, N = wg.shape[0], wg.shape[1]
    y = torch.empty((T, k, N), dtype=x.dtype, device=x.device)
    check(lib().mi_gather_qmv_gate_up_swiglu(_ptr(y), _ptr(x), _ptr(wg), _ptr(sg), _ptr(bg),
                                             _ptr(wu), _ptr(su), _ptr(bu), _ptr(inds), T, k, N,
                                             K, E, opt(gs), opt(nb),
                                             mode.encode() if mode else None, _stream(x)))
    return y


def moe_route_gate_up_swiglu(logits, x, wg, sg, bg, wu, su, bu, k, group_size=None, bits=None,
                             mode="affine"):
    """Routing + gatherQmvGateUp in one call (src/transformer.zig:17748, :20303-20396):
    logits fp32 [T, E], x [T, K] -> (y [T, k, N], inds [T, k], bf16 scores [T, k])."""
    _contig(logits, x, wg, sg, bg, wu, su, bu)
    _require(logits.dtype == torch.float32, "logits must be float32")
    T, K = x.shape
    E = logits.shape[-1]
    gs, nb = _resolve(_packed(wg), sg, group_size, bits, K, mode)
    N = wg.shape[1]
    y = torch.empty((T, k, N), dtype=x.dtype, device=x.device)
    inds = torch.empty((T, k), dtype=torch.int32, device=x.device)
    scores = torch.empty((T, k), dtype=torch.bfloat16, device=x.device)
    check(lib().mi_moe_route_gate_up_swiglu(_ptr(y), _ptr(inds), _ptr(scores), _ptr(logits),
                                            _ptr(x), _ptr(wg), _ptr(sg), _ptr(bg), _ptr(wu),
                                            _ptr(su), _ptr(bu), T, E, int(k), N, K, opt(gs),
                                            opt(nb), mode.encode() if mode else None,
                                            _dtype_code(scores, "scores"), _stream(x)))
    return y, inds, scores


def gather_qmv_down_reduce(act, wd, sd, bd, inds, scores, group_size=None, bits=None,
                           mode="affine"):
    """gatherQmvDownReduce (src/transformer.zig:20675-20761): act [T, k, K], inds/scores
    [T, k] -> [T, N]."""
    _contig(act, wd, sd, bd, inds, scores)
    T, k, K = act.shape
    gs, nb = _resolve(_packed(wd), sd, group_size, bits, K, mode)
    E, N = wd.shape[0], wd.shape[1]
    y = torch.empty((T, N), dtype=act.dtype, device=act.device)
    check(lib().mi_gather_qmv_down_reduce(_ptr(y), _ptr(act), _ptr(wd), _ptr(sd), _ptr(bd),
                                          _ptr(inds), _ptr(scores), T, k, N, K, E, opt(gs),
                                          opt(nb), mode.encode() if mode else None, _stream(act)))
    return y


def library_gemm_calls():
    """GEMMs this process has run through the vendor library (hipBLASLt); every default
    route uses this project's kernels, so it stays 0 unless MI_QMM_DQGEMM=1."""
    return int(lib().mi_library_gemm_calls())


def workspace_release(device=None):
    """Free the workspace generations that graphs captured earlier kept alive
    (mi_workspace_release). Call it once no such graph will be replayed again."""
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else device
    check(lib().mi_workspace_release(ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)))


def workspace_reserve(nbytes, device=None):
    """Grow the library's per-device workspace ahead of HIP graph capture."""
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else device
    check(lib().mi_workspace_reserve(int(nbytes),
                                     ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)))
