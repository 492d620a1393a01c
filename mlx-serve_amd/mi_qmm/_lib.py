"""Loads libmi_qmm.so (built in-tree by mlx-serve_amd/build.py) and declares its C ABI
(include/mi_qmm.h). Fails loudly when the library is missing: there is no CPU path."""
import ctypes
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libmi_qmm.so")

MI_OK, MI_ERR_UNSUPPORTED, MI_ERR_INVALID, MI_ERR_HIP = 0, 1, 2, 3
DT_UINT8, DT_UINT32, DT_FLOAT16, DT_FLOAT32, DT_BFLOAT16 = 1, 3, 9, 10, 12


class MiError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"mi_qmm error {code}: {msg}")
        self.code = code


class MiUnsupported(MiError):
    """The library declines the call (the reference's 'return null, use fallback')."""


class OptInt(ctypes.Structure):
    _fields_ = [("value", ctypes.c_int), ("has_value", ctypes.c_bool)]


def opt(v):
    return OptInt(0, False) if v is None else OptInt(int(v), True)


_lib = None


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is missing: run mlx-serve_amd/build.py "
                          "(or __graft_entry__.build()) first")
    L = ctypes.CDLL(LIB_PATH)
    P, i64, i32, b = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_bool
    s = ctypes.c_char_p
    L.mi_quantized_matmul.argtypes = [P, P, P, P, P, i64, i64, i64, b, OptInt, OptInt, s, i32,
                                      i32, P]
    L.mi_gather_qmm.argtypes = [P, P, P, P, P, P, P, i64, i64, i64, i64, i64, i64, i64, b,
                                OptInt, OptInt, s, b, i32, i32, P]
    L.mi_dequantize.argtypes = [P, P, P, P, i64, i64, OptInt, OptInt, s, P, i32, i32, P]
    L.mi_dequantize_rounding.argtypes = [P, P, P, P, i64, i64, OptInt, OptInt, s, P, i32, i32,
                                         i32, P]
    L.mi_quantize.argtypes = [P, P, P, P, i64, i64, OptInt, OptInt, s, P, i32, P]
    L.mi_affine_params_from_geometry.argtypes = [i64, i64, i64, ctypes.POINTER(i32),
                                                 ctypes.POINTER(i32)]
    L.mi_fill_randn.argtypes = [P, i64, ctypes.c_uint64, ctypes.c_float, ctypes.c_float, i32, P]
    L.mi_moe_route_topk.argtypes = [P, P, P, i64, i64, i32, i32, P]
    L.mi_moe_sort_dispatch.argtypes = [P, P, P, P, P, P, i64, i32, i64, P]
    L.mi_take_rows.argtypes = [P, P, P, i64, i64, i64, P]
    L.mi_swiglu.argtypes = [P, P, P, i64, i32, P]
    L.mi_moe_down_reduce.argtypes = [P, P, P, i64, i32, i64, i32, P]
    L.mi_gather_qmv_gate_up_swiglu.argtypes = [P, P, P, P, P, P, P, P, P, i64, i32, i64, i64,
                                               i64, OptInt, OptInt, s, P]
    L.mi_gather_qmv_down_reduce.argtypes = [P, P, P, P, P, P, P, i64, i32, i64, i64, i64, OptInt,
                                            OptInt, s, P]
    L.mi_gather_qmm_noalloc.argtypes = L.mi_gather_qmm.argtypes
    L.mi_gather_qmm_swiglu.argtypes = [P] + L.mi_gather_qmm.argtypes
    L.mi_gather_qmm_gate_up_swiglu.argtypes = (L.mi_gather_qmm.argtypes[:5] + [P, P, P] +
                                                L.mi_gather_qmm.argtypes[5:])
    L.mi_moe_down_reduce_rows.argtypes = [P, P, P, P, i64, i64, i32, i64, i32, P]
    L.mi_moe_route_grouped.argtypes = [P, P, P, P, i64, i64, i32, i32, i32, b, ctypes.c_float, P]
    L.mi_moe_route_gate_up_swiglu.argtypes = [P, P, P, P, P, P, P, P, P, P, P, i64, i64, i32,
                                              i64, i64, OptInt, OptInt, s, i32, P]
    L.mi_workspace_reserve.argtypes = [i64, P]
    L.mi_workspace_release.argtypes = [P]
    L.mi_library_gemm_calls.argtypes = []
    L.mi_library_gemm_calls.restype = ctypes.c_int64
    L.mi_last_error.restype = ctypes.c_char_p
    PP = ctypes.POINTER(P)
    L.mi_ckpt_open.argtypes = [s, i32, PP]
    L.mi_ckpt_open_file.argtypes = [s, PP]
    L.mi_ckpt_close.argtypes = [P]
    L.mi_ckpt_close.restype = None
    L.mi_parse_quant_config.argtypes = [s, ctypes.c_size_t, P]
    L.mi_ckpt_quant_config.argtypes = [P, P]
    L.mi_ckpt_set_quant_config.argtypes = [P, P]
    L.mi_ckpt_count.argtypes = [P]
    L.mi_ckpt_count.restype = i64
    L.mi_ckpt_name.argtypes = [P, i64]
    L.mi_ckpt_name.restype = ctypes.c_char_p
    L.mi_ckpt_info.argtypes = [P, s, P]
    L.mi_ckpt_read.argtypes = [P, s, P, ctypes.c_size_t]
    L.mi_ckpt_upload.argtypes = [P, s, P, ctypes.c_size_t]
    L.mi_ckpt_linear.argtypes = [P, s, i64, P]
    L.mi_version.restype = ctypes.c_char_p
    for name in EXTRA_SIGNATURES:
        if hasattr(L, name):
            getattr(L, name).argtypes = EXTRA_SIGNATURES[name]
    _lib = L
    return L


# Entry points added by later modules register their argtypes here.
EXTRA_SIGNATURES = {}


def last_error():
    return lib().mi_last_error().decode()


def check(rc):
    if rc == MI_OK:
        return
    msg = last_error()
    if rc == MI_ERR_UNSUPPORTED:
        raise MiUnsupported(rc, msg)
    raise MiError(rc, msg)
