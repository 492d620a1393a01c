"""Quantized-checkpoint loader (include/mi_ckpt.h) on the Python side.

Opens an MLX model directory the way the reference's loadWeights does
(src/model.zig:2946-3146), with the model-wide "quantization" declaration of
parseConfig (src/model.zig:1480-1505), and hands out the tensors of one quantized
linear layer ("{prefix}.weight/.scales/.biases", src/transformer.zig:21068-21153)
with the (bits, group_size, mode) computeQuantParams resolves for it
(src/transformer.zig:16876-16924). Reading goes to host tensors; upload() copies
straight into device buffers that mi_quantized_matmul / mi_gather_qmm then read.
"""
import ctypes

import torch

from ._lib import check, lib, MiError, MI_ERR_INVALID

MODES = ("affine", "nvfp4", "mxfp4", "mxfp8")
_MAX_DIMS = 8

# mlx_dtype codes (src/mlx.zig:20-35) -> torch dtypes for the tensors a checkpoint holds.
_TORCH_DTYPE = {
    0: torch.bool, 1: torch.uint8, 2: torch.uint16, 3: torch.uint32, 4: torch.uint64,
    5: torch.int8, 6: torch.int16, 7: torch.int32, 8: torch.int64, 9: torch.float16,
    10: torch.float32, 11: torch.float64, 12: torch.bfloat16, 13: torch.complex64,
}


class QuantConfig(ctypes.Structure):
    _fields_ = [("bits", ctypes.c_int), ("group_size", ctypes.c_int), ("mode", ctypes.c_int)]

    def as_tuple(self):
        return self.bits, self.group_size, MODES[self.mode]


class TensorInfo(ctypes.Structure):
    _fields_ = [("dtype", ctypes.c_int), ("ndim", ctypes.c_int),
                ("shape", ctypes.c_int64 * _MAX_DIMS), ("nbytes", ctypes.c_int64)]


class LinearDesc(ctypes.Structure):
    _fields_ = [("has_scales", ctypes.c_int), ("has_biases", ctypes.c_int),
                ("bits", ctypes.c_int), ("group_size", ctypes.c_int), ("mode", ctypes.c_int),
                ("out_dim", ctypes.c_int64), ("in_dim", ctypes.c_int64)]


def parse_quant_config(text):
    """(bits, group_size, mode) from a config.json text; bits 0 = dense."""
    raw = text.encode() if isinstance(text, str) else bytes(text)
    q = QuantConfig()
    check(lib().mi_parse_quant_config(raw, len(raw), ctypes.byref(q)))
    return q.as_tuple()


class Checkpoint:
    """One opened checkpoint; close() (or a with-block) unmaps its files."""

    def __init__(self, path, load_vision=False, single_file=False):
        L = lib()
        h = ctypes.c_void_p()
        if single_file:
            check(L.mi_ckpt_open_file(str(path).encode(), ctypes.byref(h)))
        else:
            check(L.mi_ckpt_open(str(path).encode(), int(bool(load_vision)), ctypes.byref(h)))
        self._h = h

    def close(self):
        if self._h:
            lib().mi_ckpt_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def quant_config(self):
        q = QuantConfig()
        check(lib().mi_ckpt_quant_config(self._h, ctypes.byref(q)))
        return q.as_tuple()

    def set_quant_config(self, bits, group_size, mode="affine"):
        q = QuantConfig(int(bits), int(group_size), MODES.index(mode))
        check(lib().mi_ckpt_set_quant_config(self._h, ctypes.byref(q)))

    def names(self):
        L = lib()
        return [L.mi_ckpt_name(self._h, i).decode() for i in range(L.mi_ckpt_count(self._h))]

    def info(self, name):
        t = TensorInfo()
        check(lib().mi_ckpt_info(self._h, name.encode(), ctypes.byref(t)))
        return _TORCH_DTYPE[t.dtype], tuple(t.shape[:t.ndim]), t.nbytes

    def __contains__(self, name):
        try:
            self.info(name)
            return True
        except MiError as e:
            if e.code != MI_ERR_INVALID:
                raise
            return False

    def read(self, name):
        """The tensor as a new host torch tensor (f16 side tensors narrowed to bf16)."""
        dt, shape, nbytes = self.info(name)
        out = torch.empty(shape, dtype=dt)
        check(lib().mi_ckpt_read(self._h, name.encode(), ctypes.c_void_p(out.data_ptr()),
                                 nbytes))
        return out

    def upload(self, name, device="cuda"):
        """The tensor copied into a new device tensor (synchronous)."""
        dt, shape, nbytes = self.info(name)
        out = torch.empty(shape, dtype=dt, device=device)
        check(lib().mi_ckpt_upload(self._h, name.encode(), ctypes.c_void_p(out.data_ptr()),
                                   nbytes))
        return out

    def linear(self, prefix, in_dim=0):
        """dict(bits, group_size, mode, has_scales, has_biases, out_dim, in_dim)."""
        d = LinearDesc()
        check(lib().mi_ckpt_linear(self._h, prefix.encode(), int(in_dim), ctypes.byref(d)))
        return dict(bits=d.bits, group_size=d.group_size, mode=MODES[d.mode],
                    has_scales=bool(d.has_scales), has_biases=bool(d.has_biases),
                    out_dim=d.out_dim, in_dim=d.in_dim)

    def load_linear(self, prefix, in_dim=0, device=None):
        """The layer's tensors (weight, scales, biases; absent ones None) plus its params,
        on `device` (host tensors when None)."""
        d = self.linear(prefix, in_dim)
        get = self.read if device is None else (lambda n: self.upload(n, device))
        w = get(prefix + ".weight")
        s = get(prefix + ".scales") if d["has_scales"] else None
        b = get(prefix + ".biases") if d["has_biases"] else None
        return w, s, b, d
