"""mi_qmm -- MI355X (gfx950) affine quantized matmul, Python host side.

Mirrors the mlx-c calls that ddalcu/mlx-serve makes through src/mlx.zig
(mlx_quantized_matmul, mlx_gather_qmm, mlx_dequantize, mlx_quantize) on torch
device tensors, and the reference's MoE dispatch around them (src/transformer.zig
moeMLP2). Every call goes to libmi_qmm.so; there is no fallback path.
"""
from ._lib import MiError, MiUnsupported, lib, last_error, LIB_PATH  # noqa: F401
from .ops import (quantized_matmul, gather_qmm, dequantize, quantize, fill_randn,  # noqa: F401
                  affine_params_from_geometry, moe_route_topk, moe_sort_dispatch, take_rows,
                  swiglu, moe_down_reduce, moe_down_reduce_rows, gather_qmm_swiglu,
                  gather_qmm_gate_up_swiglu,
                  gather_qmv_gate_up_swiglu, gather_qmv_down_reduce, workspace_reserve,
                  workspace_release, library_gemm_calls,
                  moe_route_gate_up_swiglu, moe_route_grouped)
from .ckpt import Checkpoint, parse_quant_config  # noqa: F401
