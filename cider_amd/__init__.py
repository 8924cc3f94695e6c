"""cider_amd - cider's fused quantize -> int8 GEMM -> dequant linear on MI355X.

Public surface of the reference package (``cider/__init__.py:18-57``):
``convert_model``, ``CiderLinear``/``W8A8Linear``, ``W4A8Linear``,
``perchannel_linear``, ``pergroup_linear``, ``w4a8_linear``,
``int8_matmul_int32``, ``quantize_weight_int8``, ``pack_weight_int4``,
``is_available``, ``kernel_dir``, ``set_mode``/``get_mode``.

Unlike the reference there are no silent no-op stubs: every entry point that
needs the HIP extension raises ``RuntimeError`` when it is missing.
"""

__version__ = "0.1.0"

from .convert import convert_model
from .nn import CiderLinear, W4A8GroupLinear, W4A8Linear, W8A8Linear, get_mode, set_mode
from .ops import (
    int8_matmul_int32,
    is_available,
    kernel_dir,
    pack_weight_int4,
    pack_weight_int4_pergroup,
    perchannel_gemm,
    perchannel_linear,
    pergroup_linear,
    quantize_per_token,
    quantize_weight_int8,
    quantize_weight_pergroup,
    repack_w4_ref,
    w4a8_linear,
    w4a8_linear_packed,
    w4a8_pergroup_linear,
)

__all__ = [
    "convert_model",
    "set_mode",
    "get_mode",
    "CiderLinear",
    "W8A8Linear",
    "W4A8Linear",
    "W4A8GroupLinear",
    "perchannel_linear",
    "perchannel_gemm",
    "w4a8_linear",
    "w4a8_linear_packed",
    "w4a8_pergroup_linear",
    "pergroup_linear",
    "int8_matmul_int32",
    "quantize_per_token",
    "quantize_weight_int8",
    "quantize_weight_pergroup",
    "pack_weight_int4",
    "pack_weight_int4_pergroup",
    "repack_w4_ref",
    "is_available",
    "kernel_dir",
]
