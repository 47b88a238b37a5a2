"""INT8 tier on MI355X: GS128 W8A8 kernels behind the reference's ksdraft.kernels API
(reference ksdraft/kernels/__init__.py:7-14)."""

from .quant import GROUP_SIZE, SCALE_DTYPE, quantize_last_dim, dequantize_last_dim
from .linear import Int8Linear

__all__ = [
    "GROUP_SIZE", "SCALE_DTYPE",
    "quantize_last_dim", "dequantize_last_dim",
    "Int8Linear",
]
