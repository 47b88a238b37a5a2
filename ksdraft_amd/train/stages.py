"""PTQR rounding-dither quantization (reference ksdraft/train/stages.py:27-50).

Only the kernel-facing helper lives here; the stage/loss logic of the reference module
is outside the INT8 hot path."""

from ..kernels.quant import quantize_last_dim_dithered

__all__ = ["quantize_last_dim_dithered"]
