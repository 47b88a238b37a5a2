"""ksdraft_amd — MI355X (gfx950) kernels for KSDraft's INT8 tier.

``ksdraft_amd.kernels`` mirrors the reference's ``ksdraft.kernels`` API (W8A8 GS128
GEMMs, quantization, Int8Linear, the KS3 int8 cell and the Rosa mixer step); the compute
runs in hand-written HIP kernels of ``libksdraft_amd.so`` loaded through ctypes.
"""

__version__ = "0.1.0"
