"""``project_fused`` under the reference's module name (ksdraft/kernels/ks3_triton.py).

The reference's Triton kernel fuses the down-projection GEMM, the Horner spine, ReLU^2 and
the per-group requantization (ks3_triton.py:100-156). Here the GEMM is ksd_w8a8_gemm_nt
(fp32 accumulator out) and the spine + requantization follow the fused kernel's own
arithmetic contract, not the composed one: 'int8' (NL == 2) is ksd_ks3_spine_fused (fp32
coordinates and LUT index, no truncation, group pre-scale, second requantization); 'fp16'
and 'fp32' (NL == 1, 0; ks3_triton.py:76-98) are ksd_ks3_spine_float on the accumulator
(the coordinates not rounded to fp16, the warp scalars in fp16), every fp16/fp32 op of
the Triton source rounded separately.
"""

from __future__ import annotations

import torch

from .gemm import w8a8_gemm
from .ks3_int8 import spine_float, spine_fused_int8

FP16 = torch.float16
TANH_DOMAIN = 3.2


def project_fused(
    a_codes: torch.Tensor, a_scales: torch.Tensor,
    w_codes: torch.Tensor, w_scales: torch.Tensor,
    spine_codes: torch.Tensor, spine_scale: torch.Tensor,
    warp_scale: torch.Tensor, warp_shift: torch.Tensor,
    tanh_lut: torch.Tensor,
    group: int, nonlinear: str,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Input projection + Horner spine + requant (ks3_triton.py:159-195).

    warp_scale/warp_shift: dequantized fp16 per-chart scalars. Returns
    (h_codes int8 (M, N), h_scales fp16 (M, ceil(N/group)))."""
    if group & (group - 1):
        raise ValueError("group must be a power of two (32 or 128)")
    nl = {"fp32": 0, "fp16": 1, "int8": 2}[nonlinear]
    acc = w8a8_gemm(a_codes, a_scales, w_codes, w_scales, group)
    if nl == 2:
        return spine_fused_int8(acc, spine_codes, spine_scale, warp_scale.to(FP16),
                                warp_shift.to(FP16), tanh_lut, group)
    _, hq, hs = spine_float(acc, spine_codes, spine_scale, warp_scale.to(FP16).float(),
                            warp_shift.to(FP16).float(), nonlinear, group)
    return hq, hs
