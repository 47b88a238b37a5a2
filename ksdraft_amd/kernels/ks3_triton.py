"""``project_fused`` under the reference's module name (ksdraft/kernels/ks3_triton.py).

The reference's Triton kernel fuses the down-projection GEMM, the Horner spine, ReLU^2 and
the per-group requantization (ks3_triton.py:100-156), following the fused kernel's own
arithmetic contract, not the composed one.

* 'int8' (NL == 2) with group 128, up to ONE_LAUNCH_MAX_ROWS rows (the eval path's
  decode and short-prefill shapes): the reference's single-kernel form,
  ksd_ks3_project_fused, a GEMM whose epilogue runs the fused contract (fp32 coordinates
  and LUT index, no truncation, group pre-scale, second requantization) on each finished
  fp32 accumulator tile and stores only the h codes and scales, after a small kernel has
  tabulated the per-chart increments. Its accumulator is the unsplit ordered sum over all
  K groups, so it is taken only where the standalone GEMM would not split K either: the
  outputs are then identical to the two-launch form's. At d 1536, F 5888 on MI355X it
  takes about 29 us against 49-53 us for M <= 256 and 53 against 58 us at M = 1024.
* 'int8' otherwise: ksd_w8a8_gemm_nt (fp32 accumulator out), then ksd_ks3_spine_fused,
  the same per-element arithmetic with the per-chart table staged in LDS per 128-chart
  segment. At M >= 2048 this is the faster form (223 against 254 us at M 8192): in one
  launch the table (128 KB per 128-chart tile) cannot sit in LDS beside the GEMM's
  132 KB operand ring, so the epilogue gathers it from L2, and the spine's VALU work runs
  between the MFMA steps instead of beside them. ``one_launch`` forces either form.
* 'fp16' and 'fp32' (NL == 1, 0; ks3_triton.py:76-98): ksd_ks3_spine_float on the
  accumulator (the coordinates not rounded to fp16, the warp scalars in fp16), every
  fp16/fp32 op of the Triton source rounded separately.
"""

from __future__ import annotations

import torch

from .. import _lib
from .gemm import _prepare, gemm_splits, w8a8_gemm
from .ks3_int8 import spine_float, spine_fused_int8

FP16 = torch.float16
TANH_DOMAIN = 3.2


def project_fused(
    a_codes: torch.Tensor, a_scales: torch.Tensor,
    w_codes: torch.Tensor, w_scales: torch.Tensor,
    spine_codes: torch.Tensor, spine_scale: torch.Tensor,
    warp_scale: torch.Tensor, warp_shift: torch.Tensor,
    tanh_lut: torch.Tensor,
    group: int, nonlinear: str, *, one_launch: bool | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Input projection + Horner spine + requant (ks3_triton.py:159-195).

    warp_scale/warp_shift: dequantized fp16 per-chart scalars. one_launch: None picks the
    form by shape (see above); True forces the single launch ('int8', group 128 only),
    False the two launches. Returns (h_codes int8 (M, N), h_scales fp16 (M, ceil(N/group)))."""
    if group & (group - 1):
        raise ValueError("group must be a power of two (32 or 128)")
    nl = {"fp32": 0, "fp16": 1, "int8": 2}[nonlinear]
    if one_launch and (nl != 2 or group != 128):
        raise ValueError("one_launch: 'int8' with group 128 only")
    if one_launch is None:
        one_launch = nl == 2 and group == 128 and _one_launch_pays(a_codes, w_codes)
    if one_launch:
        out = _project_fused_int8(a_codes, a_scales, w_codes, w_scales, spine_codes, spine_scale,
                                  warp_scale.to(FP16), warp_shift.to(FP16), tanh_lut)
        if out is not None:
            return out
    acc = w8a8_gemm(a_codes, a_scales, w_codes, w_scales, group)
    if nl == 2:
        return spine_fused_int8(acc, spine_codes, spine_scale, warp_scale.to(FP16),
                                warp_shift.to(FP16), tanh_lut, group)
    _, hq, hs = spine_float(acc, spine_codes, spine_scale, warp_scale.to(FP16).float(),
                            warp_shift.to(FP16).float(), nonlinear, group)
    return hq, hs


# Largest M for which project_fused takes the single launch by default (measured on MI355X
# at d 1536, F 5888: 29 against 49-53 us up to M 256, 53 against 58 us at M 1024, 75
# against 69 us at M 2048).
ONE_LAUNCH_MAX_ROWS = 1024


def _one_launch_pays(a_codes: torch.Tensor, w_codes: torch.Tensor) -> bool:
    """Few rows, and a GEMM shape the standalone launch would not split along K (so both
    forms compute the same ordered accumulator)."""
    if a_codes.dim() != 2 or w_codes.dim() != 2:
        return False
    M, K = a_codes.shape
    N = w_codes.shape[0]
    K128 = -(-K // 128) * 128
    return 0 < M <= ONE_LAUNCH_MAX_ROWS and N > 0 and K128 > 0 and gemm_splits(M, N, K128) == 1


def _project_fused_int8(a_codes, a_scales, w_codes, w_scales, spine_codes, spine_scale,
                        warp_scale16, warp_shift16, tanh_lut):
    """GEMM + spine + requantization in one launch (group 128, 'int8'); None for K = 0,
    which the two-launch path covers (its GEMM returns zeros)."""
    dev, M, N, K, a, as_, w, ws = _prepare(a_codes, a_scales, w_codes, w_scales, 128)
    if K == 0:
        return None
    dev = _lib.require_gpu(spine_codes, spine_scale, warp_scale16, warp_shift16, tanh_lut)
    if spine_codes.numel() != 6 * N or spine_scale.numel() != N:
        raise ValueError(f"spine buffers do not match {N} charts")
    if warp_scale16.numel() != N or warp_shift16.numel() != N:
        raise ValueError(f"warp scalars do not match {N} charts")
    if tanh_lut.numel() != 256:
        raise ValueError("tanh_lut must have 256 entries")
    hq = torch.empty((M, N), dtype=torch.int8, device=dev)
    hs = torch.empty((M, -(-N // 128)), dtype=FP16, device=dev)
    if M == 0 or N == 0:
        return hq, hs
    table = torch.empty((N, 256), dtype=torch.float32, device=dev)
    sc, ps = spine_codes.reshape(N, 6).contiguous(), spine_scale.reshape(N).contiguous()
    wsc, wsh = warp_scale16.reshape(N).contiguous(), warp_shift16.reshape(N).contiguous()
    lut = tanh_lut.contiguous()
    _lib.call("ksd_ks3_project_fused", a.data_ptr(), as_.data_ptr(), w.data_ptr(), ws.data_ptr(),
              M, N, K, sc.data_ptr(), ps.data_ptr(), wsc.data_ptr(), wsh.data_ptr(),
              lut.data_ptr(), 128, hq.data_ptr(), hs.data_ptr(), table.data_ptr(),
              _lib.stream_ptr(dev))
    return hq, hs
