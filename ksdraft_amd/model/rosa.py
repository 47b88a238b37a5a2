"""RWKV-8 Rosa hard-retrieval mixer on gfx950 (mirror of reference ksdraft/model/rosa.py).

Same module surface: ``_match_payload_sign`` and ``RosaMixer`` (parameters, init,
``_shifted``, ``forward``). The match runs in ksd_rosa_match (bit-sliced longest-suffix
search, any T up to 65536; the reference's own form needs O(T^2) int64 tensors per
length); training on the GPU goes through ``HardRosaGPU`` (exact counterfactual credits).
With Int8Linear projections (``to_int8`` surfaces) the time shift and the three input
quantizations are one kernel: ksd_rosa_shift_quant in eval, and in training
ksd_rosa_shift_quant_dual (each input's row codes and dW's transposed operand) with
ksd_rosa_shift_backward for the shift's gradient (ShiftedInt8Projections); the shifted
inputs are never materialised.
"""

from __future__ import annotations

import torch
from torch import nn
from torch.nn import functional as F

from ..kernels import rosa as R


def _match_payload_sign(qbits: torch.Tensor, kbits: torch.Tensor, vbits: torch.Tensor,
                        max_match_len: int | None = None) -> torch.Tensor:
    """rosa.py:40-98. qbits/kbits/vbits (..., T) in {0, 1} on the GPU -> (..., T) float32
    in {+1, -1}: the successor-value sign at the latest longest-match endpoint, -1 when
    nothing matches."""
    *lead, T = qbits.shape
    n = 1
    for s in lead:
        n *= s
    packed = [R.pack_bits(b.reshape(n, T, 1).to(torch.float16)) for b in (qbits, kbits, vbits)]
    sign, _ = R.match_packed(*(p.reshape(n, -1) for p in packed), T, max_match_len)
    return sign.reshape(*lead, T).float()


class RosaMixer(nn.Module):
    """rosa.py:101-165."""

    # training with Int8Linear q/k/v: shift + dual quantization fused (False: torch's
    # _shifted, then each Int8Linear quantizes its own input)
    fused_shift = True

    def __init__(self, d_model: int, streams: int = 512, bits: int = 1):
        super().__init__()
        if bits != 1:
            raise NotImplementedError(
                "reference implements 1-bit streams (the decided configuration); "
                "n-bit packed symbols arrive with the production kernel")
        self.d_model = d_model
        self.streams = streams
        self.bits = bits
        self.q_proj = nn.Linear(d_model, streams, bias=True)
        self.k_proj = nn.Linear(d_model, streams, bias=True)
        self.v_proj = nn.Linear(d_model, streams, bias=True)
        self.out_proj = nn.Linear(streams, d_model, bias=True)
        self.time_mix_q = nn.Parameter(torch.zeros(d_model))
        self.time_mix_k = nn.Parameter(torch.zeros(d_model))
        self.time_mix_v = nn.Parameter(torch.zeros(d_model))
        self.payload = nn.Parameter(torch.ones(streams))
        nn.init.zeros_(self.out_proj.weight)
        nn.init.zeros_(self.out_proj.bias)

    def extra_repr(self) -> str:
        return f"d_model={self.d_model}, streams={self.streams}, bits={self.bits}"

    def _shifted(self, x: torch.Tensor):
        prev = F.pad(x, (0, 0, 1, 0))[:, :-1, :]
        q_in = prev + (x - prev) * torch.sigmoid(self.time_mix_q)
        k_in = prev + (x - prev) * torch.sigmoid(self.time_mix_k)
        v_in = prev + (x - prev) * torch.sigmoid(self.time_mix_v)
        return q_in, k_in, v_in

    def _int8_projections(self) -> bool:
        from ..kernels.linear import Int8Linear
        return all(isinstance(getattr(self, n), Int8Linear) for n in ("q_proj", "k_proj", "v_proj"))

    def _fused_training_projections(self, x: torch.Tensor):
        """Training with Int8Linear q/k/v: ShiftedInt8Projections, or None when its
        preconditions fail (then the composed path runs)."""
        from ..kernels.linear import Int8Linear
        projs = (self.q_proj, self.k_proj, self.v_proj)
        mixes = (self.time_mix_q, self.time_mix_k, self.time_mix_v)
        if not (self.fused_shift and self._int8_projections()
                and x.dtype in (torch.float32, torch.bfloat16, torch.float16)
                and x.shape[-1] % 8 == 0 and all(m.dtype == torch.float32 for m in mixes)
                and not any(p.ste_training for p in projs)):
            return None
        x = x.contiguous()
        if x.data_ptr() % 16:
            return None
        args = []
        for p in projs:
            assert isinstance(p, Int8Linear)
            if not p._codes_current():  # as Int8Linear.forward: live masters stay authoritative
                p._codes_key = None
                p._quantize_weight()
            args += [p.weight, p.bias, p.weight_codes, p.weight_scales]
        sig = [torch.sigmoid(m) for m in mixes]
        return R.ShiftedInt8Projections.apply(x, *sig, *args,
                                              tuple(p.current_transpose() for p in projs))

    def _fused_projections(self, x: torch.Tensor):
        """Eval with Int8Linear q/k/v: shift + quantize in one pass, then the W8A8 GEMMs
        (+ bias) exactly as Int8Linear.forward computes them (linear.py:62-73)."""
        from ..kernels.gemm import w8a8_gemm_out
        sig = [torch.sigmoid(m.detach().float()) for m in (self.time_mix_q, self.time_mix_k,
                                                           self.time_mix_v)]
        quant = R.shift_quantize(x, *sig)
        B, T, _ = x.shape
        outs = []
        for (codes, scales), proj in zip(quant, (self.q_proj, self.k_proj, self.v_proj)):
            proj._quantize_weight()
            y = w8a8_gemm_out(codes, scales, proj.weight_codes, proj.weight_scales,
                              bias=None if proj.bias is None else proj.bias.detach().float(),
                              out_dtype=x.dtype)
            outs.append(y.reshape(B, T, -1))
        return outs

    def _out(self, hard: torch.Tensor, residual: torch.Tensor | None) -> torch.Tensor:
        from ..kernels.linear import Int8Linear
        if residual is None:
            return self.out_proj(hard)
        if isinstance(self.out_proj, Int8Linear):
            return self.out_proj(hard, residual=residual)
        return residual + self.out_proj(hard)

    def forward(self, x: torch.Tensor, residual: torch.Tensor | None = None) -> torch.Tensor:
        """x (B, T, d) -> (B, T, d) (rosa.py:135-165). Training on the GPU uses the exact
        credit backward (HardRosaGPU); eval computes the hard match without gradients to
        the symbol projections, like the reference path. With ``residual`` the result is
        residual + mixer(x), the add fused into the output projection's store."""
        if not x.is_cuda:
            raise RuntimeError("ksdraft_amd's Rosa mixer runs on the GPU only (no CPU path)")
        from ..kernels.rosa_credit_gpu import HardRosaGPU
        if self.training:
            fused = self._fused_training_projections(x) if torch.is_grad_enabled() else None
            if fused is not None:
                q_full, k_full, v_full = fused
            else:
                q_in, k_in, v_in = self._shifted(x)
                q_full, k_full, v_full = self.q_proj(q_in), self.k_proj(k_in), self.v_proj(v_in)
            hard = HardRosaGPU.apply(q_full, k_full, v_full, self.payload)
            return self._out(hard.to(x.dtype), residual)
        if self._int8_projections() and not torch.is_grad_enabled():
            q_full, k_full, v_full = self._fused_projections(x)
        else:
            q_in, k_in, v_in = self._shifted(x)
            q_full, k_full, v_full = self.q_proj(q_in), self.k_proj(k_in), self.v_proj(v_in)
        with torch.no_grad():
            qb, kb, vb = R.pack_bits3(q_full.detach(), k_full.detach(), v_full.detach())
            B, T, S = q_full.shape
            sign, _ = R.match_packed(qb.reshape(B * S, -1), kb.reshape(B * S, -1),
                                     vb.reshape(B * S, -1), T)
        out = self.payload[None, :, None] * sign.reshape(B, S, T).float()
        return self._out(out.permute(0, 2, 1).to(x.dtype), residual)
