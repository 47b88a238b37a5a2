"""Rosa mixer step kernels on gfx950 (the R1/R2/R4 pieces of reference
ksdraft/model/rosa.py and ksdraft/kernels/rosa_credit_gpu.py).

  shift_quantize   RosaMixer._shifted fused with each projection input's quantization
  pack_bits        (x > 0) symbol bits of (B, T, S) projections, packed along T
  match_packed     _match_payload_sign on packed bits: sign and matched endpoint
  hard_out         payload * sign back in (B, T, S)
"""

from __future__ import annotations

import torch

from .. import _lib
from .quant import GROUP_SIZE, SCALE_DTYPE


def resolve_max_match_len(T: int, max_match_len: int | None = None) -> int:
    """rosa.py:50-55."""
    if max_match_len is None:
        return max(1, min(62, T - 1)) if T > 1 else 0
    return min(max_match_len, T - 1)


def shift_quantize(x: torch.Tensor, sig_q: torch.Tensor, sig_k: torch.Tensor,
                   sig_v: torch.Tensor, group: int = GROUP_SIZE):
    """quantize_last_dim of the three time-shifted inputs (rosa.py:128-133) in one pass.

    x (B, T, d) fp32/bf16/fp16; sig_* (d,) fp32 = torch.sigmoid(time_mix_*).
    Returns three (codes (B*T, d) int8, scales (B*T, ceil(d/group)) fp16) pairs."""
    dev = _lib.require_gpu(x, sig_q, sig_k, sig_v)
    if x.dim() != 3:
        raise ValueError("x must be (B, T, d)")
    B, T, d = x.shape
    x = x.contiguous()
    ng = -(-d // group)
    outs = []
    for _ in range(3):
        outs.append((torch.empty((B * T, d), dtype=torch.int8, device=dev),
                     torch.empty((B * T, ng), dtype=SCALE_DTYPE, device=dev)))
    sq, sk, sv = (s.to(device=dev, dtype=torch.float32).contiguous() for s in (sig_q, sig_k, sig_v))
    _lib.call("ksd_rosa_shift_quant", x.data_ptr(), _lib.dtype_code(x.dtype), B, T, d,
              sq.data_ptr(), sk.data_ptr(), sv.data_ptr(), group,
              outs[0][0].data_ptr(), outs[0][1].data_ptr(), outs[1][0].data_ptr(),
              outs[1][1].data_ptr(), outs[2][0].data_ptr(), outs[2][1].data_ptr(),
              _lib.stream_ptr(dev))
    return tuple(outs)


def pack_bits(x: torch.Tensor) -> torch.Tensor:
    """(B, T, S) float -> (B, S, ceil(T/32)) int32 words of the (x > 0) bits."""
    dev = _lib.require_gpu(x)
    if x.dim() != 3:
        raise ValueError("x must be (B, T, S)")
    if not torch.is_floating_point(x) or x.dtype == torch.float64:
        x = x.float()
    x = x.contiguous()
    B, T, S = x.shape
    out = torch.empty((B, S, -(-T // 32)), dtype=torch.int32, device=dev)
    _lib.call("ksd_rosa_pack_bits", x.data_ptr(), _lib.dtype_code(x.dtype), B, T, S,
              out.data_ptr(), _lib.stream_ptr(dev))
    return out


def match_packed(q_bits: torch.Tensor, k_bits: torch.Tensor, v_bits: torch.Tensor, T: int,
                 max_match_len: int | None = None, want_j: bool = False):
    """Longest-suffix match on packed bits (n_streams, ceil(T/32)).

    Returns (sign int8 (n_streams, T) in {-1, +1}, endpoint int32 or None)."""
    dev = _lib.require_gpu(q_bits, k_bits, v_bits)
    n = q_bits.shape[0]
    lmax = resolve_max_match_len(T, max_match_len)
    if lmax > 63:
        raise ValueError(f"max_match_len {lmax} exceeds the 63-bit exact code width")
    sign = torch.empty((n, T), dtype=torch.int8, device=dev)
    mj = torch.empty((n, T), dtype=torch.int32, device=dev) if want_j else None
    if lmax < 1:
        sign.fill_(-1)
        if mj is not None:
            mj.fill_(-1)
        return sign, mj
    q_bits, k_bits, v_bits = (b.reshape(n, -1).contiguous() for b in (q_bits, k_bits, v_bits))
    _lib.call("ksd_rosa_match", q_bits.data_ptr(), k_bits.data_ptr(), v_bits.data_ptr(), n, T,
              lmax, sign.data_ptr(), _lib.ptr(mj), _lib.stream_ptr(dev))
    return sign, mj


def hard_out(sign: torch.Tensor, payload: torch.Tensor, out_dtype=torch.float32) -> torch.Tensor:
    """(B, S, T) int8 sign -> (B, T, S) payload[s] * sign (rosa_credit_gpu.py:75)."""
    dev = _lib.require_gpu(sign, payload)
    B, S, T = sign.shape
    out = torch.empty((B, T, S), dtype=out_dtype, device=dev)
    p = payload.to(device=dev, dtype=torch.float32).contiguous()
    _lib.call("ksd_rosa_hard", sign.contiguous().data_ptr(), p.data_ptr(), B, T, S,
              out.data_ptr(), _lib.dtype_code(out_dtype), _lib.stream_ptr(dev))
    return out
