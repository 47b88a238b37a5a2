"""Rosa mixer step kernels on gfx950 (the R1/R2/R4 pieces of reference
ksdraft/model/rosa.py and ksdraft/kernels/rosa_credit_gpu.py).

  shift_quantize   RosaMixer._shifted fused with each projection input's quantization
  shift_quantize_dual   the same for training: row codes plus dW's transposed operand
  shift_backward   the shift's backward: the input gradient and the sigmoid(mix) gradients
  ShiftedInt8Projections   autograd of shift + the three Int8Linear q/k/v projections
  pack_bits        (x > 0) symbol bits of (B, T, S) projections, packed along T
  match_packed     _match_payload_sign on packed bits: sign and matched endpoint
  hard_out         payload * sign back in (B, T, S)
"""

from __future__ import annotations

import ctypes

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


def _ptr_array(ptrs):
    return (ctypes.c_void_p * len(ptrs))(*ptrs)


def shift_quantize_dual(x: torch.Tensor, sig_q: torch.Tensor, sig_k: torch.Tensor,
                        sig_v: torch.Tensor):
    """The three time-shifted inputs (rosa.py:128-133), each quantized in both layouts of
    an Int8Linear training forward (group 128): the row codes, and the input transposed and
    requantized along the tokens from them (quantize_dual(., t_from_codes=True)).

    x (B, T, d) fp32/bf16/fp16 with d % 8 == 0; sig_* (d,) fp32 = torch.sigmoid(time_mix_*).
    Returns three (codes (B*T, d), scales (B*T, d/128), codes_t (d, B*T),
    scales_t (d, ceil(B*T/128))) tuples."""
    dev = _lib.require_gpu(x, sig_q, sig_k, sig_v)
    if x.dim() != 3:
        raise ValueError("x must be (B, T, d)")
    B, T, d = x.shape
    x = x.contiguous()
    M = B * T
    outs = []
    for _ in range(3):
        outs.append((torch.empty((M, d), dtype=torch.int8, device=dev),
                     torch.empty((M, -(-d // 128)), dtype=SCALE_DTYPE, device=dev),
                     torch.empty((d, M), dtype=torch.int8, device=dev),
                     torch.empty((d, -(-M // 128)), dtype=SCALE_DTYPE, device=dev)))
    sq, sk, sv = (s.to(device=dev, dtype=torch.float32).contiguous() for s in (sig_q, sig_k, sig_v))
    arrs = [_ptr_array([o[i].data_ptr() for o in outs]) for i in range(4)]
    _lib.call("ksd_rosa_shift_quant_dual", x.data_ptr(), _lib.dtype_code(x.dtype), B, T, d,
              sq.data_ptr(), sk.data_ptr(), sv.data_ptr(), *arrs, _lib.stream_ptr(dev))
    return tuple(outs)


def shift_backward(x: torch.Tensor, g_q: torch.Tensor, g_k: torch.Tensor, g_v: torch.Tensor,
                   sig_q: torch.Tensor, sig_k: torch.Tensor, sig_v: torch.Tensor):
    """Backward of the three lerps of RosaMixer._shifted given dL/d(q_in, k_in, v_in)
    (fp32, shaped like x). Returns (dx in x's dtype, dL/dsig (3, d) fp32)."""
    dev = _lib.require_gpu(x, g_q, g_k, g_v, sig_q, sig_k, sig_v)
    B, T, d = x.shape
    x = x.contiguous()
    gs = [g.reshape(B * T, d).float().contiguous() for g in (g_q, g_k, g_v)]
    sq, sk, sv = (s.to(device=dev, dtype=torch.float32).contiguous() for s in (sig_q, sig_k, sig_v))
    nb = ctypes.c_int64(0)
    _lib.call("ksd_rosa_shift_backward_blocks", B, T, ctypes.byref(nb))
    dx = torch.empty_like(x)
    part = torch.empty((max(nb.value, 1), 3, d), dtype=torch.float32, device=dev)
    _lib.call("ksd_rosa_shift_backward", x.data_ptr(), _lib.dtype_code(x.dtype), B, T, d,
              gs[0].data_ptr(), gs[1].data_ptr(), gs[2].data_ptr(), sq.data_ptr(),
              sk.data_ptr(), sv.data_ptr(), dx.data_ptr(), part.data_ptr(), _lib.stream_ptr(dev))
    return dx, part[:nb.value].sum(0)


class ShiftedInt8Projections(torch.autograd.Function):
    """(q, k, v) = (q_proj, k_proj, v_proj)(RosaMixer._shifted(x)) (rosa.py:128-149) for
    Int8Linear projections in training, without materialising the shifted inputs:

      forward   shift_quantize_dual (one pass over x: each input's row codes and its
                requantized transpose), then the three W8A8 GEMMs + bias, fp32 out
      backward  per projection the Int8Linear int8 backward (dX, dW; db = sum of dY), then
                shift_backward folds the three dX into dx and the sigmoid(mix) gradients

    The int8 operands, GEMM outputs, dX and dW are those of Int8Linear on the shifted
    inputs; dx and the sigmoid gradients are fp32 sums in this kernel's order.
    Inputs: x, sig_q, sig_k, sig_v, then per projection (weight, bias, weight_codes,
    weight_scales), then optionally the three projections' dX operands (codes_t, scales_t)
    or None each (Int8Linear.current_transpose)."""

    @staticmethod
    def forward(ctx, x, sig_q, sig_k, sig_v, wq, bq, cq, sq, wk, bk, ck, sk, wv, bv, cv, sv, wts=None):
        from .gemm import w8a8_gemm_out
        B, T, _ = x.shape
        quant = shift_quantize_dual(x, sig_q, sig_k, sig_v)
        outs = []
        for (codes, scales, _, _), bias, wc, ws in zip(quant, (bq, bk, bv), (cq, ck, cv),
                                                       (sq, sk, sv)):
            y = w8a8_gemm_out(codes, scales, wc, ws, bias=None if bias is None else bias.detach(),
                              out_dtype=torch.float32)
            outs.append(y.reshape(B, T, -1))
        ctx.save_for_backward(x, sig_q, sig_k, sig_v, quant[0][2], quant[0][3], quant[1][2],
                              quant[1][3], quant[2][2], quant[2][3], cq, sq, ck, sk, cv, sv)
        ctx.has_bias = (bq is not None, bk is not None, bv is not None)
        ctx.wts = wts if wts is not None else (None, None, None)
        return tuple(outs)

    @staticmethod
    def backward(ctx, gq, gk, gv):
        from .linear import w8a8_linear_backward
        (x, sig_q, sig_k, sig_v, xtq0, xts0, xtq1, xts1, xtq2, xts2,
         cq, sq, ck, sk, cv, sv) = ctx.saved_tensors
        B, T, d = x.shape
        need = ctx.needs_input_grad
        dxs, grads = [], []
        for m, (g, xt, wc, ws) in enumerate(zip(
                (gq, gk, gv), ((xtq0, xts0), (xtq1, xts1), (xtq2, xts2)), (cq, ck, cv),
                (sq, sk, sv))):
            S = wc.shape[0]
            if g is None:
                g = torch.zeros((B, T, S), dtype=torch.float32, device=x.device)
            g2 = g.reshape(-1, S).float().contiguous()
            want_db = ctx.has_bias[m] and need[5 + 4 * m]
            res = w8a8_linear_backward(g2, None, None, wc, ws, need_dx=True,
                                       need_dw=need[4 + 4 * m], xt=xt, wt=ctx.wts[m],
                                       want_db=want_db)
            dx_m, dw = res[0], res[1]
            db = res[2] if want_db else None
            dxs.append(dx_m)
            grads.extend([dw, db, None, None])
        dx, dsig = shift_backward(x, *dxs, sig_q, sig_k, sig_v)
        return (dx if need[0] else None, dsig[0], dsig[1], dsig[2], *grads, None)


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


def pack_bits3(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor):
    """pack_bits of three (B, T, S) projections of one shape and dtype, in one launch."""
    dev = _lib.require_gpu(q, k, v)
    if q.dim() != 3 or k.shape != q.shape or v.shape != q.shape:
        raise ValueError("q, k, v must be (B, T, S) tensors of one shape")
    xs = []
    for x in (q, k, v):
        if not torch.is_floating_point(x) or x.dtype == torch.float64:
            x = x.float()
        xs.append(x.contiguous())
    if not (xs[0].dtype == xs[1].dtype == xs[2].dtype):
        xs = [x.float() for x in xs]
    B, T, S = q.shape
    outs = [torch.empty((B, S, -(-T // 32)), dtype=torch.int32, device=dev) for _ in range(3)]
    _lib.call("ksd_rosa_pack_bits3", xs[0].data_ptr(), xs[1].data_ptr(), xs[2].data_ptr(),
              _lib.dtype_code(xs[0].dtype), B, T, S, outs[0].data_ptr(), outs[1].data_ptr(),
              outs[2].data_ptr(), _lib.stream_ptr(dev))
    return outs


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
    sign = sign.contiguous()  # bound to a name: it must outlive the enqueued kernel
    _lib.call("ksd_rosa_hard", sign.data_ptr(), p.data_ptr(), B, T, S,
              out.data_ptr(), _lib.dtype_code(out_dtype), _lib.stream_ptr(dev))
    return out
