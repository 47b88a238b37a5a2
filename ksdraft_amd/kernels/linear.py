"""Int8Linear — W8A8 GS128 drop-in for nn.Linear (mirror of reference ksdraft/kernels/linear.py).

Same constructor, attributes and methods as the reference (linear.py:23-97): fp32
masters ``weight``/``bias`` stay authoritative and are requantized (per-output-row
groups along the input dim) on every call into non-persistent ``weight_codes`` /
``weight_scales`` buffers.

Training differs from the reference on purpose: where the reference runs an fp32
straight-through estimator (``fake_quant_forward``, linear.py:75-97), this layer runs
the INT8-native autograd function ``W8A8LinearFunction`` — int8 forward GEMM and int8
backward GEMMs built with the recipe of reference ksdraft/kernels/ks3_int8.py:403-424:

    dX = quant_N(dY) . requant_N(W)^T              (W^T requantized along N)
    dW = quant_M(dY)^T . requant_M(dequant(quant(X)))^T   (both along tokens M)

Setting ``ste_training = True`` on a module restores the reference's STE behaviour.
"""

from __future__ import annotations

import torch
from torch import nn

from .gemm import w8a8_gemm, w8a8_gemm_out, w8a8_gemm_pair
from .quant import (GROUP_SIZE, dequantize_last_dim, quantize_dual, quantize_dual2,
                    quantize_dual_colsum, quantize_last_dim, quantize_last_dim_dithered,
                    quantize_transpose, requant_transpose)


_OUT_DTYPES = (torch.float32, torch.bfloat16, torch.float16)


def _out_dtype(dtype: torch.dtype) -> torch.dtype:
    return dtype if dtype in _OUT_DTYPES else torch.float32


def w8a8_linear_forward(x2: torch.Tensor, wq: torch.Tensor, ws: torch.Tensor,
                        bias: torch.Tensor | None, group: int = GROUP_SIZE,
                        out_dtype: torch.dtype | None = None,
                        residual: torch.Tensor | None = None):
    """y = W8A8(x2, W) + bias in one quantize + one GEMM launch (linear.py:68-73), plus an
    optional residual (M, N) of the output dtype added in the GEMM's store.

    Returns (y, xq, xs); the activation codes are what the backward keeps."""
    xq, xs = quantize_last_dim(x2, group)          # == quantize_last_dim(x2.float())
    y = w8a8_gemm_out(xq, xs, wq, ws, group, bias=bias,
                      out_dtype=_out_dtype(out_dtype or x2.dtype), residual=residual)
    return y, xq, xs


def w8a8_linear_forward_train(x2: torch.Tensor, wq: torch.Tensor, ws: torch.Tensor,
                              bias: torch.Tensor | None, group: int = GROUP_SIZE,
                              out_dtype: torch.dtype | None = None,
                              residual: torch.Tensor | None = None, xpre: tuple | None = None):
    """w8a8_linear_forward that also builds dW's activation operand in the same pass
    over x: X^T requantized along the tokens from the row codes (the double-quant recipe
    of ks3_int8.py:417-420, quantize_dual). The backward needs only that operand, not
    the row codes. ``xpre``: x's (codes, scales, codes_t, scales_t) when the caller has
    them already (quantize_dual2 with the weight). Returns (y, xtq (K, M), xts (K,
    ceil(M/group)))."""
    xq, xs, xtq, xts = xpre if xpre is not None else quantize_dual(x2, group, t_from_codes=True)
    y = w8a8_gemm_out(xq, xs, wq, ws, group, bias=bias,
                      out_dtype=_out_dtype(out_dtype or x2.dtype), residual=residual)
    return y, xtq, xts


def w8a8_linear_backward(g: torch.Tensor, xq: torch.Tensor | None, xs: torch.Tensor | None,
                         wq: torch.Tensor, ws: torch.Tensor, group: int = GROUP_SIZE,
                         dx_dtype: torch.dtype = torch.float32, need_dx: bool = True,
                         need_dw: bool = True, xt: tuple | None = None, wt: tuple | None = None,
                         want_db: bool = False):
    """INT8 backward GEMMs of the linear layer (recipe of ks3_int8.py:403-424).

    g (M, N) upstream gradient; xq/xs the forward's activation codes, or ``xt`` =
    (xtq, xts) the already requantized X^T operand; wq/ws the weight codes, and ``wt`` =
    (wtq, wts) their requantized transpose when the caller already has it (e.g. from
    quantize_dual(w, t_from_codes=True)). When both gradients are needed, dY is quantized
    in both layouts in one pass (quantize_dual).
    Returns (dx (M, K) in dx_dtype or None, dw (N, K) fp32 or None), and with ``want_db``
    a third entry, the bias gradient g.float().sum(0) (N,) fp32, formed in the dual
    quantization's pass over g when both GEMMs run."""
    dx = dw = db = None
    gq = gs = gtq = gts = None
    if need_dx and need_dw:
        if want_db:  # the column sums of g come out of the same read
            gq, gs, gtq, gts, db = quantize_dual_colsum(g, group)
        else:
            gq, gs, gtq, gts = quantize_dual(g, group)          # along N and along M
        if group == GROUP_SIZE:  # dX and dW in one launch (balanced over the CUs)
            wtq, wts = wt if wt is not None else requant_transpose(wq, ws, group, group)
            xtq, xts = xt if xt is not None else requant_transpose(xq, xs, group, group)
            dx, dw = w8a8_gemm_pair((gq, gs, wtq, wts, _out_dtype(dx_dtype)),
                                    (gtq, gts, xtq, xts, torch.float32), group)
            return (dx, dw, db) if want_db else (dx, dw)
    elif want_db:
        db = g.float().sum(0)
    if need_dx:
        if gq is None:
            gq, gs = quantize_last_dim(g, group)                # along N (per token)
        if wt is not None:
            wtq, wts = wt
        else:
            wtq, wts = requant_transpose(wq, ws, group, group)  # W^T (K, N) along N
        dx = w8a8_gemm_out(gq, gs, wtq, wts, group, out_dtype=_out_dtype(dx_dtype))
    if need_dw:
        if gtq is None:
            gtq, gts = quantize_transpose(g, group)             # dY^T (N, M) along M
        if xt is not None:
            xtq, xts = xt
        else:
            xtq, xts = requant_transpose(xq, xs, group, group)  # X^T (K, M) along M
        dw = w8a8_gemm(gtq, gts, xtq, xts, group)                # (N, K) fp32
    return (dx, dw, db) if want_db else (dx, dw)


class W8A8LinearFunction(torch.autograd.Function):
    """y = W8A8(x, W) + b (+ residual) with int8 backward GEMMs; returns fp32-master
    gradients. The residual, when given, is added in the GEMM's store and its gradient
    is the upstream gradient itself."""

    @staticmethod
    def forward(ctx, x, weight, bias, wq, ws, group, residual=None, wt=None, xpre=None):
        K = x.shape[-1]
        N = wq.shape[0]
        x2 = x.reshape(-1, K)
        r2 = None if residual is None else residual.reshape(-1, N)
        if ctx.needs_input_grad[1]:
            # dW's operand X^T comes out of the same pass over x as the forward's codes
            y, xtq, xts = w8a8_linear_forward_train(x2, wq, ws, bias, group, x.dtype, r2, xpre)
        else:
            y, _, _ = w8a8_linear_forward(x2, wq, ws, bias, group, x.dtype, r2)
            xtq = xts = None
        ctx.save_for_backward(xtq, xts, wq, ws)
        ctx.wt = wt  # (W^T codes, scales) for dX when the caller has them
        ctx.x_shape = x.shape
        ctx.x_dtype = x.dtype
        ctx.group = group
        ctx.has_bias = bias is not None
        return y.reshape(*x.shape[:-1], N)

    @staticmethod
    def backward(ctx, grad_out):
        xtq, xts, wq, ws = ctx.saved_tensors
        N = wq.shape[0]
        g = grad_out.reshape(-1, N)
        if g.dtype not in _OUT_DTYPES:
            g = g.float()
        g = g.contiguous()
        want_db = ctx.has_bias and ctx.needs_input_grad[2]
        res = w8a8_linear_backward(g, None, None, wq, ws, ctx.group, ctx.x_dtype,
                                   ctx.needs_input_grad[0], ctx.needs_input_grad[1],
                                   xt=(xtq, xts) if xtq is not None else None, wt=ctx.wt,
                                   want_db=want_db)
        dx, dw = res[0], res[1]
        db = res[2] if want_db else None
        if dx is not None:
            dx = dx.reshape(ctx.x_shape).to(ctx.x_dtype)
        dres = grad_out if len(ctx.needs_input_grad) > 6 and ctx.needs_input_grad[6] else None
        return dx, dw, db, None, None, None, dres, None, None


class Int8Linear(nn.Module):
    ste_training = False  # True: reference fp32 STE training path (fake_quant_forward)

    def __init__(self, in_features: int, out_features: int, bias: bool = True):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        # zeros, not empty: uninitialised memory could hold NaN patterns (linear.py:27-28)
        self.weight = nn.Parameter(torch.zeros(out_features, in_features))
        self.bias = nn.Parameter(torch.zeros(out_features)) if bias else None
        self.register_buffer("weight_codes", None, persistent=False)
        self.register_buffer("weight_scales", None, persistent=False)
        if self.weight.is_cuda:
            self._quantize_weight()

    @classmethod
    def from_float(cls, module: nn.Linear) -> "Int8Linear":
        lin = cls(module.in_features, module.out_features, bias=module.bias is not None)
        with torch.no_grad():
            lin.weight.copy_(module.weight)
            if module.bias is not None:
                lin.bias.copy_(module.bias)
        lin = lin.to(module.weight.device)
        if lin.weight.is_cuda:
            lin._quantize_weight()  # codes must reflect the copied masters
        return lin

    @torch.no_grad()
    def _quantize_weight(self) -> None:
        dither = float(getattr(self, "_dither", 0.0))
        w = self.weight.detach()
        if w.dtype not in (torch.float32, torch.bfloat16, torch.float16):
            w = w.float()
        wt = None
        if dither > 0:
            codes, scales = quantize_last_dim_dithered(w.float(), GROUP_SIZE, dither)
        elif self.training and self.weight.requires_grad and w.dim() == 2:
            # training: the row codes and dX's operand W^T = quant(dequant(W)^T) (the recipe
            # of ks3_int8.py:349-351) from one pass over the master
            codes, scales, ct, st = quantize_dual(w.float(), GROUP_SIZE, t_from_codes=True)
            wt = (ct, st)
        else:
            codes, scales = quantize_last_dim(w.float())
        self.weight_codes = codes
        self.weight_scales = scales
        self._wt = wt  # valid while weight_codes is these codes
        self._wt_src = codes

    def _quantize_weight_dithered(self, dither: float) -> None:
        self._dither = dither
        self._quantize_weight()

    def invalidate_codes(self) -> None:
        """Forget codes handed over by an optimizer (train.AdamWRequant.register_int8):
        the next call requantizes the master. Needed after a write to the master that
        torch does not version, i.e. through ``weight.data`` or a raw pointer."""
        self._codes_key = None

    def _codes_current(self) -> bool:
        """True when train.AdamWRequant wrote the codes in the same pass that last
        updated the master and the master has kept its storage and in-place version."""
        key = getattr(self, "_codes_key", None)
        return (key is not None and self.weight_codes is not None
                and getattr(self, "_codes_owner", None) is not None
                and getattr(self, "_dither", 0.0) <= 0
                and key == (self.weight.data_ptr(), self.weight._version))

    def current_transpose(self):
        """(codes_t, scales_t) = requant_transpose(weight_codes, weight_scales), dX's operand,
        when it was built for the codes the module holds now (by its training forward or by
        the optimizer that handed the codes over), else None."""
        wt = getattr(self, "_wt", None)
        if wt is None or getattr(self, "_wt_src", None) is not self.weight_codes:
            return None
        return wt

    def _apply(self, fn, *args, **kwargs):
        self.invalidate_codes()  # .to(), .cuda(), .half() ... may replace the master
        return super()._apply(fn, *args, **kwargs)

    def _load_from_state_dict(self, *args, **kwargs):
        self.invalidate_codes()  # load_state_dict writes the master in place
        return super()._load_from_state_dict(*args, **kwargs)

    def forward(self, x: torch.Tensor, residual: torch.Tensor | None = None) -> torch.Tensor:
        """y = linear(x) (linear.py:62-73); with ``residual`` (shaped like y, x's dtype),
        residual + linear(x), the residual added in the GEMM's store."""
        # live fp32 masters stay authoritative (linear.py:66): the codes are rebuilt on every
        # call unless an optimizer handed over the codes of the master as it is now
        # (_codes_current); dithered codes are redrawn every call
        train = torch.is_grad_enabled() and (self.weight.requires_grad or x.requires_grad
                                             or (residual is not None and residual.requires_grad))
        xpre = None
        if not self._codes_current():
            self._codes_key = None
            w = self.weight.detach()
            if (train and not self.ste_training and self.training and self.weight.requires_grad
                    and float(getattr(self, "_dither", 0.0)) == 0.0 and w.dim() == 2
                    and w.dtype == torch.float32 and x.dtype == torch.float32):
                # a training forward quantizes the master (both layouts) and x (both
                # layouts) in one launch
                (codes, scales, ct, st), xpre = quantize_dual2(w, x.reshape(-1, x.shape[-1]))
                self.weight_codes, self.weight_scales = codes, scales
                self._wt, self._wt_src = (ct, st), codes
            else:
                self._quantize_weight()
        fuse_res = (residual is not None and x.dtype in _OUT_DTYPES
                    and residual.dtype == x.dtype and not self.ste_training)
        if train:
            if self.ste_training:
                y = self.fake_quant_forward(x)
                return y if residual is None else residual + y
            # other float dtypes (float64) go through .float() as the reference's
            # quantize_last_dim(x2.float()) does (linear.py:69); the result is cast back
            xin = x if x.dtype in _OUT_DTYPES else x.float()
            wt = self.current_transpose()  # None: the backward requantizes the codes
            y = W8A8LinearFunction.apply(xin, self.weight, self.bias, self.weight_codes,
                                         self.weight_scales, GROUP_SIZE,
                                         residual if fuse_res else None, wt, xpre)
            y = y.to(x.dtype)
            return y if fuse_res or residual is None else residual + y
        # linear.py:68-73: fp32 GEMM, + bias in fp32, then cast to x.dtype (fused)
        x2 = x.reshape(-1, x.shape[-1])
        if x2.dtype not in _OUT_DTYPES:
            x2 = x2.float()
        r2 = residual.reshape(-1, self.out_features) if fuse_res else None
        y, _, _ = w8a8_linear_forward(
            x2, self.weight_codes, self.weight_scales,
            self.bias.detach() if self.bias is not None else None, residual=r2)
        y = y.reshape(*x.shape[:-1], self.out_features).to(x.dtype)
        return y if fuse_res or residual is None else residual + y

    def fake_quant_forward(self, x: torch.Tensor) -> torch.Tensor:
        """Reference STE path (linear.py:75-97): fp32 GEMM on quantize-dequantized
        operands with straight-through gradients. Quantization runs on the HIP kernels;
        the fp32 product is torch's."""
        self._quantize_weight()
        w = dequantize_last_dim(self.weight_codes.detach(), self.weight_scales.detach()) \
            + (self.weight - self.weight.detach())
        x2 = x.reshape(-1, x.shape[-1]).float()
        codes, scales = quantize_last_dim(x2)
        xq = dequantize_last_dim(codes, scales) + (x2 - x2.detach())
        y = xq @ w.reshape(self.out_features, self.in_features).T
        if self.bias is not None:
            y = y + self.bias.float()
        return y.reshape(*x.shape[:-1], self.out_features).to(x.dtype)
