"""Fused float surfaces of the draft training step (config 5) on gfx950.

  TransferSpaceLoss   the transfer-space term of distillation_losses
                      (reference ksdraft/train/__init__.py:79-85) with its gradient
  FusedInjection      the float DSpine adjacent injection (reference
                      ksdraft/model/spine.py:38-68), forward and backward
  ResidualLayerNorm   nn.LayerNorm whose backward also takes the gradient of the residual
                      branch reading the same input (reference ksdraft/model/block.py:39-41)

Both are fp32 and agree with the torch composition of the reference to fp32 rounding
(their sums run in another order); the INT8 surfaces of the step are elsewhere. The
weight gradients of the low-rank maps reduce over all M tokens into a (rank, d) matrix;
``tn`` splits that reduction into batched chunks, which fills the GPU where a single
(rank x M) . (M x d) product does not.
"""

from __future__ import annotations

import ctypes

import torch

from .. import _lib


def _f32c(t: torch.Tensor) -> torch.Tensor:
    return t.float().contiguous()


def transfer_cos(f: torch.Tensor, e_hat: torch.Tensor):
    """Per row r of f (M, d): cos = <f_r, e_r> / max(|f_r|, 1e-12) and |f_r|."""
    dev = _lib.require_gpu(f, e_hat)
    M, d = f.shape
    cos = torch.empty(M, dtype=torch.float32, device=dev)
    nrm = torch.empty(M, dtype=torch.float32, device=dev)
    _lib.call("ksd_transfer_cos", f.data_ptr(), e_hat.data_ptr(), M, d, cos.data_ptr(),
              nrm.data_ptr(), _lib.stream_ptr(dev))
    return cos, nrm


def transfer_grad(f, e_hat, cos, nrm, coef, df, grad_e, first: bool):
    dev = _lib.require_gpu(f, e_hat, cos, nrm, coef, df, grad_e)
    M, d = f.shape
    _lib.call("ksd_transfer_grad", f.data_ptr(), e_hat.data_ptr(), cos.data_ptr(), nrm.data_ptr(),
              coef.data_ptr(), M, d, df.data_ptr(), grad_e.data_ptr(), int(first),
              _lib.stream_ptr(dev))


class TransferSpaceLoss(torch.autograd.Function):
    """ts = (1 / L) sum_l mean_r (1 - <normalize(f_l[r]), e_hat[r]>) (train/__init__.py:79-85),
    e_hat = F.normalize(embedding[targets]) computed by the caller (its gradient flows back
    through torch). features: L tensors shaped (..., d) with M rows; returns a 0-dim tensor."""

    @staticmethod
    def forward(ctx, e_hat, *features):
        M, d = e_hat.shape
        e2 = _f32c(e_hat)
        fs, cs, ns = [], [], []
        for f in features:
            f2 = _f32c(f.reshape(M, d))
            c, n = transfer_cos(f2, e2)
            fs.append(f2)
            cs.append(c)
            ns.append(n)
        L = len(features)
        if L == 0:
            ts = e_hat.new_zeros((), dtype=torch.float32)
        else:
            ts = (1.0 - torch.stack(cs)).mean(1).sum() / L
        ctx.save_for_backward(e2, *fs, *cs, *ns)
        ctx.L, ctx.shapes = L, [(f.shape, f.dtype) for f in features]
        ctx.e_dtype = e_hat.dtype
        return ts

    @staticmethod
    def backward(ctx, g):
        L = ctx.L
        saved = ctx.saved_tensors
        e2, fs, cs, ns = saved[0], saved[1:1 + L], saved[1 + L:1 + 2 * L], saved[1 + 2 * L:]
        if L == 0:
            return (torch.zeros_like(e2).to(ctx.e_dtype),)
        M = e2.shape[0]
        coef = (g.float() / (L * M)).reshape(1).contiguous()
        ge = torch.empty_like(e2)
        dfs = []
        for i in range(L):
            df = torch.empty_like(fs[i])
            transfer_grad(fs[i], e2, cs[i], ns[i], coef, df, ge, i == 0)
            shape, dt = ctx.shapes[i]
            dfs.append(df.reshape(shape).to(dt))
        return (ge.to(ctx.e_dtype), *dfs)


# ---------------------------------------------------------------- injection
def tn(a: torch.Tensor, b: torch.Tensor, chunks: int = 8) -> torch.Tensor:
    """a^T . b for a (M, r), b (M, n): the M-long reduction split into `chunks` batched
    products and summed (a (rank x M) . (M x n) product alone leaves most of the GPU idle)."""
    M = a.shape[0]
    if M % chunks or M < 64 * chunks:
        return a.t() @ b
    if a.shape[1] > b.shape[1]:  # transpose the narrower operand: (b^T a)^T
        return tn(b, a, chunks).t()
    ac = a.reshape(chunks, M // chunks, a.shape[1]).transpose(1, 2).contiguous()
    bc = b.reshape(chunks, M // chunks, b.shape[1])
    if not bc.is_contiguous():
        bc = bc.contiguous()
    return torch.bmm(ac, bc).sum(0)


def injection_update(zs, wc, wiu, bias, z2):
    dev = _lib.require_gpu(zs, wc, wiu, z2)
    M, d = z2.shape
    out = torch.empty_like(z2)
    _lib.call("ksd_injection_update", zs.data_ptr(), wc.data_ptr(), wiu.data_ptr(),
              _lib.ptr(bias), z2.data_ptr(), M, d, out.data_ptr(), _lib.stream_ptr(dev))
    return out


def injection_update_backward(zs, wc, wiu, bias, g2):
    dev = _lib.require_gpu(zs, wc, wiu, g2)
    M, d = g2.shape
    dpre = torch.empty_like(g2)
    du = torch.empty_like(g2)
    _lib.call("ksd_injection_update_backward", zs.data_ptr(), wc.data_ptr(), wiu.data_ptr(),
              _lib.ptr(bias), g2.data_ptr(), M, d, dpre.data_ptr(), du.data_ptr(),
              _lib.stream_ptr(dev))
    return dpre, du


class FusedInjection(torch.autograd.Function):
    """The float adjacent injection (spine.py:38-68) of one layer, ranks 32 (gates,
    injection) and 64 (feature):

        zd  = z . [feature_down; gate_q.down]^T                       (M, 96)
        p   = zd[:, :64] . feature_up^T                               (M, d), returned
        pd  = p_prev . [gate_p.down; inject.down]^T = shift(p . W^T)   (M, 64)
        out = z + sigmoid(gate_q.up(zd[:, 64:]) + gate_p.up(pd[:, :32]) + bias)
                  * inject.up(pd[:, 32:])

    p_prev is p one token later (0 at t = 0, or the previous layer's feature there): the
    product with the down weights is taken on p and its rows shifted, so p_prev is never
    materialised. The gated update is one HIP pass (ksd_injection_update); the backward
    recomputes its pre-activations (ksd_injection_update_backward) and takes every
    weight gradient with ``tn``.

    Inputs: z (B, T, d) fp32, prev0 (B, 1, d) or None, then the weights feature_down (64, d),
    gate_q.down (32, d), feature_up (d, 64), gate_p.down (32, d), inject.down (32, d),
    gate_q.up (d, 32), gate_p.up (d, 32), gate_bias (d,), inject.up (d, 32)."""

    @staticmethod
    def forward(ctx, z, prev0, w_fd, w_gqd, w_fu, w_gpd, w_id, w_gqu, w_gpu, bias, w_iu):
        B, T, d = z.shape
        M = B * T
        r1 = w_fd.shape[0]
        z2 = _f32c(z.reshape(M, d))
        wa = torch.cat([w_fd, w_gqd]).float()                 # (96, d)
        wb = torch.cat([w_gpd, w_id]).float()                 # (64, d)
        wc = torch.cat([w_gqu, w_gpu], dim=1).float().contiguous()  # (d, 64)
        wiu = _f32c(w_iu)                                     # (d, 32)
        zd = z2 @ wa.t()                                      # (M, 96)
        p = zd[:, :r1] @ w_fu.float().t()                     # (M, d)
        pp = (p @ wb.t()).reshape(B, T, -1)
        pd = torch.zeros_like(pp)
        pd[:, 1:] = pp[:, :-1]
        if prev0 is not None:
            pd[:, 0] = prev0.reshape(B, d).float() @ wb.t()
        zs = torch.cat([zd[:, r1:], pd.reshape(M, -1)], dim=1).contiguous()  # (M, 96)
        b = None if bias is None else _f32c(bias)
        out = injection_update(zs, wc, wiu, b, z2)
        ctx.save_for_backward(z2, zd, p, zs, wa, wb, wc, wiu, b, w_fu,
                              prev0 if prev0 is not None else None)
        ctx.dims = (B, T, d, r1)
        ctx.has_prev = prev0 is not None
        ctx.has_bias = bias is not None
        ctx.dtypes = (z.dtype, w_fd.dtype)
        return out.reshape(B, T, d).to(z.dtype), p.reshape(B, T, d).to(z.dtype)

    @staticmethod
    def backward(ctx, dout, dp_ext):
        z2, zd, p, zs, wa, wb, wc, wiu, b, w_fu, prev0 = ctx.saved_tensors
        B, T, d, r1 = ctx.dims
        M = B * T
        r2 = wc.shape[1] // 2
        g2 = torch.zeros((M, d), device=z2.device) if dout is None else _f32c(dout.reshape(M, d))
        dpre, du = injection_update_backward(zs, wc, wiu, b, g2)
        dzg = dpre @ wc                                        # (M, 64): [zd_g | pd_g]
        dpi = du @ wiu                                         # (M, 32)
        dwc = tn(dpre, zs[:, :2 * r2])                         # (d, 64)
        dwiu = tn(du, zs[:, 2 * r2:])                          # (d, 32)
        db = dpre.sum(0) if ctx.has_bias else None
        dpd = torch.cat([dzg[:, r2:], dpi], dim=1).reshape(B, T, -1)   # d pd (B, T, 64)
        dpp = torch.zeros_like(dpd)
        dpp[:, :-1] = dpd[:, 1:]
        dpp = dpp.reshape(M, -1)
        dwb = tn(dpp, p)                                       # (64, d)
        dprev0 = None
        if ctx.has_prev:
            d0 = dpd[:, 0]                                     # (B, 64)
            dprev0 = (d0 @ wb).reshape(B, 1, d).to(prev0.dtype)
            dwb = dwb + d0.t() @ prev0.reshape(B, d).float()
        if dp_ext is not None:
            dp = torch.addmm(_f32c(dp_ext.reshape(M, d)), dpp, wb)
        else:
            dp = dpp @ wb                                      # (M, d)
        wfu = w_fu.float()
        dzd1 = dp @ wfu                                        # (M, 64)
        dwfu = tn(dp, zd[:, :r1])                              # (d, 64)
        dzd = torch.cat([dzd1, dzg[:, :r2]], dim=1)            # (M, 96)
        dz = torch.addmm(g2, dzd, wa)                          # dout + dzd . wa
        dwa = tn(dzd, z2)                                      # (96, d)
        zdt, wdt = ctx.dtypes
        cast = (lambda t: t.to(wdt).contiguous())
        return (dz.reshape(B, T, d).to(zdt), dprev0, cast(dwa[:r1]), cast(dwa[r1:]), cast(dwfu),
                cast(dwb[:r2]), cast(dwb[r2:]), cast(dwc[:, :r2]), cast(dwc[:, r2:]),
                None if db is None else cast(db), cast(dwiu))


# ---------------------------------------------------------------- layer norm
def layernorm_backward(x2, dy2, dres2, mean, rstd, weight):
    """(dx, dweight, dbias) of nn.LayerNorm for fp32 rows (M, d), plus dres2 (or None)."""
    dev = _lib.require_gpu(x2, dy2, mean, rstd, weight)
    M, d = x2.shape
    nb = ctypes.c_int64(0)
    _lib.call("ksd_layernorm_backward_blocks", M, ctypes.byref(nb))
    dx = torch.empty_like(x2)
    part = torch.empty((max(nb.value, 1), 2, d), dtype=torch.float32, device=dev)
    _lib.call("ksd_layernorm_backward", x2.data_ptr(), dy2.data_ptr(), _lib.ptr(dres2),
              mean.data_ptr(), rstd.data_ptr(), weight.data_ptr(), M, d, dx.data_ptr(),
              part.data_ptr(), _lib.stream_ptr(dev))
    dwb = part[:nb.value].sum(0)
    return dx, dwb[0], dwb[1]


class ResidualLayerNorm(torch.autograd.Function):
    """(layer_norm(x), x): nn.LayerNorm (block.py:27-41) and the residual branch's copy of
    its input as a second output, so that the backward receives both gradients and forms
    dx = LN_backward(dy) + dres in one pass (ksd_layernorm_backward) instead of autograd
    adding them. x (..., d) fp32 with d % 256 == 0; the forward is torch's."""

    @staticmethod
    def forward(ctx, x, weight, bias, eps):
        d = x.shape[-1]
        y, mean, rstd = torch.native_layer_norm(x, (d,), weight, bias, eps)
        ctx.save_for_backward(x, mean, rstd, weight)
        ctx.has_bias = bias is not None
        return y, x.view_as(x)

    @staticmethod
    def backward(ctx, dy, dres):
        x, mean, rstd, weight = ctx.saved_tensors
        d = x.shape[-1]
        x2 = _f32c(x.reshape(-1, d))
        M = x2.shape[0]
        dy2 = torch.zeros_like(x2) if dy is None else _f32c(dy.reshape(M, d))
        dr2 = None if dres is None else _f32c(dres.reshape(M, d))
        dx, dw, db = layernorm_backward(x2, dy2, dr2, _f32c(mean.reshape(M)),
                                        _f32c(rstd.reshape(M)), _f32c(weight))
        return (dx.reshape(x.shape).to(x.dtype), dw.to(weight.dtype),
                db.to(weight.dtype) if ctx.has_bias else None, None)
