"""Oracle chains of whole INT8 surfaces, built from oracle/ (test infrastructure only).

Each function takes the surface's fp32 masters and its inputs as numpy arrays and returns
what the GPU path must produce bit-exactly: the int8 operands of every GEMM come from the
oracle quantizer following the recipes of reference ksdraft/kernels/ks3_int8.py:326-429,
and every GEMM output from the ordered-group contract (oracle/gemm.py).
"""

from __future__ import annotations

import numpy as np

from oracle import gemm as og
from oracle import ks3 as ok
from oracle import quant as oq


def linear_chain(x, w, bias, g):
    """Int8Linear (W8A8LinearFunction) forward and int8 backward, fp32 values.

    x (M, K), w (N, K), bias (N,) or None, g (M, N) upstream gradient (fp32 values).
    Returns dict(y, dx, dw, wq, ws)."""
    x = np.asarray(x, np.float32)
    xq, xs = oq.quantize_last_dim(x)
    wq, ws = oq.quantize_last_dim(np.asarray(w, np.float32))
    y = og.gemm_ordered(xq, xs, wq, ws, bias=bias)
    gq, gs = oq.quantize_last_dim(g)
    dx = og.gemm_ordered(gq, gs, *oq.requant_transpose(wq, ws))
    gtq, gts = oq.quantize_transpose(g)
    dw = og.gemm_ordered(gtq, gts, *oq.requant_transpose(xq, xs))
    return dict(y=y, dx=dx, dw=dw, wq=wq, ws=ws)


def ks3_cell_chain(master_down, master_up, master_coefficients, master_raw_scale,
                   master_raw_shift, x, grad_out):
    """_KS3Int8Train forward and backward (ks3_int8.py:326-429), rank 1, 'int8' mode.

    x (M, d) fp32 values; grad_out (M, d) (rounded to fp16 as the backward does).
    Returns dict(y, dx, ddown, dup, dcoeff, dscale, dshift, packed)."""
    p = ok.pack_masters(master_down, master_up, master_coefficients, master_raw_scale,
                        master_raw_shift)
    sc, sh = ok.warp_scalars(p["warp_scale_codes"], p["warp_scale_scales"],
                             p["warp_shift_codes"], p["warp_shift_scales"])
    lut = ok.make_tanh_lut()
    xq, xs = oq.quantize_last_dim(np.asarray(x, np.float32))
    coords = ok.coords_from_gemm(og.gemm_ordered(xq, xs, p["down_codes"], p["down_scales"]))
    h = ok.spine_features_int8(coords, p["spine_codes"], p["spine_scale"], sc, sh, lut)
    hq, hs = oq.quantize_last_dim(h)
    y = og.gemm_ordered(hq, hs, p["up_codes"], p["up_scales"])
    g16 = ok.h(grad_out)
    gq, gs = oq.quantize_last_dim(g16)
    value = ok.h(og.gemm_ordered(gq, gs, *oq.requant_transpose(p["up_codes"], p["up_scales"])))
    coef, _, _ = ok.spine_params(p["spine_codes"], p["spine_scale"], p["warp_scale_codes"],
                                 p["warp_scale_scales"], p["warp_shift_codes"],
                                 p["warp_shift_scales"])
    dc, sums, dcoeff, dscale, dshift = ok.vjp(value, coords, coef, sc, sh, master_raw_scale,
                                              master_raw_shift)
    dcq, dcs = oq.quantize_last_dim(dc)
    dx = og.gemm_ordered(dcq, dcs, *oq.requant_transpose(p["down_codes"], p["down_scales"]))
    dtq, dts = oq.quantize_last_dim(np.ascontiguousarray(dc.T))
    ddown = og.gemm_ordered(dtq, dts, *oq.requant_transpose(xq, xs))
    gtq, gts = oq.quantize_last_dim(np.ascontiguousarray(g16.T))
    dup = og.gemm_ordered(gtq, gts, *oq.requant_transpose(hq, hs))
    return dict(y=y, dx=dx, ddown=ddown, dup=dup, dcoeff=dcoeff, dscale=dscale, dshift=dshift,
                packed=p)


def handoff(t):
    """_grad_handoff (ks3_int8.py:75-84) on values: fp16 when finite, else fp32."""
    t16 = ok.h(t)
    return t16 if np.isfinite(t16).all() else np.asarray(t, np.float32)
