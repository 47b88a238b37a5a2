"""All-INT8 KS3 cell on gfx950 (mirror of reference ksdraft/kernels/ks3_int8.py).

Same module surface as the reference: ``TANH_DOMAIN``, ``FP16``, ``make_tanh_lut``,
``_round_div127``, ``_lut_index``, ``_grad_handoff``, ``pack_spine``, ``KS3Int8Cell``
(constructor, buffer names, ``master_*`` parameters, ``_warp_scalars``,
``_spine_features``, ``_project``, ``_repack_masters``, ``_forward_composed``, ``forward``)
and ``_KS3Int8Train``.

Compute runs in libksdraft_amd.so:
  * the down/up projections and the four backward GEMMs: ksd_w8a8_gemm_nt;
  * the composed 'int8' spine + ReLU^2 + requantization: ksd_ks3_spine_fwd (coordinates
    materialised as fp16, ks3_int8.py:241-242, straight from the GEMM epilogue);
  * the fp16 geometry VJP, emitting dc as the two int8 GEMM operands and the eight
    column sums: ksd_ks3_vjp + ksd_ks3_vjp_finalize;
  * the transposed operands: ksd_requant_transpose, and the upstream gradient's fp16
    rounding in both layouts from one pass (ksd_quantize_dual, fp16 mode);
  * the 'fp16' and 'fp32' nonlinear modes (ks3_int8.py:172-203): ksd_ks3_spine_float,
    composed (on the fp16 coordinates) and under the project_fused contract (on the fp32
    accumulator), with the features' requantization in the same pass.
The cell evaluates rank 1 (subspace_rank == 1, the only rank the draft model builds,
model/block.py:32). The reference cannot evaluate a higher rank either: its _project
reshapes the (charts * rank,) packed row scales to (charts,) (ks3_int8.py:253), and its
backward multiplies a (charts * rank,) warp gradient by a (charts,) one (:394-395); here a
rank above 1 raises NotImplementedError (a RuntimeError, as the reference's shape errors
are) at forward time.
"""

from __future__ import annotations

import ctypes

import torch
from torch import nn
import torch.nn.functional as F

from .. import _lib
from .gemm import w8a8_gemm, w8a8_gemm_out, w8a8_gemm_pair
from .quant import (GROUP_SIZE, dequantize_last_dim, quantize_dual, quantize_last_dim,
                    requant_transpose)

TANH_DOMAIN = 3.2
FP16 = torch.float16


def make_tanh_lut(device) -> torch.Tensor:
    """256-entry INT8 tanh table over [-3.2, 3.2] (ks3_int8.py:50-54)."""
    idx = torch.arange(-128, 128, device=device, dtype=torch.float32)
    return (torch.tanh(idx * (TANH_DOMAIN / 127.0)) * 127.0) \
        .round().clamp(-127.0, 127.0).to(torch.int8)


def _round_div127(value: torch.Tensor) -> torch.Tensor:
    """Symmetric round-to-nearest division by 127 (ks3_int8.py:57-66)."""
    quotient = torch.div(value, 127, rounding_mode="trunc")
    remainder = value - quotient * 127
    return quotient + torch.where(remainder > 63, 1,
                                  torch.where(remainder < -63, -1, 0)).to(value.dtype)


def _lut_index(x_fp16: torch.Tensor) -> torch.Tensor:
    """FP16 pre-LUT value -> int32 index into the 256-entry table (ks3_int8.py:69-72)."""
    scaled = torch.clamp(x_fp16, -TANH_DOMAIN, TANH_DOMAIN) * (127.0 / TANH_DOMAIN)
    return torch.round(scaled).to(torch.int32)


def _grad_handoff(t: torch.Tensor) -> torch.Tensor:
    """FP16 gradient handoff with the FP32 overflow fallback (ks3_int8.py:75-84)."""
    t16 = t.to(FP16)
    if bool(torch.isfinite(t16).all()):
        return t16
    return t.float()


def _gpu_quantize(t: torch.Tensor, group: int):
    """quantize_last_dim on the GPU for a tensor that may live on the CPU (module
    construction from a CPU cell): results come back to t's device."""
    if t.device.type == "cuda":
        return quantize_last_dim(t, group)
    if not torch.cuda.is_available():
        raise RuntimeError("ksdraft_amd quantizes on the GPU only (no CPU path)")
    codes, scales = quantize_last_dim(t.cuda(), group)
    return codes.to(t.device), scales.to(t.device)


def pack_spine(coefficients: torch.Tensor, group: int = GROUP_SIZE):
    """(charts*rank, 6) coefficient rows, one scale per row (ks3_int8.py:87-92)."""
    rows = coefficients.reshape(-1, 6)
    codes, scales = _gpu_quantize(rows, group)
    return codes, scales.flatten().to(FP16)


def _c(t: torch.Tensor) -> torch.Tensor:
    return t.contiguous()


def spine_int8(coords16: torch.Tensor, spine_codes: torch.Tensor, spine_scale: torch.Tensor,
               warp_scale16: torch.Tensor, warp_shift16: torch.Tensor, tanh_lut: torch.Tensor,
               group: int = GROUP_SIZE, *, want_h: bool = False, want_codes: bool = True):
    """Composed 'int8' spine (ks3_int8.py:205-234, rank 1) on fp16 coordinates (M, F),
    fused with quantize_last_dim(h, group).

    Returns (h fp32 (M, F) or None, h_codes int8 (M, F) or None, h_scales fp16 or None)."""
    dev = _lib.require_gpu(coords16, spine_codes, spine_scale, warp_scale16, warp_shift16,
                           tanh_lut)
    if coords16.dtype != FP16 or coords16.dim() != 2:
        raise TypeError("coords must be a 2-D float16 tensor")
    M, Fn = coords16.shape
    coords16 = _c(coords16)
    sc = _c(spine_codes.reshape(Fn, 6))
    h = torch.empty((M, Fn), dtype=torch.float32, device=dev) if want_h else None
    hq = torch.empty((M, Fn), dtype=torch.int8, device=dev) if want_codes else None
    hs = (torch.empty((M, -(-Fn // group)), dtype=FP16, device=dev) if want_codes else None)
    table = torch.empty((max(Fn, 1), 256), dtype=FP16, device=dev)   # per-chart increments
    # operands bound to names: a converted temporary must outlive the enqueued kernel
    ps, ws, wh, lut = (_c(spine_scale.reshape(Fn)), _c(warp_scale16.reshape(Fn)),
                       _c(warp_shift16.reshape(Fn)), _c(tanh_lut))
    _lib.call("ksd_ks3_spine_fwd", coords16.data_ptr(), M, Fn, sc.data_ptr(), ps.data_ptr(),
              ws.data_ptr(), wh.data_ptr(), lut.data_ptr(), group,
              _lib.ptr(h), _lib.ptr(hq), _lib.ptr(hs), table.data_ptr(), _lib.stream_ptr(dev))
    return h, hq, hs


def spine_fused_int8(acc: torch.Tensor, spine_codes: torch.Tensor, spine_scale: torch.Tensor,
                     warp_scale16: torch.Tensor, warp_shift16: torch.Tensor,
                     tanh_lut: torch.Tensor, group: int = GROUP_SIZE):
    """The project_fused contract (ks3_triton.py:47-75, 137-156) on the fp32 down-GEMM
    accumulator (M, F): returns (h_codes int8 (M, F), h_scales fp16 (M, ceil(F/group)))."""
    dev = _lib.require_gpu(acc, spine_codes, spine_scale, warp_scale16, warp_shift16, tanh_lut)
    if acc.dtype != torch.float32 or acc.dim() != 2:
        raise TypeError("acc must be a 2-D float32 tensor")
    M, Fn = acc.shape
    acc = _c(acc)
    hq = torch.empty((M, Fn), dtype=torch.int8, device=dev)
    hs = torch.empty((M, -(-Fn // group)), dtype=FP16, device=dev)
    table = torch.empty((max(Fn, 1), 256), dtype=torch.float32, device=dev)
    sc, ps, ws, wh, lut = (_c(spine_codes.reshape(Fn, 6)), _c(spine_scale.reshape(Fn)),
                           _c(warp_scale16.reshape(Fn)), _c(warp_shift16.reshape(Fn)), _c(tanh_lut))
    _lib.call("ksd_ks3_spine_fused", acc.data_ptr(), M, Fn, sc.data_ptr(), ps.data_ptr(),
              ws.data_ptr(), wh.data_ptr(), lut.data_ptr(), group,
              hq.data_ptr(), hs.data_ptr(), table.data_ptr(), _lib.stream_ptr(dev))
    return hq, hs


_MODES = {"fp32": 0, "fp16": 1}


def spine_float(x: torch.Tensor, spine_codes: torch.Tensor, spine_scale: torch.Tensor,
                warp_scale: torch.Tensor, warp_shift: torch.Tensor, nonlinear: str,
                group: int = GROUP_SIZE, *, want_h: bool = False, want_codes: bool = True):
    """The 'fp32' / 'fp16' spine features (ks3_int8.py:172-203, rank 1) fused with
    quantize_last_dim(h, group).

    x: (M, F) float16 coordinates (the composed path) or the float32 down-GEMM
    accumulator (the project_fused contract, clamped to +-65504 in the kernel);
    warp_scale / warp_shift: (F,) values of the arithmetic the path uses (fp32 or fp16),
    passed as fp32. Returns (h fp32 (M, F) or None, h_codes or None, h_scales or None)."""
    dev = _lib.require_gpu(x, spine_codes, spine_scale, warp_scale, warp_shift)
    if nonlinear not in _MODES:
        raise ValueError(f"spine_float implements 'fp32' and 'fp16' (got {nonlinear!r})")
    if x.dim() != 2 or x.dtype not in (FP16, torch.float32):
        raise TypeError("x must be a 2-D float16 or float32 tensor")
    M, Fn = x.shape
    x = _c(x)
    h = torch.empty((M, Fn), dtype=torch.float32, device=dev) if want_h else None
    hq = torch.empty((M, Fn), dtype=torch.int8, device=dev) if want_codes else None
    hs = torch.empty((M, -(-Fn // group)), dtype=FP16, device=dev) if want_codes else None
    # operands bound to names: a converted temporary must outlive the enqueued kernel
    sc, ps = _c(spine_codes.reshape(Fn, 6)), _c(spine_scale.reshape(Fn).to(FP16))
    ws, wh = _c(warp_scale.reshape(Fn).float()), _c(warp_shift.reshape(Fn).float())
    _lib.call("ksd_ks3_spine_float", x.data_ptr(), _lib.dtype_code(x.dtype), M, Fn,
              sc.data_ptr(), ps.data_ptr(), ws.data_ptr(), wh.data_ptr(),
              _MODES[nonlinear], group, _lib.ptr(h), _lib.ptr(hq), _lib.ptr(hs), _lib.stream_ptr(dev))
    return h, hq, hs


def ks3_vjp(value16: torch.Tensor, coords16: torch.Tensor, spine_codes: torch.Tensor,
            spine_scale: torch.Tensor, warp_scale16: torch.Tensor, warp_shift16: torch.Tensor,
            warp_scale_raw: torch.Tensor, warp_shift_raw: torch.Tensor,
            group: int = GROUP_SIZE, *, want_dc: bool = False, want_sums: bool = False):
    """fp16 geometry VJP of _KS3Int8Train.backward (ks3_int8.py:354-401), rank 1.

    Returns a dict with dc_codes/dc_scales (quantize_last_dim(dc)), dct_codes/dct_scales
    (quantize_last_dim(dc.t())), dcoeff (F, 6) fp16, dscale (F,) fp16, dshift (F,) fp16,
    and, on request, dc (M, F) fp16 and the fp32 column sums (8, F)."""
    dev = _lib.require_gpu(value16, coords16, spine_codes, spine_scale, warp_scale16,
                           warp_shift16, warp_scale_raw, warp_shift_raw)
    if value16.dtype != FP16 or coords16.dtype != FP16:
        raise TypeError("value and coords must be float16")
    M, Fn = coords16.shape
    if value16.shape != (M, Fn):
        raise ValueError(f"value shape {tuple(value16.shape)} != coords shape {(M, Fn)}")
    nrb_c = ctypes.c_int64(0)
    _lib.call("ksd_ks3_vjp_row_blocks", M, ctypes.byref(nrb_c))
    nrb = nrb_c.value
    f16 = dict(dtype=FP16, device=dev)
    out = {
        "dc": torch.empty((M, Fn), **f16) if want_dc else None,
        "dc_codes": torch.empty((M, Fn), dtype=torch.int8, device=dev),
        "dc_scales": torch.empty((M, -(-Fn // group)), **f16),
        "dct_codes": torch.empty((Fn, M), dtype=torch.int8, device=dev),
        "dct_scales": torch.empty((Fn, -(-M // group)), **f16),
        "sums": torch.empty((8, Fn), dtype=torch.float32, device=dev) if want_sums else None,
        "dcoeff": torch.empty((Fn, 6), **f16),
        "dscale": torch.empty((Fn,), **f16),
        "dshift": torch.empty((Fn,), **f16),
    }
    if M == 0 or Fn == 0:
        for k in ("dcoeff", "dscale", "dshift"):
            out[k].zero_()
        if out["sums"] is not None:
            out["sums"].zero_()
        return out
    partials = torch.empty((nrb, 8, Fn), dtype=torch.float32, device=dev)
    st = _lib.stream_ptr(dev)
    # operands bound to names: a converted temporary must outlive the enqueued kernel
    sc16, sh16 = _c(warp_scale16.reshape(Fn)), _c(warp_shift16.reshape(Fn))
    v16, c16 = _c(value16), _c(coords16)
    scd, ps = _c(spine_codes.reshape(Fn, 6)), _c(spine_scale.reshape(Fn))
    _lib.call("ksd_ks3_vjp", v16.data_ptr(), c16.data_ptr(), M, Fn, scd.data_ptr(), ps.data_ptr(),
              sc16.data_ptr(), sh16.data_ptr(), group, _lib.ptr(out["dc"]),
              out["dc_codes"].data_ptr(), out["dc_scales"].data_ptr(), out["dct_codes"].data_ptr(),
              out["dct_scales"].data_ptr(), partials.data_ptr(), nrb, st)
    rs = _c(warp_scale_raw.reshape(Fn).float())
    rh = _c(warp_shift_raw.reshape(Fn).float())
    _lib.call("ksd_ks3_vjp_finalize", partials.data_ptr(), nrb, Fn, rs.data_ptr(), rh.data_ptr(),
              _lib.ptr(out["sums"]), out["dcoeff"].data_ptr(), out["dscale"].data_ptr(),
              out["dshift"].data_ptr(), st)
    return out


def tanh16(x: torch.Tensor) -> torch.Tensor:
    """Test export: fp16 tanh through the VJP's table (torch.tanh on fp16 tensors)."""
    dev = _lib.require_gpu(x)
    if x.dtype != FP16:
        raise TypeError("tanh16 expects float16")
    x = _c(x)
    y = torch.empty_like(x)
    _lib.call("ksd_ks3_tanh16", x.data_ptr(), x.numel(), y.data_ptr(), _lib.stream_ptr(dev))
    return y


class KS3Int8Cell(nn.Module):
    """W8A8 GS-group KS3 with all-INT8 runtime (ks3_int8.py:95-314).

    Built from a torch KS3 cell (``ksdraft.model.ks3.KS3`` or anything with its
    attributes); ``trainable=True`` owns fp32 masters and repacks every forward."""

    def __init__(self, cell, group: int = GROUP_SIZE, nonlinear: str = "int8",
                 *, trainable: bool = False):
        super().__init__()
        if nonlinear not in ("fp32", "fp16", "int8"):
            raise ValueError("nonlinear must be fp32, fp16 or int8")
        self.group = group
        self.nonlinear = nonlinear
        self.num_subspaces = cell.num_charts
        self.subspace_rank = cell.subspace_rank
        self.in_features = cell.down.weight.shape[1]
        self.out_features = cell.up.weight.shape[0]
        features = self.num_subspaces * self.subspace_rank
        if cell.down.weight.shape[0] != features or cell.up.weight.shape[1] != features:
            raise ValueError("Projection shapes do not match subspace count and rank")

        down = cell.down.weight.detach().float()
        up = cell.up.weight.detach().float()
        coeffs = cell.coefficients.detach().reshape(
            self.num_subspaces, self.subspace_rank, 6)
        raw_scale = cell.raw_scale.detach().float().reshape(self.num_subspaces)
        raw_shift = cell.raw_shift.detach().float().reshape(self.num_subspaces)

        dq, ds = _gpu_quantize(down, group)
        uq, us = _gpu_quantize(up, group)
        self.register_buffer("down_codes", dq)
        self.register_buffer("down_scales", ds)
        self.register_buffer("up_codes", uq)
        self.register_buffer("up_scales", us)
        sq, ss = pack_spine(coeffs, group)
        self.register_buffer("spine_codes", sq)
        self.register_buffer("spine_scale", ss)

        self.register_buffer("warp_scale_raw", raw_scale)
        self.register_buffer("warp_shift_raw", raw_shift)
        scale_t = F.softplus(raw_scale) + 1e-4
        shift_t = 0.5 * torch.tanh(raw_shift)
        wsc, wss = _gpu_quantize(scale_t.reshape(-1, 1), group)
        whc, whs = _gpu_quantize(shift_t.reshape(-1, 1), group)
        self.register_buffer("warp_scale_codes", wsc)
        self.register_buffer("warp_scale_scales", wss)
        self.register_buffer("warp_shift_codes", whc)
        self.register_buffer("warp_shift_scales", whs)

        self.register_buffer("tanh_lut", make_tanh_lut(down.device))
        self.trainable = trainable
        self._master_codes_keys = {}  # master name -> (storage, version) its codes came from
        self._master_t = {}  # master name -> ((codes_t, scales_t), the codes they came from)
        if trainable:
            for name, value in (("down", down), ("up", up),
                                ("coefficients", coeffs),
                                ("raw_scale", raw_scale), ("raw_shift", raw_shift)):
                setattr(self, "master_" + name, nn.Parameter(value.clone()))

    # ---- scalar dequantization into the active arithmetic domain ----

    def _warp_scalars(self, dtype: torch.dtype):
        """ks3_int8.py:158-165. Kept per dtype while the four warp code/scale tensors are
        the same objects at the same in-place version (the cache holds them, so their
        storage cannot be reused under it): a training step dequantizes them once, not in
        its forward and again in its backward. Inference tensors (made under
        torch.inference_mode) carry no version counter: with any of those the scalars are
        dequantized every call and nothing is cached. The returned tensors are not to be
        modified."""
        src = (self.warp_scale_codes, self.warp_scale_scales, self.warp_shift_codes,
               self.warp_shift_scales)
        cacheable = not any(t.is_inference() for t in src)
        cache = getattr(self, "_warp_cache", None)
        if cache is None:
            cache = self._warp_cache = {}
        hit = cache.get(dtype) if cacheable else None
        if (hit is not None and all(a is b for a, b in zip(hit[0], src))
                and hit[1] == tuple(t._version for t in src)):
            return hit[2]
        scale = dequantize_last_dim(self.warp_scale_codes, self.warp_scale_scales,
                                    self.group).reshape(-1).to(dtype)
        shift = dequantize_last_dim(self.warp_shift_codes, self.warp_shift_scales,
                                    self.group).reshape(-1).to(dtype)
        if cacheable:
            cache[dtype] = (src, tuple(t._version for t in src), (scale, shift))
        else:
            cache.pop(dtype, None)
        return scale, shift

    def _check_supported(self):
        if self.subspace_rank != 1:
            raise NotImplementedError(
                "KS3Int8Cell evaluates subspace_rank 1; the reference cell fails for a higher "
                "rank too (ks3_int8.py:253 reshapes the (charts*rank,) row scales to (charts,))")

    def _arith(self):
        return torch.float32 if self.nonlinear == "fp32" else FP16

    def _spine(self, coords16, scale, shift, *, want_h=False, want_codes=True):
        """The composed spine of this cell's mode on fp16 coordinates (M, F)."""
        if self.nonlinear == "int8":
            return spine_int8(coords16, self.spine_codes, self.spine_scale, scale.to(FP16),
                              shift.to(FP16), self.tanh_lut, self.group, want_h=want_h,
                              want_codes=want_codes)
        return spine_float(coords16, self.spine_codes, self.spine_scale, scale, shift,
                           self.nonlinear, self.group, want_h=want_h, want_codes=want_codes)

    def _spine_features(self, x, mean, c0, c1, c2, c3, c4, c5, ps, scale, shift):
        """ks3_int8.py:167-234. x/mean (..., charts, 1) fp32 holding fp16 values (the
        coordinates _project materialises); c* int8 codes (charts, 1); ps (charts,) fp16;
        scale/shift (charts,) in the mode's arithmetic (fp32 for 'fp32', else fp16).
        Returns the fp32 ReLU^2 features shaped like x."""
        self._check_supported()
        lead = x.shape
        Fn = self.num_subspaces
        codes = torch.stack([c.reshape(Fn) for c in (c0, c1, c2, c3, c4, c5)], -1).to(torch.int8)
        coords16 = x.reshape(-1, Fn).to(FP16)
        if self.nonlinear == "int8":
            h, _, _ = spine_int8(coords16, codes, ps.to(FP16), scale.to(FP16), shift.to(FP16),
                                 self.tanh_lut, self.group, want_h=True, want_codes=False)
        else:
            h, _, _ = spine_float(coords16, codes, ps.to(FP16), scale, shift, self.nonlinear,
                                  self.group, want_h=True, want_codes=False)
        return h.reshape(lead)

    def _coords16(self, xq, xs, down_codes, down_scales):
        """fp16(GEMM(x, down)).clamp(+-65504) from the GEMM epilogue (ks3_int8.py:241-242)."""
        return w8a8_gemm_out(xq, xs, down_codes, down_scales, self.group, fp16_saturate=True)

    def _project(self, x, codes, scales, down_codes, down_scales):
        """ks3_int8.py:238-260: (h (M, F) fp32, coords (M, F, 1) fp32)."""
        self._check_supported()
        M = x.shape[0]
        coords16 = self._coords16(codes, scales, down_codes, down_scales)
        scale, shift = self._warp_scalars(self._arith())
        h, _, _ = self._spine(coords16, scale, shift, want_h=True, want_codes=False)
        return h.reshape(M, -1), coords16.float().reshape(M, self.num_subspaces,
                                                          self.subspace_rank)

    def _project_codes(self, xq, xs):
        """_project + quantize_last_dim(h) in two kernels: (hq, hs, coords16)."""
        self._check_supported()
        coords16 = self._coords16(xq, xs, self.down_codes, self.down_scales)
        scale, shift = self._warp_scalars(self._arith())
        _, hq, hs = self._spine(coords16, scale, shift)
        return hq, hs, coords16

    def invalidate_codes(self) -> None:
        """Forget down/up codes handed over by an optimizer (train.AdamWRequant): the next
        forward requantizes the masters. Needed after a write to a master that torch does
        not version (through ``.data`` or a raw pointer)."""
        self._master_codes_keys = {}

    def _apply(self, fn, *args, **kwargs):
        self.invalidate_codes()
        return super()._apply(fn, *args, **kwargs)

    def _load_from_state_dict(self, *args, **kwargs):
        self.invalidate_codes()
        return super()._load_from_state_dict(*args, **kwargs)

    def current_transpose(self, name: str):
        """requant_transpose of the down or up codes (a backward GEMM's operand) when the
        optimizer built it for the codes the cell holds now, else None."""
        ent = (getattr(self, "_master_t", None) or {}).get(name)
        if ent is None or ent[1] is not getattr(self, name + "_codes"):
            return None
        return ent[0]

    def _master_codes_current(self, name: str) -> bool:
        """True when train.AdamWRequant wrote `name`'s codes in the pass that last updated
        the master, and the master has kept its storage and in-place version since."""
        keys = getattr(self, "_master_codes_keys", None) or {}
        m = getattr(self, "master_" + name)
        return (getattr(self, "_codes_owner", None) is not None
                and keys.get(name) == (m.data_ptr(), m._version))

    @torch.no_grad()
    def _repack_masters(self):
        """ks3_int8.py:262-277. The down/up codes are skipped when the optimizer already
        wrote them from the masters as they are (the same quantize_last_dim)."""
        if not self._master_codes_current("down"):
            self.down_codes, self.down_scales = quantize_last_dim(self.master_down, self.group)
        if not self._master_codes_current("up"):
            self.up_codes, self.up_scales = quantize_last_dim(self.master_up, self.group)
        sq, ss = pack_spine(self.master_coefficients, self.group)
        self.spine_codes, self.spine_scale = sq, ss
        scale_t = F.softplus(self.master_raw_scale.detach()) + 1e-4
        shift_t = 0.5 * torch.tanh(self.master_raw_shift.detach())
        wsc, wss = quantize_last_dim(scale_t.reshape(-1, 1), self.group)
        whc, whs = quantize_last_dim(shift_t.reshape(-1, 1), self.group)
        self.warp_scale_codes, self.warp_scale_scales = wsc, wss
        self.warp_shift_codes, self.warp_shift_scales = whc, whs
        self.warp_scale_raw = self.master_raw_scale.detach()
        self.warp_shift_raw = self.master_raw_shift.detach()

    def _out_dtype(self, x):
        return (torch.get_autocast_gpu_dtype()
                if torch.is_autocast_enabled("cuda") else x.dtype)

    def _forward_composed(self, x: torch.Tensor) -> torch.Tensor:
        """The composed path (ks3_int8.py:279-288)."""
        x2 = x.reshape(-1, x.shape[-1])
        xq, xs = quantize_last_dim(x2.float(), self.group)
        hq, hs, _ = self._project_codes(xq, xs)
        y = w8a8_gemm(hq, hs, self.up_codes, self.up_scales, self.group)
        return y.reshape(*x.shape[:-1], self.out_features).to(self._out_dtype(x))

    def forward(self, x: torch.Tensor, residual: torch.Tensor | None = None) -> torch.Tensor:
        """ks3_int8.py:290-314: trainable -> _KS3Int8Train; eval on the GPU -> the fused
        (project_fused) contract. With ``residual`` (shaped like the output, of its dtype)
        the result is residual + cell(x), the add done in the up-projection's store."""
        out_dt = self._out_dtype(x)
        fuse = (residual is not None and residual.dtype == out_dt
                and out_dt in (torch.float32, torch.bfloat16, torch.float16))
        if self.trainable:
            y = _KS3Int8Train.apply(
                x, self.master_down, self.master_up, self.master_coefficients,
                self.master_raw_scale, self.master_raw_shift, self, residual if fuse else None)
            return y if fuse or residual is None else residual + y
        self._check_supported()
        x2 = x.reshape(-1, x.shape[-1])
        xq, xs = quantize_last_dim(x2.float(), self.group)
        from .ks3_triton import project_fused
        scale_dq, shift_dq = self._warp_scalars(FP16)
        hq, hs = project_fused(
            xq, xs, self.down_codes, self.down_scales,
            self.spine_codes, self.spine_scale,
            scale_dq.reshape(-1), shift_dq.reshape(-1),
            self.tanh_lut, self.group, self.nonlinear)
        if fuse:
            y = w8a8_gemm_out(hq, hs, self.up_codes, self.up_scales, self.group, out_dtype=out_dt,
                              residual=residual.reshape(-1, self.out_features))
            return y.reshape(*x.shape[:-1], self.out_features)
        y = w8a8_gemm(hq, hs, self.up_codes, self.up_scales, self.group)
        y = y.reshape(*x.shape[:-1], self.out_features).to(out_dt)
        return y if residual is None else residual + y


def grad_handoff_device(t: torch.Tensor) -> torch.Tensor:
    """The values _grad_handoff hands to autograd for an fp32 master (ks3_int8.py:75-84),
    as fp32, without reading anything back to the host: fp16(t) when every element of it is
    finite, else t (ksd_grad_handoff, decided on the device)."""
    dev = _lib.require_gpu(t)
    t = _c(t.float())
    flag = torch.zeros(1, dtype=torch.int32, device=dev)
    out = torch.empty_like(t)
    _lib.call("ksd_grad_handoff", t.data_ptr(), t.numel(), flag.data_ptr(), out.data_ptr(),
              _lib.stream_ptr(dev))
    return out


class _KS3Int8Train(torch.autograd.Function):
    """Training forward/backward of the all-INT8 cell (ks3_int8.py:317-429): INT8 GEMMs,
    fp16 geometry VJP, fp16 gradient handoff."""

    @staticmethod
    def forward(ctx, inputs, down, up, coefficients, raw_scale, raw_shift, cell, residual=None):
        cell._repack_masters()
        x = inputs.reshape(-1, inputs.shape[-1]).float()
        xq, xs = quantize_last_dim(x, cell.group)
        hq, hs, coords16 = cell._project_codes(xq, xs)
        out_dt = cell._out_dtype(inputs)
        if residual is not None:  # residual + y, added in the up-projection's store
            y = w8a8_gemm_out(hq, hs, cell.up_codes, cell.up_scales, cell.group, out_dtype=out_dt,
                              residual=residual.reshape(-1, cell.out_features))
        else:
            y = w8a8_gemm(hq, hs, cell.up_codes, cell.up_scales, cell.group)
        ctx.cell = cell
        ctx.input_shape = inputs.shape
        ctx.has_residual = residual is not None
        ctx.save_for_backward(xq, xs, hq, hs, coords16)
        return y.reshape(*inputs.shape[:-1], cell.out_features).to(out_dt)

    @staticmethod
    def backward(ctx, grad_out):
        cell = ctx.cell
        group = cell.group
        xq, xs, hq, hs, coords16 = ctx.saved_tensors
        # g16 = grad.to(fp16) in both int8 layouts, from one pass over the gradient: along
        # the features for the value GEMM (ks3_int8.py:345-348) and along the tokens for
        # dup (:421-422)
        gq, gs, gT_q, gT_s = quantize_dual(grad_out.reshape(-1, cell.out_features), group,
                                           round_fp16=True)

        # output-projection backward GEMM (ks3_int8.py:345-352), launched with dup (its
        # operands are ready already; ks3_int8.py:421-424)
        upT_q, upT_s = (cell.current_transpose("up")
                        or requant_transpose(cell.up_codes, cell.up_scales, group, group))
        hT_q, hT_s = requant_transpose(hq, hs, group, group)
        value, dup = w8a8_gemm_pair((gq, gs, upT_q, upT_s, FP16),
                                    (gT_q, gT_s, hT_q, hT_s, torch.float32), group)
        dup = grad_handoff_device(dup)

        # geometry VJP (ks3_int8.py:354-401) -> dc in both int8 layouts + column sums
        scale, shift = cell._warp_scalars(FP16)
        v = ks3_vjp(value, coords16, cell.spine_codes, cell.spine_scale, scale, shift,
                    cell.warp_scale_raw, cell.warp_shift_raw, group)
        dcoeff = v["dcoeff"].reshape(cell.num_subspaces, cell.subspace_rank, 6)

        # INT8 backward GEMMs (ks3_int8.py:403-424)
        downT_q, downT_s = (cell.current_transpose("down")
                            or requant_transpose(cell.down_codes, cell.down_scales, group, group))
        dx_dtype = grad_out.dtype if grad_out.dtype in (torch.float32, torch.bfloat16,
                                                        torch.float16) else torch.float32
        xT_q, xT_s = requant_transpose(xq, xs, group, group)
        dx, ddown = w8a8_gemm_pair((v["dc_codes"], v["dc_scales"], downT_q, downT_s, dx_dtype),
                                   (v["dct_codes"], v["dct_scales"], xT_q, xT_s, torch.float32),
                                   group)
        ddown = grad_handoff_device(ddown)

        dx = dx.reshape(ctx.input_shape).to(grad_out.dtype)
        dres = grad_out if ctx.has_residual and ctx.needs_input_grad[7] else None
        # dcoeff / dscale / dshift are fp16 already: _grad_handoff would return them (or,
        # with a non-finite entry, the same values as fp32), and autograd casts to fp32
        return (dx, ddown, dup, dcoeff, v["dscale"], v["dshift"], None, dres)
