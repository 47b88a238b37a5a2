"""W8A8 GS128 GEMM on the gfx950 int8 matrix cores (mirror of reference ksdraft/kernels/gemm.py).

``w8a8_gemm`` keeps the reference signature, validation and errors (gemm.py:53-90) and
returns fp32 (M, N). The kernel computes, per output element, the ordered per-group
contract acc = fmaf(float(P_g), sa*sw, acc) for g ascending, with P_g the exact int32
group dot product. Shapes with few output tiles (``gemm_splits`` > 1) split the groups into
contiguous parts, each summed that way from zero, and add the parts in order.
``w8a8_gemm_out`` exposes the fused epilogue (fp32 bias, bf16/fp16 output) used by the
linear layer and the KS3 cell.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from .. import _lib
from .quant import GROUP_SIZE, SCALE_DTYPE

_OUT_CODE = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16, torch.float16: _lib.F16}


def _validate(a_codes, a_scales, w_codes, w_scales, group):
    """gemm.py:60-70: the reference's checks, in its order, with its messages."""
    M, K = a_codes.shape
    N = w_codes.shape[0]
    if w_codes.shape[1] != K:
        raise ValueError(f"K mismatch: A {K} vs W {w_codes.shape[1]}")
    n_groups = a_scales.shape[-1]
    if w_scales.shape[-1] != n_groups:
        raise ValueError(
            f"scale group mismatch: A {n_groups} vs W {w_scales.shape[-1]}")
    Kp = n_groups * group
    if Kp < K:
        raise ValueError(f"K {K} exceeds the scales' padded length {Kp}")
    # The reference reads the scales through raw row strides and never checks their rows;
    # here a short scale tensor would send the kernel's loads past its allocation.
    if tuple(a_scales.shape) != (M, n_groups):
        raise ValueError(f"a_scales shape {tuple(a_scales.shape)} != ({M}, {n_groups})")
    if tuple(w_scales.shape) != (N, n_groups):
        raise ValueError(f"w_scales shape {tuple(w_scales.shape)} != ({N}, {n_groups})")
    return M, N, K, n_groups, Kp


def _aligned(t: torch.Tensor) -> torch.Tensor:
    t = t.contiguous()
    if t.data_ptr() % 16:
        t = t.clone()
    return t


def _prepare(a_codes, a_scales, w_codes, w_scales, group):
    M, N, K, n_groups, Kp = _validate(a_codes, a_scales, w_codes, w_scales, group)
    dev = _lib.require_gpu(a_codes, a_scales, w_codes, w_scales)
    if a_codes.dtype != torch.int8 or w_codes.dtype != torch.int8:
        raise TypeError("w8a8_gemm expects int8 codes")
    if a_scales.dtype != SCALE_DTYPE or w_scales.dtype != SCALE_DTYPE:
        raise TypeError("w8a8_gemm expects float16 scales")
    # The kernel steps K by 128. Zero-pad codes (gemm.py:71-73) and, for groups smaller
    # than 128, the scale columns of the padding groups (their codes are zero, so any
    # finite scale leaves the sum unchanged).
    K128 = -(-Kp // 128) * 128
    if K128 != K:
        a_codes = F.pad(a_codes, (0, K128 - K))
        w_codes = F.pad(w_codes, (0, K128 - K))
    g128 = K128 // group
    if g128 != n_groups:
        a_scales = F.pad(a_scales, (0, g128 - n_groups))
        w_scales = F.pad(w_scales, (0, g128 - n_groups))
    return (dev, M, N, K128, _aligned(a_codes), a_scales.contiguous(), _aligned(w_codes),
            w_scales.contiguous())


def w8a8_gemm_out(a_codes: torch.Tensor, a_scales: torch.Tensor, w_codes: torch.Tensor,
                  w_scales: torch.Tensor, group: int = GROUP_SIZE, *,
                  bias: torch.Tensor | None = None, out_dtype: torch.dtype = torch.float32,
                  fp16_saturate: bool = False, out: torch.Tensor | None = None,
                  residual: torch.Tensor | None = None) -> torch.Tensor:
    """(M,K)x(N,K)^T -> (M,N) with the fused epilogue: + bias (fp32) then cast.

    fp16_saturate: fp16 output clamped to +-65504 (ks3_int8.py:241-242).
    residual: (M, N) tensor of the output dtype added in the store, as
    ``residual + (gemm + bias).to(out_dtype)`` computes it (group 128)."""
    dev, M, N, K, a, as_, w, ws = _prepare(a_codes, a_scales, w_codes, w_scales, group)
    if fp16_saturate:
        out_dtype = torch.float16
    code = _lib.F16_SAT if fp16_saturate else _OUT_CODE.get(out_dtype)
    if code is None:
        raise TypeError(f"unsupported output dtype {out_dtype}")
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=dev)
    elif out.shape != (M, N) or out.dtype != out_dtype or not out.is_contiguous():
        raise ValueError("out must be a contiguous (M, N) tensor of the output dtype")
    if bias is not None:
        bias = bias.to(device=dev, dtype=torch.float32).contiguous()
        if bias.numel() != N:
            raise ValueError(f"bias has {bias.numel()} elements, expected {N}")
    if residual is not None:
        if residual.shape != (M, N) or residual.dtype != out_dtype or fp16_saturate:
            raise ValueError("residual must be an (M, N) tensor of the output dtype")
        residual = residual.contiguous()
    if K == 0:
        out.zero_()
        if bias is not None:
            out += bias.to(out_dtype)
        if residual is not None:
            out.copy_(residual + out)
        return out
    splits = gemm_splits(M, N, K, group)
    if splits > 1 or residual is not None:
        # few output tiles: K split into parts, summed in order (fp32 workspace)
        work = (torch.empty(splits * M * N, dtype=torch.float32, device=dev) if splits > 1
                else None)
        _lib.call("ksd_w8a8_gemm_nt_ex", a.data_ptr(), as_.data_ptr(), w.data_ptr(),
                  ws.data_ptr(), M, N, K, group, _lib.ptr(bias), _lib.ptr(residual),
                  out.data_ptr(), code, _lib.ptr(work), 0 if work is None else work.numel() * 4,
                  _lib.stream_ptr(dev))
    else:
        _lib.call("ksd_w8a8_gemm_nt", a.data_ptr(), as_.data_ptr(), w.data_ptr(), ws.data_ptr(),
                  M, N, K, group, _lib.ptr(bias), out.data_ptr(), code, _lib.stream_ptr(dev))
    return out


def w8a8_gemm_pair(first: tuple, second: tuple, group: int = GROUP_SIZE) -> tuple:
    """Two independent GEMMs in one launch: each of ``first`` / ``second`` is
    (a_codes, a_scales, w_codes, w_scales, out_dtype) with out_dtype fp32, bf16 or fp16.
    Returns (y0, y1), each bit-identical to ``w8a8_gemm_out(a, as, w, ws, out_dtype=...)``.
    The launch gives the device's workgroups balanced runs of both GEMMs' tiles (e.g. a
    linear layer's dX, many short tiles, beside its dW, few tiles with K = tokens), where
    two launches would leave CUs idle through the second one's tail. Group 128 only; other
    groups run the two GEMMs one after the other."""
    probs = []
    for a_codes, a_scales, w_codes, w_scales, out_dtype in (first, second):
        dev, M, N, K, a, as_, w, ws = _prepare(a_codes, a_scales, w_codes, w_scales, group)
        code = _OUT_CODE.get(out_dtype)
        if code is None:
            raise TypeError(f"unsupported output dtype {out_dtype}")
        probs.append((dev, M, N, K, a, as_, w, ws, code, out_dtype))
    if group != GROUP_SIZE or any(p[3] == 0 for p in probs):
        return tuple(w8a8_gemm_out(a_codes, a_scales, w_codes, w_scales, group, out_dtype=dt)
                     for a_codes, a_scales, w_codes, w_scales, dt in (first, second))
    dev = probs[0][0]
    if probs[1][0] != dev:
        raise ValueError("w8a8_gemm_pair: both GEMMs must be on one device")
    outs = [torch.empty((M, N), dtype=dt, device=dev) for _, M, N, _, _, _, _, _, _, dt in probs]
    need = sum(gemm_splits(M, N, K) * M * N for _, M, N, K, *_ in probs
               if gemm_splits(M, N, K) > 1)
    work = torch.empty(need, dtype=torch.float32, device=dev) if need else None
    args = []
    for (_, M, N, K, a, as_, w, ws, code, _), y in zip(probs, outs):
        args += [a.data_ptr(), as_.data_ptr(), w.data_ptr(), ws.data_ptr(), M, N, K, y.data_ptr(), code]
    _lib.call("ksd_w8a8_gemm_pair", *args, _lib.ptr(work), 0 if work is None else work.numel() * 4,
              _lib.stream_ptr(dev))
    return outs[0], outs[1]


_SPLITS: dict = {}


def gemm_splits(M: int, N: int, K: int, group: int = GROUP_SIZE) -> int:
    """K parts the GEMM of this shape is split into (a function of the shape; 1 for most
    shapes, more when there are too few 128 x 128 output tiles to fill the device)."""
    key = (M, N, K, group)
    s = _SPLITS.get(key)
    if s is None:
        import ctypes
        c = ctypes.c_int(0)
        _lib.call("ksd_w8a8_gemm_splits", M, N, K, group, ctypes.byref(c))
        s = _SPLITS[key] = c.value
    return s


def w8a8_gemm(a_codes: torch.Tensor, a_scales: torch.Tensor, w_codes: torch.Tensor,
              w_scales: torch.Tensor, group: int = GROUP_SIZE) -> torch.Tensor:
    """(M,K)x(N,K)^T -> (M,N) fp32. Inputs as produced by quantize_last_dim with the
    matching `group` (gemm.py:53-90)."""
    return w8a8_gemm_out(a_codes, a_scales, w_codes, w_scales, group)


def w8a8_group_partials(a_codes: torch.Tensor, w_codes: torch.Tensor,
                        group: int = GROUP_SIZE) -> torch.Tensor:
    """Test-only export of the exact int32 group partials (K/group, M, N) of the GEMM
    (the int32 tl.dot of gemm.py:42), from the same MFMA code path."""
    dev = _lib.require_gpu(a_codes, w_codes)
    M, K = a_codes.shape
    N = w_codes.shape[0]
    if w_codes.shape[1] != K:
        raise ValueError(f"K mismatch: A {K} vs W {w_codes.shape[1]}")
    if K % 128:
        raise ValueError("w8a8_group_partials needs K % 128 == 0")
    a = _aligned(a_codes)
    w = _aligned(w_codes)
    out = torch.empty((K // group, M, N), dtype=torch.int32, device=dev)
    _lib.call("ksd_w8a8_group_partials", a.data_ptr(), w.data_ptr(), M, N, K, group,
              out.data_ptr(), _lib.stream_ptr(dev))
    return out
