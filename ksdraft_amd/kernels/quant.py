"""GS128 symmetric INT8 quantization on gfx950 (mirror of reference ksdraft/kernels/quant.py).

Contract (quant.py:1-17): symmetric per-group scales along the quantized dimension,
group 128 by default; scales stored fp16, rounded BEFORE encoding and bounded to
[2**-24, 65504]; codes saturate to [-127, 127] with round-half-even; a partial last group
is zero-padded and its padded lanes are dropped from the codes.

Every function runs one HIP kernel from libksdraft_amd.so on the tensor's current
stream. There is no CPU path: CPU tensors raise after the reference's own argument
checks (so its TypeError/ValueError conditions are identical on any device).
"""

from __future__ import annotations

import torch

from .. import _lib

GROUP_SIZE = 128
SCALE_DTYPE = torch.float16
SCALE_MIN = 2.0 ** -24
SCALE_MAX = 65504.0


def _padded_length(n: int, group: int = GROUP_SIZE) -> int:
    """quant.py:26-27."""
    return (n + group - 1) // group * group


def _float_input(x: torch.Tensor) -> torch.Tensor:
    if not torch.is_floating_point(x):
        raise TypeError("quantize expects floating-point input")
    if x.dtype == torch.float64:
        raise TypeError("ksdraft_amd quantizes float32/bfloat16/float16 input (got float64)")
    return x


def _quantize(x: torch.Tensor, group: int, noise: torch.Tensor | None, dither: float):
    x = _float_input(x)
    if group not in (32, 64, 128):
        raise ValueError(f"group must be 32, 64 or 128, got {group}")
    dev = _lib.require_gpu(x)
    K = x.shape[-1]
    lead = x.shape[:-1]
    x2 = x.reshape(-1, K) if K else x.reshape(-1, 0)
    rows = x2.shape[0]
    # rows may be strided (a view), elements within a row must be dense
    if K and (x2.stride(-1) != 1 or (rows > 1 and x2.stride(0) < K)):
        x2 = x2.contiguous()
    ng = -(-K // group) if group > 0 else 0
    codes = torch.empty((rows, K), dtype=torch.int8, device=dev)
    scales = torch.empty((rows, ng), dtype=SCALE_DTYPE, device=dev)
    noise_ptr = None
    if noise is not None:
        noise = noise.to(device=dev, dtype=torch.float32).contiguous()
        if noise.numel() != rows * ng * group:
            raise ValueError("dither noise must cover the padded grouped shape")
        noise_ptr = noise.data_ptr()
    stride = x2.stride(0) if rows > 1 else K
    _lib.call("ksd_quantize_lastdim", x2.data_ptr(), _lib.dtype_code(x2.dtype), rows, K,
              stride, group, codes.data_ptr(), scales.data_ptr(), noise_ptr,
              float(2.0 * dither), _lib.stream_ptr(dev))
    return codes.reshape(*lead, K), scales.reshape(*lead, ng)


def quantize_last_dim(x: torch.Tensor, group: int = GROUP_SIZE):
    """x (..., K) fp -> (codes int8 (..., K), scales fp16 (..., Kp/group)). quant.py:30-52."""
    return _quantize(x, group, None, 0.0)


def quantize_last_dim_dithered(x: torch.Tensor, group: int, dither: float,
                               generator: torch.Generator | None = None):
    """Rounding-dither variant (reference ksdraft/train/stages.py:27-50).

    The uniform draws come from torch.rand over the padded grouped shape on x's device
    with `generator`, exactly the reference's RNG call, so codes are bit-identical for
    identical generator state. dither == 0 is the exact grid (stages.py:43)."""
    _float_input(x)
    if dither > 0:
        K = x.shape[-1]
        Kp = _padded_length(K, group)
        rows = x.numel() // K if K else 0
        noise = torch.rand((rows, Kp), generator=generator, device=x.device,
                           dtype=torch.float32)
        return _quantize(x, group, noise, dither)
    return _quantize(x, group, None, 0.0)


def dequantize_last_dim(codes: torch.Tensor, scales: torch.Tensor,
                        group: int | None = None) -> torch.Tensor:
    """Inverse of quantize_last_dim, fp32 out (quant.py:55-67).

    Keeps the reference's group inference: group = _padded_length(K) // n_scales."""
    K = codes.shape[-1]
    if group is None:
        group = _padded_length(K) // max(scales.shape[-1], 1)
    if group <= 0:
        raise ValueError(f"dequantize: group must be positive, got {group}")
    lead = codes.shape[:-1]
    # quant.py:64-67 multiplies codes grouped (..., Kp/group, group) by scales[..., None]:
    # torch broadcasting decides which scale shapes are accepted (a single scale row or
    # column broadcasts). Any other shape raises torch's own error, never reads past the
    # scales.
    nsc = _padded_length(K, group) // group
    want = (*lead, nsc)
    if torch.broadcast_shapes(want, tuple(scales.shape)) != want:
        raise RuntimeError(f"scales of shape {tuple(scales.shape)} do not broadcast to the "
                           f"grouped codes {want}")
    dev = _lib.require_gpu(codes, scales)
    if codes.dtype != torch.int8:
        codes = codes.to(torch.int8)  # float-typed integral codes (linear.py:79-80)
    if scales.dtype != SCALE_DTYPE:
        raise TypeError(f"scales must be {SCALE_DTYPE}, got {scales.dtype}")
    c2 = codes.reshape(-1, K).contiguous() if K else codes.reshape(-1, 0)
    s2 = scales.expand(want).reshape(-1, nsc).contiguous()
    out = torch.empty((c2.shape[0], K), dtype=torch.float32, device=dev)
    _lib.call("ksd_dequantize_lastdim", c2.data_ptr(), s2.data_ptr(), c2.shape[0], K, nsc,
              group, out.data_ptr(), _lib.stream_ptr(dev))
    return out.reshape(*lead, K)


def quantize_transpose(x: torch.Tensor, group: int = GROUP_SIZE):
    """quantize_last_dim(x.t().contiguous(), group) for a 2-D x (R, C), without the copy.

    Returns (codes (C, R) int8, scales (C, ceil(R/group)) fp16). Builds the dW operands
    of reference ksdraft/kernels/ks3_int8.py:418, 422."""
    x = _float_input(x)
    dev = _lib.require_gpu(x)
    if x.dim() != 2:
        raise ValueError("quantize_transpose expects a 2-D tensor")
    x = x.contiguous()
    R, C = x.shape
    codes = torch.empty((C, R), dtype=torch.int8, device=dev)
    scales = torch.empty((C, -(-R // group)), dtype=SCALE_DTYPE, device=dev)
    _lib.call("ksd_quantize_transpose", x.data_ptr(), _lib.dtype_code(x.dtype), R, C, group,
              codes.data_ptr(), scales.data_ptr(), _lib.stream_ptr(dev))
    return codes, scales


def quantize_dual(x: torch.Tensor, group: int = GROUP_SIZE, t_from_codes: bool = False,
                  round_fp16: bool = False):
    """Both operand layouts of a 2-D x (R, C) from one read of x.

    Returns (codes (R, C), scales (R, ceil(C/group)), codes_t (C, R), scales_t
    (C, ceil(R/group))): codes/scales = quantize_last_dim(x, group); codes_t/scales_t =
    quantize_transpose(x, group), or with ``t_from_codes`` requant_transpose(codes,
    scales) (the double-quant recipe of reference ksdraft/kernels/ks3_int8.py:417-420).
    ``round_fp16``: both layouts of x.to(float16) (the KS3 backward's g16, ks3_int8.py:
    345-348, 421-422), rounded inside the same pass where the fused kernel applies."""
    x = _float_input(x)
    dev = _lib.require_gpu(x)
    if x.dim() != 2:
        raise ValueError("quantize_dual expects a 2-D tensor")
    if round_fp16 and t_from_codes:
        raise ValueError("quantize_dual: round_fp16 and t_from_codes are exclusive")
    x = x.contiguous()
    R, C = x.shape
    mode = 1 if t_from_codes else 0
    if round_fp16:
        if group == GROUP_SIZE and C % 8 == 0 and x.dtype != torch.float16:
            mode = 2
        else:
            x = x.to(torch.float16)
    codes = torch.empty((R, C), dtype=torch.int8, device=dev)
    scales = torch.empty((R, -(-C // group)), dtype=SCALE_DTYPE, device=dev)
    codes_t = torch.empty((C, R), dtype=torch.int8, device=dev)
    scales_t = torch.empty((C, -(-R // group)), dtype=SCALE_DTYPE, device=dev)
    _lib.call("ksd_quantize_dual", x.data_ptr(), _lib.dtype_code(x.dtype), R, C, group,
              mode, codes.data_ptr(), scales.data_ptr(), codes_t.data_ptr(),
              scales_t.data_ptr(), _lib.stream_ptr(dev))
    return codes, scales, codes_t, scales_t


def quantize_dual2(a: torch.Tensor, b: torch.Tensor, group: int = GROUP_SIZE):
    """quantize_dual(a, group, t_from_codes=True) and the same of b in one launch (two
    2-D tensors of one dtype, e.g. a layer's weight and its input): returns the two
    4-tuples (codes, scales, codes_t, scales_t)."""
    a = _float_input(a)
    b = _float_input(b)
    dev = _lib.require_gpu(a, b)
    if a.dim() != 2 or b.dim() != 2:
        raise ValueError("quantize_dual2 expects 2-D tensors")
    if a.dtype != b.dtype or group != GROUP_SIZE:
        return (quantize_dual(a, group, t_from_codes=True),
                quantize_dual(b, group, t_from_codes=True))
    xs = (a.contiguous(), b.contiguous())  # bound: they must outlive the enqueued kernel
    outs, args = [], []
    for x in xs:
        R, C = x.shape
        o = (torch.empty((R, C), dtype=torch.int8, device=dev),
             torch.empty((R, -(-C // group)), dtype=SCALE_DTYPE, device=dev),
             torch.empty((C, R), dtype=torch.int8, device=dev),
             torch.empty((C, -(-R // group)), dtype=SCALE_DTYPE, device=dev))
        outs.append(o)
        args += [x.data_ptr(), R, C, *(t.data_ptr() for t in o)]
    _lib.call("ksd_quantize_dual2", *args, _lib.dtype_code(a.dtype), group, _lib.stream_ptr(dev))
    return outs[0], outs[1]


def quantize_dual_colsum(g: torch.Tensor, group: int = GROUP_SIZE):
    """quantize_dual(g, group) plus the column sums g.float().sum(0) (a linear layer's bias
    gradient) from the same read of g: (codes, scales, codes_t, scales_t, colsum). The
    column sums run in another order than torch's sum (fp32, within rounding). Falls back to
    quantize_dual + torch's sum where the fused kernel does not apply (group other than 128,
    C % 8 != 0, no rows)."""
    g = _float_input(g)
    dev = _lib.require_gpu(g)
    if g.dim() != 2:
        raise ValueError("quantize_dual_colsum expects a 2-D tensor")
    g = g.contiguous()
    R, C = g.shape
    esz = g.element_size()
    if group != GROUP_SIZE or C % 8 or R == 0 or C == 0 or g.data_ptr() % 16 or (C * esz) % 16:
        return (*quantize_dual(g, group), g.float().sum(0))
    codes = torch.empty((R, C), dtype=torch.int8, device=dev)
    scales = torch.empty((R, -(-C // group)), dtype=SCALE_DTYPE, device=dev)
    codes_t = torch.empty((C, R), dtype=torch.int8, device=dev)
    scales_t = torch.empty((C, -(-R // group)), dtype=SCALE_DTYPE, device=dev)
    colsum = torch.empty(C, dtype=torch.float32, device=dev)
    work = torch.empty(-(-R // 128) * C, dtype=torch.float32, device=dev)
    _lib.call("ksd_quantize_dual_colsum", g.data_ptr(), _lib.dtype_code(g.dtype), R, C, group,
              codes.data_ptr(), scales.data_ptr(), codes_t.data_ptr(), scales_t.data_ptr(),
              colsum.data_ptr(), work.data_ptr(), work.numel() * 4, _lib.stream_ptr(dev))
    return codes, scales, codes_t, scales_t, colsum


def requant_transpose(codes: torch.Tensor, scales: torch.Tensor,
                      group_in: int = GROUP_SIZE, group: int = GROUP_SIZE):
    """quantize_last_dim(dequantize_last_dim(codes, scales).t(), group) in one pass.

    The dequantize -> transpose -> requantize operand builds of reference
    ksdraft/kernels/ks3_int8.py:349-351, 407-408, 417-419, 423."""
    dev = _lib.require_gpu(codes, scales)
    if codes.dim() != 2 or codes.dtype != torch.int8:
        raise ValueError("requant_transpose expects 2-D int8 codes")
    codes = codes.contiguous()
    scales = scales.contiguous()
    R, C = codes.shape
    if scales.shape != (R, -(-C // group_in)):
        raise ValueError(f"scales shape {tuple(scales.shape)} does not match codes {R}x{C} "
                         f"with group {group_in}")
    out_c = torch.empty((C, R), dtype=torch.int8, device=dev)
    out_s = torch.empty((C, -(-R // group)), dtype=SCALE_DTYPE, device=dev)
    _lib.call("ksd_requant_transpose", codes.data_ptr(), scales.data_ptr(), R, C, group_in,
              group, out_c.data_ptr(), out_s.data_ptr(), _lib.stream_ptr(dev))
    return out_c, out_s


def requant_transpose_multi(pairs, group: int = GROUP_SIZE):
    """requant_transpose(codes, scales, group, group) of every (codes, scales) pair in a few
    launches (ksd_requant_transpose_multi); returns the (codes_t, scales_t) pairs in order.
    Built for the weight transposes of a whole model after an optimizer step."""
    import numpy as np
    if not pairs:
        return []
    if group != GROUP_SIZE:
        raise ValueError(f"requant_transpose_multi supports group {GROUP_SIZE} only")
    dev = _lib.require_gpu(*[t for pr in pairs for t in pr])
    arr = np.zeros(len(pairs), dtype=np.dtype([("codes", "<u8"), ("scales", "<u8"), ("R", "<i8"),
                                               ("C", "<i8"), ("codes_t", "<u8"), ("scales_t", "<u8")]))
    out, keep = [], []
    for i, (codes, scales) in enumerate(pairs):
        if codes.dim() != 2 or codes.dtype != torch.int8:
            raise ValueError("requant_transpose_multi expects 2-D int8 codes")
        codes, scales = codes.contiguous(), scales.contiguous()
        R, C = codes.shape
        if scales.shape != (R, -(-C // group)):
            raise ValueError(f"scales shape {tuple(scales.shape)} does not match codes {R}x{C}")
        oc = torch.empty((C, R), dtype=torch.int8, device=dev)
        osc = torch.empty((C, -(-R // group)), dtype=SCALE_DTYPE, device=dev)
        keep.append((codes, scales))
        out.append((oc, osc))
        arr[i] = (codes.data_ptr(), scales.data_ptr(), R, C, oc.data_ptr(), osc.data_ptr())
    _lib.call("ksd_requant_transpose_multi", arr.ctypes.data, len(pairs), group, _lib.stream_ptr(dev))
    return out


def layer_norm_quantize(x: torch.Tensor, weight: torch.Tensor | None = None,
                        bias: torch.Tensor | None = None, eps: float = 1e-5,
                        group: int = GROUP_SIZE, return_y: bool = False,
                        return_stats: bool = False):
    """F.layer_norm(x, (d,), weight, bias, eps) followed by quantize_last_dim(., group), in
    one pass over x: the pre-norm of a block (reference ksdraft/model/block.py:27-41)
    producing the A operand of the Int8Linear after it (kernels/linear.py:69).

    y is computed in fp32 from x's values and rounded to x's dtype, the dtype torch's
    LayerNorm returns; the codes are quantize_last_dim of that y. Returns (codes, scales),
    then y if return_y, then (mean, rstd) fp32 per row if return_stats. d <= 4096, group 128.
    """
    x = _float_input(x)
    if group != 128:
        raise ValueError(f"layer_norm_quantize supports group 128, got {group}")
    d = x.shape[-1] if x.dim() else 0
    if d < 1 or d > 4096:
        raise ValueError(f"layer_norm_quantize supports 1 <= d <= 4096, got {d}")
    dev = _lib.require_gpu(x, *(t for t in (weight, bias) if t is not None))
    lead = x.shape[:-1]
    x2 = x.reshape(-1, d)
    rows = x2.shape[0]
    if x2.stride(-1) != 1 or (rows > 1 and x2.stride(0) < d):
        x2 = x2.contiguous()
    params = []
    for name, p in (("weight", weight), ("bias", bias)):
        if p is not None:
            if p.shape != (d,):
                raise ValueError(f"{name} must have shape ({d},), got {tuple(p.shape)}")
            p = p.detach().to(device=dev, dtype=torch.float32).contiguous()
        params.append(p)
    ng = -(-d // group)
    codes = torch.empty((rows, d), dtype=torch.int8, device=dev)
    scales = torch.empty((rows, ng), dtype=SCALE_DTYPE, device=dev)
    y = torch.empty((rows, d), dtype=x2.dtype, device=dev) if return_y else None
    mean = torch.empty(rows, dtype=torch.float32, device=dev) if return_stats else None
    rstd = torch.empty(rows, dtype=torch.float32, device=dev) if return_stats else None
    ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    stride = x2.stride(0) if rows > 1 else d
    _lib.call("ksd_layernorm_quant", x2.data_ptr(), _lib.dtype_code(x2.dtype), rows, d, stride,
              ptr(params[0]), ptr(params[1]), float(eps), group, codes.data_ptr(),
              scales.data_ptr(), ptr(y), ptr(mean), ptr(rstd), _lib.stream_ptr(dev))
    out = (codes.reshape(*lead, d), scales.reshape(*lead, ng))
    if return_y:
        out += (y.reshape(*lead, d),)
    if return_stats:
        out += (mean.reshape(lead), rstd.reshape(lead))
    return out
