"""numpy restatement of GS symmetric int8 quantization (test infrastructure only).

Follows reference ksdraft/kernels/quant.py:20-67 and ksdraft/train/stages.py:27-50:
fp32 amax/127, clamp to [2^-24, 65504], round through fp16, codes = clamp(rne(x/s), +-127),
zero-padded partial groups. numpy's float32 division is IEEE correctly rounded, np.rint
is round-half-even and astype(float16) rounds to nearest even with subnormals — the same
operations torch performs on CPU.

Pinned by: the reference's KATs (zero row, tests/test_int8.py:35-40; dither 0 == exact,
tests/test_stages.py:36-45), its error-bound invariant (tests/test_int8.py:10-24), and an
independent exact-rational restatement (tests/test_oracle_quant.py) that derives every
rounding from the IEEE definitions with fractions.Fraction.
"""

from __future__ import annotations

import numpy as np

GROUP_SIZE = 128
SCALE_MIN = np.float32(2.0 ** -24)
SCALE_MAX = np.float32(65504.0)


def padded_length(n: int, group: int = GROUP_SIZE) -> int:
    """quant.py:26-27."""
    return (n + group - 1) // group * group


def quantize_last_dim(x, group: int = GROUP_SIZE, noise=None, dither: float = 0.0):
    """quant.py:30-52 (noise/dither: stages.py:42-48).

    x: (..., K) float array (converted to float32, as the reference's callers pass
    `.float()`). noise: optional (..., Kp) uniform draws for the dithered variant.
    Returns (codes int8 (..., K), scales float16 (..., Kp/group)).
    """
    x = np.asarray(x, dtype=np.float32)
    K = x.shape[-1]
    Kp = padded_length(K, group)
    lead = x.shape[:-1]
    if Kp != K:
        x = np.concatenate([x, np.zeros(lead + (Kp - K,), np.float32)], axis=-1)
    grouped = x.reshape(lead + (Kp // group, group))
    amax = np.abs(grouped).max(axis=-1) if Kp else np.zeros(lead + (0,), np.float32)
    scale = (amax / np.float32(127.0)).astype(np.float32)
    scale = np.clip(scale, SCALE_MIN, SCALE_MAX).astype(np.float16).astype(np.float32)
    q = (grouped / scale[..., None]).astype(np.float32)
    if noise is not None and dither > 0:
        n = np.asarray(noise, dtype=np.float32).reshape(q.shape)
        nz = ((n - np.float32(0.5)).astype(np.float32) * np.float32(2.0 * dither)).astype(np.float32)
        q = (q + nz).astype(np.float32)
    # NaN groups (torch: amax and clamp propagate NaN, NaN -> int8 gives 0, and the fp16
    # NaN scale is 0x7fff); pinned against torch in tests/test_oracle_quant.py
    nan = np.isnan(q)
    codes = np.where(nan, 0.0, np.clip(np.rint(np.where(nan, 0.0, q)), -127.0, 127.0)).astype(np.int8)
    codes = codes.reshape(lead + (Kp,))[..., :K]
    s16 = scale.astype(np.float16)
    s16.view(np.uint16)[np.isnan(s16)] = 0x7fff
    return np.ascontiguousarray(codes), s16


def dequantize_last_dim(codes, scales, group: int | None = None):
    """quant.py:55-67, including its group inference from the scale count."""
    codes = np.asarray(codes)
    scales = np.asarray(scales)
    K = codes.shape[-1]
    if group is None:
        group = padded_length(K) // max(scales.shape[-1], 1)
    Kp = padded_length(K, group)
    lead = codes.shape[:-1]
    c = codes.astype(np.float32)
    if Kp != K:
        c = np.concatenate([c, np.zeros(lead + (Kp - K,), np.float32)], axis=-1)
    grouped = c.reshape(lead + (Kp // group, group))
    out = grouped * scales.astype(np.float32)[..., None]
    return out.reshape(lead + (Kp,))[..., :K].astype(np.float32)


def quantize_transpose(x, group: int = GROUP_SIZE):
    """quantize_last_dim(x.T) — the dW operand build of ks3_int8.py:418, 422."""
    x = np.asarray(x, dtype=np.float32)
    return quantize_last_dim(np.ascontiguousarray(x.T), group)


def requant_transpose(codes, scales, group_in: int = GROUP_SIZE, group: int = GROUP_SIZE):
    """quantize_last_dim(dequantize_last_dim(codes, scales).T) — ks3_int8.py:349-351, 407-408, 417-419."""
    real = dequantize_last_dim(codes, scales, group_in)
    return quantize_last_dim(np.ascontiguousarray(real.T), group)
