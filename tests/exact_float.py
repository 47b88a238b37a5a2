"""Exact IEEE rounding on rationals (fractions.Fraction), for pinning the oracle.

Independent of numpy/torch: every rounding is derived from the format definition
(precision p, minimum normal exponent, max finite), round-to-nearest-even."""

from __future__ import annotations

from fractions import Fraction

import numpy as np

INF = float("inf")


def _floor_log2(a: Fraction) -> int:
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    return e


def round_to_format(x: Fraction, p: int, emin: int, max_finite: Fraction):
    """Nearest-even rounding of x into a binary format; returns Fraction or +-inf."""
    if x == 0:
        return Fraction(0)
    sign = -1 if x < 0 else 1
    a = abs(x)
    e = max(_floor_log2(a), emin)
    q = Fraction(2) ** (e - p + 1)
    n = a / q
    fl = n.numerator // n.denominator
    rem = n - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    r = fl * q
    # IEEE overflow: round to inf once the value rounds beyond the max finite
    if r > max_finite:
        return sign * INF
    return sign * r


FP32_MAX = Fraction((2 ** 24 - 1) * 2 ** 104)
FP16_MAX = Fraction(65504)


def rn_f32(x: Fraction):
    return round_to_format(x, 24, -126, FP32_MAX)


def rn_f16(x: Fraction):
    return round_to_format(x, 11, -14, FP16_MAX)


def rne_int(x: Fraction) -> int:
    fl = x.numerator // x.denominator
    rem = x - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    return fl


def frac(v) -> Fraction:
    return Fraction(float(v))


def exact_quantize_group(values, group: int):
    """quantize_last_dim of one row, derived with exact arithmetic (quant.py:45-52)."""
    vals = [frac(v) for v in np.asarray(values, np.float32)]
    K = len(vals)
    Kp = (K + group - 1) // group * group
    vals = vals + [Fraction(0)] * (Kp - K)
    codes, scales = [], []
    for g0 in range(0, Kp, group):
        grp = vals[g0:g0 + group]
        amax = max(abs(v) for v in grp)
        s = rn_f32(amax / 127)                       # fp32 division, correctly rounded
        s = min(max(s, Fraction(1, 2 ** 24)), Fraction(65504))
        s = rn_f16(s)                                # round through fp16
        scales.append(float(s))
        for v in grp:
            q = rn_f32(v / s)                        # fp32 division
            c = rne_int(q)
            codes.append(max(-127, min(127, c)))
    return np.array(codes[:K], np.int8), np.array(scales, np.float16)
