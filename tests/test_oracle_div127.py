"""The library's group scale divides by 127 with a reciprocal multiply and one FMA
correction step (ksdraft_amd/csrc/ksd_common.h, div127) instead of the IEEE division the
reference's amax / 127 is (kernels/quant.py:48). The identity was checked once over every
positive normal fp32 value; this test re-checks whole binades at both ends of the range and
around 1, plus the signed zeros, subnormals, infinities and a random sample of the rest,
through the oracle's C checker (gcc's fmaf and IEEE division)."""

import numpy as np

from oracle._clib import lib


def _binade(e):
    lo = e << 23
    return lo, lo + (1 << 23)


def test_div127_whole_binades():
    L = lib()
    for e in (1, 2, 3, 100, 126, 127, 128, 140, 152, 253, 254):
        lo, hi = _binade(e)
        assert L.ksd_check_div127(lo, hi) == 0, e
        assert L.ksd_check_div127(lo | 0x80000000, hi | 0x80000000) == 0, -e


def test_div127_specials_and_sample():
    L = lib()
    assert L.ksd_check_div127(0, 1 << 16) == 0                      # +0 and subnormals
    assert L.ksd_check_div127(0x7f800000, 0x7f800000 + (1 << 16)) == 0   # inf, NaNs
    rng = np.random.default_rng(127)
    for u in rng.integers(0, 1 << 32, 20000, dtype=np.uint64):
        u = int(u)
        assert L.ksd_check_div127(u, min(u + 64, 1 << 32)) == 0, hex(u)
