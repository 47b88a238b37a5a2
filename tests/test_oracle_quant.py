"""Pins the numpy quantization oracle (oracle/quant.py) — CPU only.

Checks: the reference's own KATs and invariants (tests/test_int8.py:10-40,
tests/test_stages.py:36-45) and an exact-rational restatement of every rounding step
(tests/exact_float.py), on inputs chosen so that plausible mistakes fail: reciprocal
multiply instead of division (half-integer quotients), flushing subnormal fp16 scales,
a missing scale clamp, round-half-away instead of half-even.
"""

import numpy as np
import pytest

from oracle import quant as oq
from tests.exact_float import exact_quantize_group


def test_zero_row_kat():
    # reference tests/test_int8.py:35-40
    codes, scales = oq.quantize_last_dim(np.zeros((2, 128), np.float32))
    assert (codes == 0).all()
    assert (oq.dequantize_last_dim(codes, scales) == 0).all()


def test_partial_group_shapes():
    # reference tests/test_int8.py:27-32
    x = np.random.default_rng(0).standard_normal((4, 100)).astype(np.float32)
    codes, scales = oq.quantize_last_dim(x)
    assert codes.shape == (4, 100) and scales.shape == (4, 1)


def test_roundtrip_error_bound():
    # reference tests/test_int8.py:10-24
    x = (np.random.default_rng(0).standard_normal((64, 256)) * 3).astype(np.float32)
    codes, scales = oq.quantize_last_dim(x)
    dq = oq.dequantize_last_dim(codes, scales)
    s = scales.astype(np.float32).reshape(64, 2, 1)
    err = np.abs(x - dq).reshape(64, 2, 128)
    resid = np.clip(np.abs(x).reshape(64, 2, 128) - 127.0 * s, 0, None)
    assert (err <= s / 2 + resid + 1e-6).all()


def _adversarial_rows(rng, group):
    rows = []
    # plain gaussians at several magnitudes, incl. fp16-subnormal and clamped scales
    for mag in (1.0, 3.0, 1e-3, 1e-6, 2e-7, 1e-9, 1e5, 1e7, 1e12):
        rows.append((rng.standard_normal(group * 2) * mag).astype(np.float32))
    # exact half-integer quotients and their fp32 neighbours
    for s16 in (np.float16(0.0078125), np.float16(0.01), np.float16(3.1e-5),
                np.float16(6.0e-8), np.float16(1.5)):
        s = np.float32(s16)
        ks = rng.integers(-126, 126, 2 * group - 2)
        vals = [(np.float32(k) + np.float32(0.5)) * s for k in ks]
        # each group carries its own amax element 127*s, so its scale is exactly s
        r = np.array([np.float32(127) * s] + vals[:group - 1]
                     + [np.float32(-127) * s] + vals[group - 1:], np.float32)
        rows.append(r)
        rows.append(np.nextafter(r, np.float32(np.inf)).astype(np.float32))
        rows.append(np.nextafter(r, np.float32(-np.inf)).astype(np.float32))
    return np.stack(rows)


@pytest.mark.parametrize("group", [32, 64, 128])
def test_oracle_matches_exact_rational(group):
    rng = np.random.default_rng(1234 + group)
    x = _adversarial_rows(rng, group)
    codes, scales = oq.quantize_last_dim(x, group)
    for r in range(x.shape[0]):
        ec, es = exact_quantize_group(x[r], group)
        assert np.array_equal(codes[r], ec), r
        assert np.array_equal(scales[r].view(np.uint16), es.view(np.uint16)), r


def test_oracle_ragged_exact():
    rng = np.random.default_rng(7)
    for K in (1, 6, 100, 129, 300):
        x = rng.standard_normal((3, K)).astype(np.float32)
        codes, scales = oq.quantize_last_dim(x)
        for r in range(3):
            ec, es = exact_quantize_group(x[r], 128)
            assert np.array_equal(codes[r], ec)
            assert np.array_equal(scales[r], es)


def test_dither_zero_is_exact_and_dither_explores():
    # reference tests/test_stages.py:36-45
    rng = np.random.default_rng(0)
    x = (rng.standard_normal((8, 256)) * 3).astype(np.float32)
    c0, s0 = oq.quantize_last_dim(x, 128, noise=rng.random((8, 256)), dither=0.0)
    ce, se = oq.quantize_last_dim(x, 128)
    assert np.array_equal(c0, ce) and np.array_equal(s0, se)
    cd, _ = oq.quantize_last_dim(x, 128, noise=rng.random((8, 256)).astype(np.float32),
                                 dither=0.5)
    changed = (cd != ce).mean()
    assert 0.0 < changed < 0.6


def test_dequant_group_inference_quirk():
    # quant.py:61-62: group inferred as padded_length(K) // n_scales
    codes = np.arange(-3, 3, dtype=np.int8).reshape(1, 6)
    scales = np.array([[0.5]], np.float16)
    assert np.array_equal(oq.dequantize_last_dim(codes, scales), codes.astype(np.float32) * 0.5)
    c = np.ones((1, 256), np.int8)
    s = np.array([[1, 2, 3, 4, 5, 6, 7, 8]], np.float16)  # 8 scales -> group 32
    assert np.array_equal(oq.dequantize_last_dim(c, s)[0, ::32], np.arange(1, 9, dtype=np.float32))


def test_requant_transpose_is_quant_of_dequant_transpose():
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((200, 96)) * 0.02).astype(np.float32)
    wq, ws = oq.quantize_last_dim(w)
    tq, ts = oq.requant_transpose(wq, ws)
    assert tq.shape == (96, 200) and ts.shape == (96, 2)
    real = oq.dequantize_last_dim(wq, ws).T
    for r in range(0, 96, 7):
        ec, es = exact_quantize_group(real[r], 128)
        assert np.array_equal(tq[r], ec) and np.array_equal(ts[r], es)


def test_nonfinite_groups_follow_torch():
    """quant.py:47-51 run by torch on the CPU: a NaN in a group gives a NaN scale (fp16
    bits 0x7fff) and zero codes; inf gives scale 65504 and +-127 at the inf."""
    import torch
    x = np.zeros((3, 256), np.float32)
    x[0, 3] = np.nan
    x[0, 200] = 5.0
    x[1, 7] = np.inf
    x[1, 8] = 2.0
    x[2, 130] = -np.inf
    codes, scales = oq.quantize_last_dim(x)
    t = torch.from_numpy(x)
    amax = t.reshape(3, 2, 128).abs().amax(-1, keepdim=True)
    s = (amax / 127.0).clamp(2.0 ** -24, 65504.0).to(torch.float16).float()
    tc = torch.clamp(torch.round(t.reshape(3, 2, 128) / s), -127.0, 127.0).to(torch.int8)
    assert np.array_equal(codes, tc.reshape(3, 256).numpy())
    assert np.array_equal(scales.view(np.uint16), s.to(torch.float16).reshape(3, 2).numpy().view(np.uint16))
    assert scales.view(np.uint16)[0, 0] == 0x7fff and codes[1, 7] == 127 and codes[2, 130] == -127
