"""Pins the GEMM oracle (oracle/gemm.py, oracle/ksd_oracle.c) — CPU only.

* int32 partials: against an independent numpy int64 matmul per group.
* ordered fp32 contract: against exact rational arithmetic, one correctly rounded
  fmaf per group in ascending order (catches a wrong group order, an unfused
  multiply-add, a scale of one operand only, a transposed operand).
* the reference CPU path (dequantize + fp32 matmul, gemm.py:76-82): against a float64
  product of the dequantized operands.
* fp16 decode: all 65536 patterns against numpy.
"""

from fractions import Fraction

import numpy as np
import pytest

from oracle import _clib
from oracle import gemm as og
from oracle import quant as oq
from tests.exact_float import rn_f32


def _operands(seed, M, K, N, group=128, wscale=0.1):
    rng = np.random.default_rng(seed)
    a = rng.standard_normal((M, K)).astype(np.float32)
    w = (rng.standard_normal((N, K)) * wscale).astype(np.float32)
    aq, as_ = oq.quantize_last_dim(a, group)
    wq, ws = oq.quantize_last_dim(w, group)
    return aq, as_, wq, ws


def test_half_decode_all_patterns():
    lib = _clib.lib()
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([lib.ksd_half_to_float(int(b)) for b in bits[::1]], np.float32)
    fin = np.isfinite(ref)
    assert np.array_equal(got[fin].view(np.uint32), ref[fin].view(np.uint32))
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(np.isinf(got), np.isinf(ref))


@pytest.mark.parametrize("group", [32, 128])
def test_partials_vs_int64_matmul(group):
    aq, _, wq, _ = _operands(0, 37, 256, 29, group)
    P = og.group_partials(aq, wq, group)
    for g in range(256 // group):
        sl = slice(g * group, (g + 1) * group)
        ref = aq[:, sl].astype(np.int64) @ wq[:, sl].astype(np.int64).T
        assert np.array_equal(P[g], ref)


def test_partials_extreme_codes():
    a = np.full((2, 128), -127, np.int8)
    w = np.full((3, 128), -127, np.int8)
    assert (og.group_partials(a, w) == 128 * 127 * 127).all()


def _exact_ordered(aq, as_, wq, ws, group, m, n):
    acc = Fraction(0)
    G = aq.shape[1] // group
    for g in range(G):
        sl = slice(g * group, (g + 1) * group)
        p = int(aq[m, sl].astype(np.int64) @ wq[n, sl].astype(np.int64))
        s = Fraction(float(as_[m, g])) * Fraction(float(ws[n, g]))
        acc = rn_f32(Fraction(p) * s + acc)   # one rounding: fused multiply-add
    return np.float32(float(acc))


@pytest.mark.parametrize("group", [32, 128])
def test_ordered_contract_vs_exact_rationals(group):
    aq, as_, wq, ws = _operands(1, 9, 512, 7, group)
    y = og.gemm_ordered(aq, as_, wq, ws, group)
    for m in range(9):
        for n in range(7):
            assert y[m, n] == _exact_ordered(aq, as_, wq, ws, group, m, n), (m, n)


def test_ordered_row_subset_and_bias():
    aq, as_, wq, ws = _operands(2, 20, 256, 11)
    bias = np.random.default_rng(5).standard_normal(11).astype(np.float32)
    full = og.gemm_ordered(aq, as_, wq, ws, 128, bias=bias)
    rows = np.array([3, 0, 19], np.int64)
    sub = og.gemm_ordered(aq, as_, wq, ws, 128, bias=bias, rows=rows)
    assert np.array_equal(sub, full[rows])
    nob = og.gemm_ordered(aq, as_, wq, ws, 128)
    assert np.array_equal(full, (nob + bias).astype(np.float32))


def test_reference_cpu_path_vs_float64():
    aq, as_, wq, ws = _operands(3, 33, 384, 64)
    y = og.gemm_reference(aq, as_, wq, ws)
    ad = aq.astype(np.float64) * np.repeat(as_.astype(np.float64), 128, axis=1)
    wd = wq.astype(np.float64) * np.repeat(ws.astype(np.float64), 128, axis=1)
    np.testing.assert_allclose(y, ad @ wd.T, rtol=1e-5, atol=1e-5)
    # ordered contract and the reference path agree to the reference's GPU bar
    np.testing.assert_allclose(og.gemm_ordered(aq, as_, wq, ws), y, rtol=1e-4, atol=1e-3)


def test_ragged_k_pads_like_reference():
    rng = np.random.default_rng(4)
    a = rng.standard_normal((5, 100)).astype(np.float32)
    w = rng.standard_normal((6, 100)).astype(np.float32)
    aq, as_ = oq.quantize_last_dim(a)
    wq, ws = oq.quantize_last_dim(w)
    y = og.gemm_reference(aq, as_, wq, ws)
    np.testing.assert_allclose(y, oq.dequantize_last_dim(aq, as_) @ oq.dequantize_last_dim(wq, ws).T,
                               rtol=1e-6, atol=1e-6)
    with pytest.raises(ValueError):
        og.gemm_reference(aq, as_[:, :0], wq, ws[:, :0])


def test_split_policy_matches_the_library():
    """The oracle's split rule equals the library's for shapes on both sides of the
    192-tile threshold (a pure host query: no device work)."""
    import ctypes
    from ksdraft_amd import _lib
    c = ctypes.c_int(0)
    shapes = [(512, 1536, 8192), (1536, 512, 8192), (1536, 1536, 8192), (256, 256, 2048),
              (128, 128, 1024), (128, 128, 896), (64, 64, 128), (8192, 1536, 1536),
              (1536, 5888, 8192), (2048, 3072, 4096), (130, 257, 16384), (1, 1, 65536)]
    for M, N, K in shapes:
        _lib.call("ksd_w8a8_gemm_splits", M, N, K, 128, ctypes.byref(c))
        assert c.value == og.splits_for(M, N, K), (M, N, K, c.value)
        _lib.call("ksd_w8a8_gemm_splits", M, N, K, 64, ctypes.byref(c))
        assert c.value == 1
    assert og.splits_for(512, 1536, 8192) == 5 and og.splits_for(1536, 1536, 8192) == 1


def test_split_contract_is_the_ordered_sum_of_its_parts():
    """With S parts the contract is ((part_0 + part_1) + ...) + bias, each part the ordered
    contract over its groups: recomposed here from unsplit oracle calls on K slices."""
    rng = np.random.default_rng(8)
    M, N, K, S = 40, 24, 1280, 3
    a = rng.integers(-127, 128, (M, K)).astype(np.int8)
    w = rng.integers(-127, 128, (N, K)).astype(np.int8)
    sa = (rng.random((M, K // 128)) * 0.05 + 1e-3).astype(np.float16)
    sw = (rng.random((N, K // 128)) * 0.05 + 1e-3).astype(np.float16)
    bias = rng.standard_normal(N).astype(np.float32)
    y = og.gemm_ordered(a, sa, w, sw, bias=bias, splits=S)
    G = K // 128
    parts = []
    for q in range(S):
        g0, g1 = q * G // S, (q + 1) * G // S
        parts.append(og.gemm_ordered(a[:, g0 * 128:g1 * 128], sa[:, g0:g1], w[:, g0 * 128:g1 * 128],
                                     sw[:, g0:g1], splits=1))
    tot = parts[0]
    for p_ in parts[1:]:
        tot = (tot + p_).astype(np.float32)
    tot = (tot + bias[None, :]).astype(np.float32)
    assert np.array_equal(y.view(np.uint32), tot.view(np.uint32))
    # and the unsplit contract agrees to rounding
    y1 = og.gemm_ordered(a, sa, w, sw, bias=bias, splits=1)
    np.testing.assert_allclose(y, y1, rtol=1e-5, atol=1e-5 * np.abs(y1).max())
