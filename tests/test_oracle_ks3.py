"""Pins the KS3 int8 oracle (oracle/ks3.py) — CPU only.

Against the golden vectors written from the reference's own CPU path
(tests/golden/make_ks3_golden.py -> ks3_int8_golden.npz): bit-exact tanh LUT, int8-mode
spine features and VJP coordinate gradient given identical GEMM outputs; fp16 column
reductions within one fp16 ulp (torch's summation order is not reproduced). Plus
closed-form / brute-force checks of the integer helpers."""

import os

import numpy as np
import pytest

from oracle import ks3 as ok

GOLD = os.path.join(os.path.dirname(__file__), "golden", "ks3_int8_golden.npz")


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLD, allow_pickle=False)


def test_lut_matches_reference_and_has_margin(gold):
    lut = ok.make_tanh_lut()
    assert np.array_equal(lut, gold["tanh_lut"])
    # every entry is far from a rounding tie, so fp32 tanh error cannot flip it
    idx = np.arange(-128, 128, dtype=np.float64)
    v = np.tanh(idx * (3.2 / 127.0)) * 127.0
    assert np.min(np.abs(np.abs(v - np.floor(v)) - 0.5)) > 5e-3


def test_round_div127_brute_force():
    v = np.arange(-200000, 200001, 7, dtype=np.int64)
    got = ok.round_div127(v)
    # definition: nearest integer to v/127, ties impossible (127 odd)
    exp = np.array([int(np.floor(x / 127.0 + 0.5)) if x >= 0 else -int(np.floor(-x / 127.0 + 0.5)) for x in v])
    assert np.array_equal(got, exp)


def test_lut_index_saturates_and_rounds():
    x = np.array([-100.0, -3.2, -1.0, 0.0, 0.0126, 3.1992, 3.2, 50.0], np.float32)
    x16 = x.astype(np.float16).astype(np.float32)
    got = ok.lut_index(x16)
    assert got[0] == -127 and got[-1] == 127 and got[3] == 0


@pytest.mark.parametrize("case", ["std1", "std8"])
def test_spine_features_bit_exact_vs_reference(gold, case):
    lut = ok.make_tanh_lut()
    sc, sh = ok.warp_scalars(gold["warp_scale_codes"], gold["warp_scale_scales"],
                             gold["warp_shift_codes"], gold["warp_shift_scales"])
    got = ok.spine_features_int8(gold[f"{case}/coords"], gold["spine_codes"],
                                 gold["spine_scale"], sc, sh, lut)
    assert np.array_equal(got.view(np.uint32), gold[f"{case}/h"].view(np.uint32))


@pytest.mark.parametrize("case", ["std1", "std8"])
def test_vjp_bit_exact_dc_and_close_reductions(gold, case):
    coef, sc, sh = ok.spine_params(gold["spine_codes"], gold["spine_scale"],
                                   gold["warp_scale_codes"], gold["warp_scale_scales"],
                                   gold["warp_shift_codes"], gold["warp_shift_scales"])
    dc, sums, dcoeff, dscale, dshift = ok.vjp(gold[f"{case}/value"], gold[f"{case}/coords"],
                                              coef, sc, sh, gold["master_raw_scale"],
                                              gold["master_raw_shift"])
    assert np.array_equal(dc, gold[f"{case}/dc"])
    ref = gold[f"{case}/dcoeff"].reshape(-1, 6).astype(np.float32)
    np.testing.assert_allclose(dcoeff, ref, rtol=2e-3, atol=1e-3 * np.abs(ref).max())
    np.testing.assert_allclose(dscale, gold[f"{case}/dscale"], rtol=2e-3,
                               atol=1e-3 * np.abs(gold[f"{case}/dscale"]).max())
    np.testing.assert_allclose(dshift, gold[f"{case}/dshift"], rtol=2e-3,
                               atol=1e-3 * np.abs(gold[f"{case}/dshift"]).max() + 1e-12)


def test_pack_masters_reproduces_cell_buffers(gold):
    packed = ok.pack_masters(gold["master_down"], gold["master_up"],
                             gold["master_coefficients"], gold["master_raw_scale"],
                             gold["master_raw_shift"])
    assert np.array_equal(packed["spine_codes"], gold["spine_codes"])
    assert np.array_equal(packed["spine_scale"], gold["spine_scale"])
    for k in ("warp_scale_codes", "warp_scale_scales", "warp_shift_codes", "warp_shift_scales"):
        assert np.array_equal(packed[k], gold[k]), k
