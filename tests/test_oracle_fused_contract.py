"""The oracle's fused KS3 contract (project_fused, reference ksdraft/kernels/ks3_triton.py)
against how Triton compiles the reference kernel for gfx950.

tests/golden/ks3_fused_contract.json holds, per target, nonlinear mode and source line of
ks3_triton.py, the floating-point opcodes and constants of the reference kernel's AMD
assembly (written in the build container by tests/golden/make_ks3_fused_contract.py).
oracle.ks3.FUSED_CONTRACT says, line by line, which multiply/add pairs the oracle fuses;
each label is checked against the opcodes the compiler emitted for that line. The
oracle's fused multiply-adds are checked against exact rational arithmetic, including
inputs where one rounding and two roundings differ, and the fused oracle is shown to
differ from the unfused composition on random data (so a regression to separate roundings
cannot pass the GPU bit-exact tests unnoticed).
"""

import json
import os
from fractions import Fraction

import numpy as np
import pytest

from oracle import ks3 as ok
from oracle import quant as oq

FIX = os.path.join(os.path.dirname(__file__), "golden", "ks3_fused_contract.json")

FMA16 = {"v_fma_f16", "v_fmac_f16", "v_fmamk_f16", "v_fmaak_f16", "v_pk_fma_f16"}
FMA32 = {"v_fma_f32", "v_fmac_f32", "v_fmamk_f32", "v_fmaak_f32", "v_pk_fma_f32", "v_fma_mix_f32"}
ADD16 = {"v_add_f16", "v_sub_f16", "v_subrev_f16", "v_pk_add_f16"}
ADD32 = {"v_add_f32", "v_sub_f32", "v_subrev_f32", "v_pk_add_f32"}
MUL16 = {"v_mul_f16", "v_pk_mul_f16"}
MUL32 = {"v_mul_f32", "v_pk_mul_f32"}
DIV = {"v_div_scale_f32", "v_div_fmas_f32", "v_div_fixup_f32"}


@pytest.fixture(scope="module")
def fix():
    with open(FIX) as f:
        return json.load(f)


def _ops(fix, arch, nl, line):
    return set(fix["targets"][arch]["modes"][str(nl)][str(line)]["ops"])


def _check_label(ops, label, where):
    has = lambda fam: bool(ops & fam)  # noqa: E731
    if label == "ieee_div":
        assert DIV <= ops, where
    elif label == "fma16,mul16":
        assert has(FMA16) and has(MUL16) and not has(ADD16), (where, ops)
    elif label == "fma16":
        assert has(FMA16) and not has(ADD16) and not has(FMA32), (where, ops)
    elif label == "fma32":
        assert has(FMA32) and not has(ADD32), (where, ops)
    elif label == "add,fma32":
        assert has(FMA32) and has(ADD32) and not has(MUL32), (where, ops)
    elif label in ("mul,add", "add,mul"):
        assert has(MUL32) and has(ADD32) and not has(FMA32) and not has(FMA16), (where, ops)
    else:
        raise AssertionError(label)


def test_fixture_is_for_the_installed_kernel_shape(fix):
    assert fix["kernel"] == "_fused_gemm_spine"
    assert set(fix["targets"]) == {"gfx950", "gfx1100"}
    for arch in fix["targets"]:
        assert set(fix["targets"][arch]["modes"]) == {"0", "1", "2"}


def test_oracle_contract_matches_the_gfx950_compile(fix):
    for (nl, line), label in ok.FUSED_CONTRACT.items():
        _check_label(_ops(fix, "gfx950", nl, line), label, (nl, line))


def test_warp_step_is_one_fp16_fma_on_both_targets(fix):
    """ks3_triton.py:59: fp16(4/127) (0x2808) and a fused fp16 multiply-add, on the MI355X
    and on the reference's gfx1100 development GPU alike."""
    step_bits = "0x%04x" % int(np.float16(4.0 / 127.0).view(np.uint16))
    assert step_bits == "0x2808"
    for arch in ("gfx950", "gfx1100"):
        ent = fix["targets"][arch]["modes"]["2"]["59"]
        assert step_bits in ent["consts"], arch
        assert set(ent["ops"]) & FMA16 and not set(ent["ops"]) & ADD16, arch


def test_reference_gemm_accumulate_contract(fix):
    """ks3_triton.py:135 (and the same expression in gemm.py:43-45): the reference kernel
    accumulates fma(fl(float(P) * sa), sw, acc), a separately rounded product with the
    activation scale and then a mixed fp32/fp16 fused multiply-add with the weight scale.
    This build's GEMM contract is fma(float(P), sa * sw, acc) instead (sa * sw is exact in
    fp32); the difference is within the north-star fp32 tolerance."""
    for nl in (0, 1, 2):
        ops = fix["targets"]["gfx950"]["modes"][str(nl)]["135"]["ops"]
        assert ops.get("v_mul_f32", 0) == ops.get("v_fma_mix_f32", 0) > 0
        assert ops.get("v_cvt_f32_i32", 0) == ops.get("v_mul_f32")


def _round_exact(q, dt):
    """Correct (ties-to-even) rounding of a Fraction to dt, by comparing neighbours."""
    f = dt(float(q))
    with np.errstate(over="ignore"):
        cands = [c for c in (np.nextafter(f, dt(-np.inf)), f, np.nextafter(f, dt(np.inf)))
                 if np.isfinite(c)]
    ut = np.uint16 if dt == np.float16 else np.uint32
    return min(cands, key=lambda v: (abs(Fraction(float(v)) - q), int(dt(v).view(ut)) & 1))


def test_fma16_rounds_once():
    rng = np.random.default_rng(0)
    cases = []
    for _ in range(3000):  # random fp16 triples, subnormals included
        bits = rng.integers(0, 0x7C00, 3) | (rng.integers(0, 2, 3) << 15)
        cases.append([np.uint16(b).view(np.float16) for b in bits])
    for _ in range(3000):  # products on fp16 midpoints, tiny addends that break the tie
        a = np.float16(rng.integers(32, 64) / 32.0 * 2.0 ** rng.integers(-6, 6))
        b = np.float16(rng.integers(32, 64) / 32.0 * 2.0 ** rng.integers(-6, 6))
        cases.append([a, b, np.float16(rng.choice([-1, 1]) * 2.0 ** rng.integers(-24, -14))])
    n_double = 0
    for a, b, c in cases:
        q = Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c))
        if abs(q) > 65504:
            continue
        exp = _round_exact(q, np.float16)
        got = np.float16(ok.fma16(np.float32(a), np.float32(b), np.float32(c)))
        assert got.view(np.uint16) == exp.view(np.uint16), (a, b, c)
        with np.errstate(over="ignore"):
            n_double += ok.h(ok.h(np.float32(a) * np.float32(b)) + np.float32(c)) != np.float32(exp)
    assert n_double > 100  # the two-rounding form differs on these inputs


def test_fma32_rounds_once():
    rng = np.random.default_rng(1)
    cases = []
    for _ in range(2000):
        a, b = (rng.standard_normal(2) * 2.0 ** rng.integers(-20, 20, 2)).astype(np.float32)
        cases.append((a, b, np.float32(rng.standard_normal() * 2.0 ** rng.integers(-40, 20))))
    for _ in range(2000):  # 12-bit operands: products on fp32 midpoints, tie-breaking addends
        a = np.float32(rng.integers(2048, 4096) / 2048.0 * 2.0 ** rng.integers(-5, 5))
        b = np.float32(rng.integers(2048, 4096) / 2048.0 * 2.0 ** rng.integers(-5, 5))
        cases.append((a, b, np.float32(rng.choice([-1, 1]) * 2.0 ** rng.integers(-80, -30))))
    a1 = np.float32(1 + 2.0 ** -12)  # (1 + 2^-12)^2 = 1 + 2^-11 + 2^-24, an fp32 midpoint
    cases += [(a1, a1, np.float32(2.0 ** -60)), (a1, a1, np.float32(-2.0 ** -60))]
    n_double = 0
    for a, b, c in cases:
        q = Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c))
        exp = _round_exact(q, np.float32)
        got = ok.fma32(a, b, c)
        assert np.float32(got).view(np.uint32) == exp.view(np.uint32), (a, b, c)
        n_double += np.float32(np.float32(a) * np.float32(b) + np.float32(c)) != exp
    assert n_double > 10


def test_fused_warp_step_exhaustive_over_codes():
    """Every LUT output code times fp16(4/127) plus shifts on a grid of fp16 values: the
    oracle's warp intermediate is the single rounding of the exact value."""
    step = Fraction(float(np.float16(4.0 / 127.0)))
    rng = np.random.default_rng(2)
    shifts = np.concatenate([
        np.uint16(rng.integers(0, 0x3800, 160) | (rng.integers(0, 2, 160) << 15)).view(np.float16),
        np.array([2.0 ** -24, -2.0 ** -24, 2.0 ** -23, 0.0], np.float16)])
    tq = np.arange(-127, 128)
    got = ok.fma16(tq[:, None].astype(np.float32), np.float32(step), shifts[None, :].astype(np.float32))
    for i, t in enumerate(tq):
        for j, sh in enumerate(shifts):
            exp = _round_exact(t * step + Fraction(float(sh)), np.float16)
            assert np.float32(exp) == got[i, j], (t, sh)
    # tq = 124: 124 * fp16(4/127) is an fp16 midpoint that rounds up to even; a shift of
    # -2^-24 puts the exact value below it
    assert ok.fma16(np.float32(124), np.float32(step), np.float32(-2.0 ** -24)) != \
        ok.h(ok.h(np.float32(124) * np.float32(step)) + np.float32(-2.0 ** -24))


def _spine_inputs(seed, M, Fn):
    rng = np.random.default_rng(seed)
    sq, ss = oq.quantize_last_dim((rng.standard_normal((Fn, 6)) * 0.3).astype(np.float32))
    sc = ok.h((np.abs(rng.standard_normal(Fn)) + 0.3).astype(np.float32))
    sh = ok.h((rng.standard_normal(Fn) * 0.4).astype(np.float32))
    x = (rng.standard_normal((M, Fn)) * 3).astype(np.float32)
    return x, sq, ss.reshape(-1), sc, sh


def test_fused_int8_spine_differs_from_two_roundings():
    """The fused int8 contract on random accumulators: the warp step's single rounding
    changes some LUT picks (and so some codes) against the two-rounding form."""
    x, sq, ss, sc, sh = _spine_inputs(3, 64, 256)
    lut = ok.make_tanh_lut()
    tq = lut[np.clip(np.rint((np.clip(x * np.float32(0.25), -3.2, 3.2) * np.float32(127 / 3.2))
                             .astype(np.float32)).astype(np.int64) + 128, 0, 255)]
    step = np.float32(np.float16(4.0 / 127.0))
    one = ok.fma16(tq.astype(np.float32), step, sh[None, :])
    two = ok.h(ok.h(tq.astype(np.float32) * step) + sh[None, :])
    assert np.mean(one != two) > 0.01
    q, s = ok.spine_fused_int8(x, sq, ss, sc, sh, lut)
    assert q.shape == x.shape and s.shape == (64, 2)


@pytest.mark.parametrize("mode", ["fp16", "fp32"])
def test_fused_float_modes_differ_from_composed_roundings(mode):
    x, sq, ss, sc, sh = _spine_inputs(4, 48, 256)
    fused = ok.spine_features_float(x, sq, ss, sc, sh, mode, fused=True)
    plain = ok.spine_features_float(x, sq, ss, sc, sh, mode)
    assert fused.shape == plain.shape and np.all(np.isfinite(fused))
    assert np.mean(fused != plain) > 0.01
    # both are the same function up to rounding
    np.testing.assert_allclose(fused, plain, rtol=2e-2 if mode == "fp16" else 1e-5,
                               atol=1e-3 * np.abs(plain).max())
