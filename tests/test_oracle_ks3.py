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


@pytest.mark.parametrize("case", ["std1", "std8"])
def test_fused_contract_within_reference_tolerance_of_composed(gold, case):
    """The project_fused contract against the reference's composed output on the golden
    cell: rel < 0.05, the reference's own bar (tests/test_ks3_int8.py:82-84)."""
    from oracle import gemm as og
    from oracle import quant as oq
    packed = ok.pack_masters(gold["master_down"], gold["master_up"],
                             gold["master_coefficients"], gold["master_raw_scale"],
                             gold["master_raw_shift"])
    sc, sh = ok.warp_scalars(gold["warp_scale_codes"], gold["warp_scale_scales"],
                             gold["warp_shift_codes"], gold["warp_shift_scales"])
    xq, xs = oq.quantize_last_dim(gold[f"{case}/x"])
    acc = og.gemm_ordered(xq, xs, packed["down_codes"], packed["down_scales"])
    # the composed contract's coordinates are fp16(acc); the reference's CPU GEMM sums in
    # another order, so they agree to fp16 rounding
    np.testing.assert_allclose(ok.coords_from_gemm(acc), gold[f"{case}/coords"], rtol=1e-3,
                               atol=1e-3)
    hq, hs = ok.spine_fused_int8(acc, gold["spine_codes"], gold["spine_scale"], sc, sh,
                                 ok.make_tanh_lut())
    y = og.gemm_ordered(hq, hs, packed["up_codes"], packed["up_scales"])
    ref = gold[f"{case}/y"]
    rel = np.linalg.norm(y - ref) / np.linalg.norm(ref)
    assert rel < 0.05, rel


def test_tanh_table_is_torch_fp16_tanh():
    """The VJP's fp16 tanh table (ksdraft_amd/csrc/gen_tanh16.py) equals the oracle's
    definition and torch.tanh on fp16 CPU tensors (the reference's op) for every
    non-negative finite fp16 input; below 2**-6 tanh rounds to its argument."""
    import importlib.util
    import torch
    path = os.path.join(os.path.dirname(os.path.dirname(__file__)), "ksdraft_amd", "csrc",
                        "gen_tanh16.py")
    spec = importlib.util.spec_from_file_location("gen_tanh16", path)
    gen = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(gen)
    tab = gen.table()
    bits = np.arange(0, 0x7c00, dtype=np.uint16)
    x = bits.view(np.float16)
    want = ok.h(ok.tanh32(x.astype(np.float32))).astype(np.float16).view(np.uint16)
    got = tab[np.minimum(bits, gen.LIMIT)]
    assert np.array_equal(got, want)
    t = torch.tanh(torch.from_numpy(x.copy())).numpy().view(np.uint16)
    assert np.array_equal(got, t)
    assert np.array_equal(tab[:0x2400], bits[:0x2400])


def test_fused_warp_step_follows_triton_scalar_typing():
    """ks3_triton.py:59 multiplies an fp16 tensor by the Python float 4/127. Triton's own
    promotion rule (triton.language.semantic, computation_type_impl) keeps a float scalar
    of no higher kind than the tensor out of promotion, so the op is fp16 and the constant
    is rounded to fp16. The rule is read from the installed Triton, not restated; the
    oracle's fused warp product must then differ from the fp32-constant product exactly
    where fp16 rounding of the constant matters."""
    sem = pytest.importorskip("triton.language.semantic")
    tl = pytest.importorskip("triton.language")
    impl = sem.TritonSemantic.computation_type_impl
    # (tensor fp16, scalar fp32) -> fp16, for mul/add (not div/mod)
    assert impl(None, tl.float16, False, tl.float32, True, False) == tl.float16
    assert impl(None, tl.float32, True, tl.float16, False, False) == tl.float16
    # a division would be promoted to fp32 (ps / 64. of :70 is fp32 anyway: ps is fp32)
    assert impl(None, tl.float16, False, tl.float32, True, True) == tl.float32
    tq = np.arange(-127, 128, dtype=np.float32)
    c16 = np.float32(np.float16(4.0 / 127.0))
    assert c16 == np.float32(0.031494140625)
    fused = ok.h(tq * c16)
    composed = ok.h(tq * np.float32(4.0 / 127.0))
    # the two products differ for some table values: the choice is observable
    assert 0 < int(np.sum(fused != composed)) < 255


def test_rosa_shifted_matches_torch_ops():
    """oracle.rosa.shifted against the reference's own expression run by torch on the CPU
    (model/rosa.py:128-133: prev = F.pad(x)[:, :-1]; prev + (x - prev) * sigmoid(mix)) for
    fp32, bf16 and fp16 x, bit-exact, with torch's sigmoid as the shared input."""
    import torch
    import torch.nn.functional as F
    from oracle import rosa as orr
    g = torch.Generator().manual_seed(5)
    for dt in (torch.float32, torch.bfloat16, torch.float16):
        x = (torch.randn(2, 37, 96, generator=g) * 3).to(dt)
        mix = torch.randn(96, generator=g) * 2
        prev = F.pad(x, (0, 0, 1, 0))[:, :-1, :]
        sig = torch.sigmoid(mix)
        ref = prev + (x - prev) * sig
        assert ref.dtype == torch.float32
        got = orr.shifted(x.float().numpy(), sig.numpy(), str(dt).split(".")[-1])
        assert np.array_equal(got.view(np.uint32), ref.numpy().view(np.uint32)), dt
        # the oracle's own sigmoid (correctly rounded) is within two fp32 ulps of torch's
        s32 = orr.sigmoid32(mix.numpy())
        assert np.max(np.abs(s32.view(np.int32).astype(np.int64)
                             - sig.numpy().view(np.int32).astype(np.int64))) <= 2


def test_rosa_shifted_backward_matches_torch_autograd():
    """oracle.rosa.shifted_backward against torch autograd of the reference's expression
    (model/rosa.py:128-133) in float64 on the CPU, with the sigmoid outputs as leaves; the
    forward's x - prev rounding is fixed by running it in x's dtype and the lerp in float64."""
    import torch
    import torch.nn.functional as F
    from oracle import rosa as orr
    g = torch.Generator().manual_seed(7)
    for dt in (torch.float32, torch.bfloat16):
        x = (torch.randn(3, 21, 40, generator=g) * 2).to(dt)
        sig = torch.sigmoid(torch.randn(3, 40, generator=g) * 2).double().requires_grad_(True)
        xd = x.double().requires_grad_(True)
        prev = F.pad(xd, (0, 0, 1, 0))[:, :-1, :]
        diff_r = (x - F.pad(x, (0, 0, 1, 0))[:, :-1, :]).double()  # rounded in x's dtype
        # x - prev carries x's rounding in value and the identity in gradient
        diff = (xd - prev) + (diff_r - (xd - prev)).detach()
        grads = [torch.randn(3, 21, 40, generator=g, dtype=torch.float64) for _ in range(3)]
        loss = sum(((prev + diff * sig[m]) * grads[m]).sum() for m in range(3))
        loss.backward()
        dx, dsig = orr.shifted_backward(x.float().numpy(), sig.detach().float().numpy(),
                                        [t.numpy() for t in grads], str(dt).split(".")[-1])
        np.testing.assert_allclose(dx, xd.grad.numpy(), rtol=1e-6, atol=1e-9)
        # sig enters the oracle rounded to fp32; the reference keeps it in float64
        np.testing.assert_allclose(dsig, sig.grad.numpy(), rtol=1e-5, atol=1e-6)


def _modes_golden():
    import os
    path = os.path.join(os.path.dirname(__file__), "golden", "ks3_modes_golden.npz")
    return np.load(path)


def test_spine_float_modes_match_reference_golden():
    """oracle.ks3.spine_features_float against the reference's own CPU _spine_features
    ('fp16' bit-exact; 'fp32' within the tanh difference: the oracle's tanh is float64
    rounded to fp32, torch's is its own fp32 routine), on the coordinates and warp scalars
    the reference itself used (tests/golden/make_ks3_modes_golden.py)."""
    from oracle import ks3 as ok
    from oracle.quant import dequantize_last_dim
    g = _modes_golden()
    sc32 = dequantize_last_dim(g["warp_scale_codes"], g["warp_scale_scales"], 128).reshape(-1)
    sh32 = dequantize_last_dim(g["warp_shift_codes"], g["warp_shift_scales"], 128).reshape(-1)
    for mode in ("fp16", "fp32"):
        sc, sh = (ok.h(sc32), ok.h(sh32)) if mode == "fp16" else (sc32, sh32)
        for case in ("std1", "std8"):
            coords = g[f"{mode}/{case}/coords"]
            assert np.array_equal(ok.h(coords), coords)  # fp16 values, as _project makes them
            got = ok.spine_features_float(coords, g["spine_codes"], g["spine_scale"], sc, sh, mode)
            ref = g[f"{mode}/{case}/h"]
            if mode == "fp16":
                assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), case
            else:
                np.testing.assert_allclose(got, ref, rtol=2e-6, atol=1e-6 * np.abs(ref).max())
                assert np.mean(got != ref) < 0.05, case


def test_spine_float_tanh_forms_match_torch_on_every_fp16_input():
    """The fp16 mode's two tanh forms as the kernel evaluates them from the generated
    table (fp16(tanh32(x)) = table(x); fp16(4 tanh32(x)) = 4 table(x) for |x| >= 2^-12,
    4 x below) equal torch's `torch.tanh(x.float()).to(fp16)` and
    `(4.0 * torch.tanh(x.float())).to(fp16)` for every finite fp16 x."""
    import importlib.util
    import os
    import torch
    here = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    spec = importlib.util.spec_from_file_location(
        "gen_tanh16", os.path.join(here, "ksdraft_amd", "csrc", "gen_tanh16.py"))
    gen = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(gen)
    tab = gen.table()
    bits = np.arange(0x7c01, dtype=np.uint32).astype(np.uint16)  # 0 .. +inf
    bits = np.concatenate([bits, bits | 0x8000])
    x16 = bits.view(np.float16)
    m = np.minimum(bits & 0x7fff, gen.LIMIT)
    t1 = tab[m].view(np.float16).astype(np.float32)
    t1 = np.where(bits & 0x8000, -t1, t1)
    xf = x16.astype(np.float32)
    t4 = np.where((bits & 0x7fff) < 0x0c00, 4 * xf, 4 * t1)
    xt = torch.from_numpy(x16.copy()).float()
    ref1 = torch.tanh(xt).to(torch.float16).numpy()
    ref4 = (4.0 * torch.tanh(xt)).to(torch.float16).numpy()
    assert np.array_equal(t1.astype(np.float16).view(np.uint16), ref1.view(np.uint16))
    assert np.array_equal(t4.astype(np.float16).view(np.uint16), ref4.view(np.uint16))
