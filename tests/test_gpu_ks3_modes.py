"""GPU parity of the KS3 cell's 'fp16' and 'fp32' nonlinear modes (reference
ksdraft/kernels/ks3_int8.py:172-203; the fused contract of ks3_triton.py:76-98).

Bars: the 'fp16' spine features bit-exact (against the reference's own CPU outputs in
tests/golden/ks3_modes_golden.npz and against oracle/ks3.py on random coordinates,
composed and fused), the 'fp32' features within the fp32 tanh difference; the feature
codes and scales bit-exact against the oracle quantizer of the kernel's own features;
the cell's composed and fused outputs bit-exact against the oracle chain built with the
ordered-group GEMM contract ('fp16') or within rtol 1e-4 ('fp32'), within 1e-2 of the
reference's CPU outputs, and inside the reference's own cross-path tolerances
(tests/test_ks3_int8.py:48-90).
"""

import os

import numpy as np
import pytest
import torch
from torch import nn

from ksdraft_amd.kernels import ks3_int8 as K
from ksdraft_amd.model.ks3 import KS3
from oracle import gemm as og
from oracle import ks3 as ok
from oracle import quant as oq

pytestmark = pytest.mark.gpu
DEV = "cuda"
GOLD = os.path.join(os.path.dirname(__file__), "golden", "ks3_modes_golden.npz")


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLD, allow_pickle=False)


def _g(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _bits(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    assert a.shape == b.shape, (a.shape, b.shape)
    return bool(np.all((a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))))


def _warp(codes_s, scales_s, codes_h, scales_h):
    sc = oq.dequantize_last_dim(codes_s, scales_s, 128).reshape(-1)
    sh = oq.dequantize_last_dim(codes_h, scales_h, 128).reshape(-1)
    return sc, sh


def _check_h(mode, got, exp):
    if mode == "fp16":
        assert _bits(got, exp)
    else:
        np.testing.assert_allclose(got, exp, rtol=2e-6, atol=1e-6 * np.abs(exp).max())


@pytest.mark.parametrize("mode", ["fp16", "fp32"])
def test_spine_float_reference_golden(gold, mode):
    sc32, sh32 = _warp(gold["warp_scale_codes"], gold["warp_scale_scales"],
                       gold["warp_shift_codes"], gold["warp_shift_scales"])
    sc, sh = (ok.h(sc32), ok.h(sh32)) if mode == "fp16" else (sc32, sh32)
    for case in ("std1", "std8"):
        coords = gold[f"{mode}/{case}/coords"]
        h, hq, hs = K.spine_float(_g(coords.astype(np.float16)), _g(gold["spine_codes"]),
                                  _g(gold["spine_scale"]), _g(sc), _g(sh), mode, want_h=True)
        h = h.cpu().numpy()
        _check_h(mode, h, gold[f"{mode}/{case}/h"])
        eq, es = oq.quantize_last_dim(h)
        assert np.array_equal(hq.cpu().numpy(), eq)
        assert np.array_equal(hs.cpu().numpy().view(np.uint16), es.view(np.uint16))


def _random_spine(seed, Fn):
    rng = np.random.default_rng(seed)
    sq, ss = oq.quantize_last_dim((rng.standard_normal((Fn, 6)) * 0.3).astype(np.float32))
    sc = (np.abs(rng.standard_normal(Fn)) + 0.3).astype(np.float32)
    sh = (rng.standard_normal(Fn) * 0.4).astype(np.float32)
    return sq, ss.reshape(-1), sc, sh


@pytest.mark.parametrize("mode", ["fp16", "fp32"])
@pytest.mark.parametrize("fused", [False, True])
@pytest.mark.parametrize("M,Fn,group", [(70, 256, 128), (33, 136, 32), (40, 130, 64), (5, 13, 32)])
def test_spine_float_random_against_oracle(mode, fused, M, Fn, group):
    """Composed (fp16 coordinates with saturated and subnormal values) and fused (the fp32
    accumulator, values past +-65504 clamped in the kernel) against the oracle."""
    sq, ss, sc, sh = _random_spine(M * 31 + Fn, Fn)
    if mode == "fp16" or fused:  # fp16-valued warp scalars on those paths
        sc, sh = ok.h(sc), ok.h(sh)
    rng = np.random.default_rng(Fn * 7 + M)
    x = (rng.standard_normal((M, Fn)) * 3).astype(np.float32)
    x.flat[::97] = 0.0
    x.flat[5::131] = 70000.0 if fused else 65504.0
    x.flat[7::173] = -1e6 if fused else -65504.0
    x.flat[11::89] = 3e-6
    if not fused:
        x = ok.h(x)
    xin = _g(x) if fused else _g(x.astype(np.float16))
    h, _, _ = K.spine_float(xin, _g(sq), _g(ss), _g(sc), _g(sh), mode, group,
                            want_h=True, want_codes=False)
    _, hq, hs = K.spine_float(xin, _g(sq), _g(ss), _g(sc), _g(sh), mode, group)
    h = h.cpu().numpy()
    exp = ok.spine_features_float(np.clip(x, -65504.0, 65504.0), sq, ss, sc, sh, mode, fused=fused)
    _check_h(mode, h, exp)
    eq, es = oq.quantize_last_dim(h, group)
    assert np.array_equal(hq.cpu().numpy(), eq)
    assert np.array_equal(hs.cpu().numpy().view(np.uint16), es.view(np.uint16))


class _Cell(nn.Module):
    """The attributes KS3Int8Cell reads from a torch KS3 (model/ks3.py)."""

    def __init__(self, gold):
        super().__init__()
        Fn, d = gold["down_weight"].shape
        self.num_charts, self.subspace_rank = Fn, 1
        self.down = nn.Linear(d, Fn, bias=False)
        self.up = nn.Linear(Fn, d, bias=False)
        with torch.no_grad():
            self.down.weight.copy_(torch.from_numpy(gold["down_weight"]))
            self.up.weight.copy_(torch.from_numpy(gold["up_weight"]))
        self.coefficients = nn.Parameter(torch.from_numpy(gold["coefficients"]))
        self.raw_scale = nn.Parameter(torch.from_numpy(gold["raw_scale"]))
        self.raw_shift = nn.Parameter(torch.from_numpy(gold["raw_shift"]))


def _mode_chain(gold, mode, x, fused):
    """The cell's forward from the oracle: ordered-group GEMMs, the mode's spine."""
    p = ok.pack_masters(gold["down_weight"], gold["up_weight"], gold["coefficients"],
                        gold["raw_scale"], gold["raw_shift"])
    for k in ("down_codes", "down_scales", "up_codes", "up_scales", "spine_codes", "spine_scale",
              "warp_scale_codes", "warp_scale_scales", "warp_shift_codes", "warp_shift_scales"):
        assert _bits(p[k], gold[k]) if p[k].dtype.kind == "f" else np.array_equal(p[k], gold[k]), k
    sc32, sh32 = _warp(p["warp_scale_codes"], p["warp_scale_scales"], p["warp_shift_codes"],
                       p["warp_shift_scales"])
    xq, xs = oq.quantize_last_dim(x)
    acc = og.gemm_ordered(xq, xs, p["down_codes"], p["down_scales"])
    if fused:
        xin, sc, sh = np.clip(acc, -65504.0, 65504.0), ok.h(sc32), ok.h(sh32)
    else:
        xin = ok.coords_from_gemm(acc)
        sc, sh = (sc32, sh32) if mode == "fp32" else (ok.h(sc32), ok.h(sh32))
    hv = ok.spine_features_float(xin, p["spine_codes"], p["spine_scale"], sc, sh, mode, fused=fused)
    hq, hs = oq.quantize_last_dim(hv)
    return og.gemm_ordered(hq, hs, p["up_codes"], p["up_scales"])


@pytest.mark.parametrize("mode", ["fp16", "fp32"])
def test_cell_forward_composed_and_fused(gold, mode):
    cell = K.KS3Int8Cell(_Cell(gold).to(DEV), group=128, nonlinear=mode).eval()
    for case in ("std1", "std8"):
        x = gold[f"{mode}/{case}/x"]
        with torch.no_grad():
            yc = K.KS3Int8Cell._forward_composed(cell, _g(x)).cpu().numpy()
            yf = cell(_g(x)).cpu().numpy()
        ec, ef = _mode_chain(gold, mode, x, False), _mode_chain(gold, mode, x, True)
        if mode == "fp16":
            assert _bits(yc, ec) and _bits(yf, ef), case
        else:  # tanhf against the oracle's float64-based tanh, through one requantization
            for got, exp in ((yc, ec), (yf, ef)):
                assert np.linalg.norm(got - exp) / np.linalg.norm(exp) < 1e-4, case
        ref = gold[f"{mode}/{case}/y"]
        np.testing.assert_allclose(yc, ref, rtol=1e-2, atol=1e-2 * np.abs(ref).max())
        # the reference's cross-path check (tests/test_ks3_int8.py:82-84)
        assert np.linalg.norm(yf - yc) / np.linalg.norm(yc) < 0.05, case


@pytest.mark.parametrize("mode", ["fp32", "fp16", "int8"])
def test_cell_modes_against_float_ks3(mode):
    """tests/test_ks3_int8.py:48-90 on the GPU: each mode within 5% (8% for 'int8') of the
    float KS3, and the fused eval path within 5% of the composed one."""
    torch.manual_seed(1)
    cell = KS3(96, 368).to(DEV)
    with torch.no_grad():
        cell.up.weight.normal_(0, 0.05)
    x = torch.randn(8, 96, device=DEV)
    with torch.no_grad():
        ref = cell(x)
        q = K.KS3Int8Cell(cell, group=128, nonlinear=mode).eval()
        rel = ((q(x) - ref).norm() / ref.norm()).item()
    assert rel < (0.08 if mode == "int8" else 0.05), (mode, rel)
    torch.manual_seed(2)
    cell = KS3(96, 368).to(DEV)
    with torch.no_grad():
        cell.up.weight.normal_(0, 0.05)
        cell.coefficients.normal_(0, 0.3)
        x = torch.randn(64, 96, device=DEV)
        ref = cell(x)
        q = K.KS3Int8Cell(cell, group=128, nonlinear=mode).eval()
        yf = q(x)
        yc = K.KS3Int8Cell._forward_composed(q, x)
    assert ((yf - yc).norm() / yc.norm()).item() < 0.05, mode
    assert ((yf - ref).norm() / ref.norm()).item() < 0.08, mode


def test_trainable_cell_fp16_mode(gold):
    """Training in the 'fp16' mode: the forward is the oracle chain's bit for bit, and the
    backward (mode-independent geometry VJP, ks3_int8.py:341-429) equals the 'int8' cell's
    where it does not read the features (dx, ddown), while dup follows the fp16 features."""
    base = _Cell(gold).to(DEV)
    c16 = K.KS3Int8Cell(base, group=128, nonlinear="fp16", trainable=True)
    c8 = K.KS3Int8Cell(base, group=128, nonlinear="int8", trainable=True)
    x = gold["fp16/std1/x"]
    gout = np.random.default_rng(3).standard_normal(x.shape).astype(np.float32) * 0.1
    outs = []
    for c in (c16, c8):
        xt = _g(x).requires_grad_(True)
        y = c(xt)
        y.backward(_g(gout))
        outs.append((y.detach().cpu().numpy(), xt.grad.cpu().numpy(),
                     c.master_down.grad.float().cpu().numpy(), c.master_up.grad.float().cpu().numpy()))
    assert _bits(outs[0][0], _mode_chain(gold, "fp16", x, False))
    assert _bits(outs[0][1], outs[1][1]) and _bits(outs[0][2], outs[1][2])
    assert np.all(np.isfinite(outs[0][3])) and not _bits(outs[0][3], outs[1][3])


def test_rank_above_one_raises_like_the_reference():
    cell = KS3(64, 16, subspace_rank=2).to(DEV)
    q = K.KS3Int8Cell(cell, group=128, nonlinear="fp16").eval()
    with pytest.raises(RuntimeError):
        q(torch.randn(4, 64, device=DEV))
