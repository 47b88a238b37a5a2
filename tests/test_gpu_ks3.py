"""GPU parity: the KS3 int8 cell kernels against the oracle (oracle/ks3.py) and the
golden vectors written from the reference's CPU path (tests/golden/ks3_int8_golden.npz).

Bars: tanh table, spine features, feature codes/scales, dc and both dc operand layouts
bit-exact; the eight column reductions within rtol 2e-3 (fp32 sums in another order
than torch's, then fp16); the trainable cell's forward output and backward GEMM outputs
bit-exact against the oracle chain built with the ordered-group GEMM contract, and within
the reference's tolerances of the golden (reference CPU) outputs.
"""

import os

import numpy as np
import pytest
import torch
from torch import nn

from ksdraft_amd.kernels import ks3_int8 as K
from ksdraft_amd.kernels.ks3_triton import project_fused
from oracle import gemm as og
from oracle import ks3 as ok
from oracle import quant as oq

pytestmark = pytest.mark.gpu
DEV = "cuda"
GOLD = os.path.join(os.path.dirname(__file__), "golden", "ks3_int8_golden.npz")


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLD, allow_pickle=False)


def _g(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _f16(a):
    return _g(np.asarray(a, np.float32).astype(np.float16))


def _bits_eq(a, b):
    """Bit equality; two NaNs count as equal (x86 and gfx950 make different default NaNs)."""
    a = np.asarray(a)
    b = np.asarray(b)
    assert a.shape == b.shape, (a.shape, b.shape)
    if a.dtype.kind == "f":
        b = b.astype(a.dtype)
        both_nan = np.isnan(a) & np.isnan(b)
        ua = a.view(np.uint16 if a.itemsize == 2 else np.uint32)
        ub = b.view(np.uint16 if a.itemsize == 2 else np.uint32)
        return bool(np.all((ua == ub) | both_nan))
    return np.array_equal(a, b)


def _random_cell(seed, Fn, coeff_std=0.3):
    rng = np.random.default_rng(seed)
    coeffs = (rng.standard_normal((Fn, 6)) * coeff_std).astype(np.float32)
    raw_scale = (0.75 + rng.standard_normal(Fn) * 0.3).astype(np.float32)
    raw_shift = (rng.standard_normal(Fn) * 0.5).astype(np.float32)
    sq, ss = oq.quantize_last_dim(coeffs)
    ss = ss.reshape(-1)
    scale_t = (np.log1p(np.exp(-np.abs(raw_scale.astype(np.float64)))) +
               np.maximum(raw_scale, 0)).astype(np.float32) + np.float32(1e-4)
    shift_t = (np.float32(0.5) * ok.tanh32(raw_shift)).astype(np.float32)
    wsc, wss = oq.quantize_last_dim(scale_t.reshape(-1, 1))
    whc, whs = oq.quantize_last_dim(shift_t.reshape(-1, 1))
    sc, sh = ok.warp_scalars(wsc, wss, whc, whs)
    coef, _, _ = ok.spine_params(sq, ss, wsc, wss, whc, whs)
    return dict(spine_codes=sq, spine_scale=ss, sc=sc, sh=sh, raw_scale=raw_scale,
                raw_shift=raw_shift, coef=coef)


def _random_coords(seed, M, Fn, scale=2.0, saturated=True):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((M, Fn)) * scale).astype(np.float32)
    x.flat[::97] = 0.0
    if saturated:                  # the GEMM epilogue's clamp values
        x.flat[5::131] = 65504.0
        x.flat[7::173] = -65504.0
    x.flat[11::89] = 3e-6          # fp16 subnormal
    return x.astype(np.float16).astype(np.float32)


# ---------------------------------------------------------------- tanh table
def test_tanh16_every_fp16_input():
    bits = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16)
    x = bits.view(np.float16)
    finite = np.isfinite(x)
    y = K.tanh16(_g(x)).cpu().numpy()
    want = ok.h(ok.tanh32(x[finite].astype(np.float32))).astype(np.float16)
    assert np.array_equal(y[finite].view(np.uint16), want.view(np.uint16))
    inf = np.isinf(x)
    assert np.array_equal(y[inf], np.sign(x[inf]).astype(np.float16))


# ---------------------------------------------------------------- spine forward
@pytest.mark.parametrize("case", ["std1", "std8"])
def test_spine_golden_bit_exact(gold, case):
    sc, sh = ok.warp_scalars(gold["warp_scale_codes"], gold["warp_scale_scales"],
                             gold["warp_shift_codes"], gold["warp_shift_scales"])
    coords = gold[f"{case}/coords"]
    h, hq, hs = K.spine_int8(_f16(coords), _g(gold["spine_codes"]), _g(gold["spine_scale"]),
                             _f16(sc), _f16(sh), _g(gold["tanh_lut"]), 128, want_h=True)
    assert _bits_eq(h.cpu().numpy(), gold[f"{case}/h"])
    eq, es = oq.quantize_last_dim(gold[f"{case}/h"])
    assert _bits_eq(hq.cpu().numpy(), eq) and _bits_eq(hs.cpu().numpy(), es)


@pytest.mark.parametrize("M,Fn,group", [(64, 256, 128), (200, 384, 32), (77, 130, 64),
                                        (130, 257, 128), (1, 5, 32), (333, 1000, 128)])
def test_spine_random_shapes_bit_exact(M, Fn, group):
    cell = _random_cell(M + Fn, Fn)
    coords = _random_coords(M * 7 + Fn, M, Fn)
    lut = ok.make_tanh_lut()
    h, hq, hs = K.spine_int8(_f16(coords), _g(cell["spine_codes"]), _g(cell["spine_scale"]),
                             _f16(cell["sc"]), _f16(cell["sh"]), _g(lut), group, want_h=True)
    exp = ok.spine_features_int8(coords, cell["spine_codes"], cell["spine_scale"], cell["sc"],
                                 cell["sh"], lut)
    assert _bits_eq(h.cpu().numpy(), exp)
    eq, es = oq.quantize_last_dim(exp, group)
    assert _bits_eq(hq.cpu().numpy(), eq) and _bits_eq(hs.cpu().numpy(), es)


@pytest.mark.parametrize("M,Fn,group", [(64, 256, 128), (100, 384, 32), (33, 130, 64),
                                        (70, 257, 128)])
def test_spine_fused_contract_bit_exact(M, Fn, group):
    cell = _random_cell(3 * M + Fn, Fn)
    rng = np.random.default_rng(M)
    acc = (rng.standard_normal((M, Fn)) * 2.5).astype(np.float32)
    acc.flat[::51] = 1e5  # beyond the fp16 range: clamped
    lut = ok.make_tanh_lut()
    hq, hs = K.spine_fused_int8(_g(acc), _g(cell["spine_codes"]), _g(cell["spine_scale"]),
                                _f16(cell["sc"]), _f16(cell["sh"]), _g(lut), group)
    eq, es = ok.spine_fused_int8(acc, cell["spine_codes"], cell["spine_scale"], cell["sc"],
                                 cell["sh"], lut, group)
    assert _bits_eq(hq.cpu().numpy(), eq) and _bits_eq(hs.cpu().numpy(), es)


@pytest.mark.parametrize("M,K,Fn", [(64, 128, 256), (200, 384, 130), (1, 256, 5),
                                     (333, 1536, 1000), (130, 2048, 300), (1000, 512, 640)])
def test_project_fused_one_launch_bit_exact(M, K, Fn):
    """project_fused 'int8', group 128, one_launch: the GEMM whose epilogue runs the spine
    and both requantizations (one launch after the table) against the oracle chain, the ordered
    sum over all K groups then the fused contract. Covers ragged M and F (partial tiles,
    charts past F), a K that the standalone GEMM would split (2048 with 6 tiles), and
    accumulators beyond the fp16 range (rows with large scales, clamped)."""
    cell = _random_cell(5 * M + Fn, Fn)
    rng = np.random.default_rng(M + K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    x[::7] *= 3e5  # large rows: accumulators past +-65504
    w = (rng.standard_normal((Fn, K)) * 0.05).astype(np.float32)
    xq, xs = oq.quantize_last_dim(x)
    wq, ws = oq.quantize_last_dim(w)
    lut = ok.make_tanh_lut()
    acc = og.gemm_ordered(xq, xs, wq, ws)
    assert (np.abs(acc) > 65504).any()
    eq, es = ok.spine_fused_int8(acc, cell["spine_codes"], cell["spine_scale"], cell["sc"],
                                 cell["sh"], lut, 128)
    hq, hs = project_fused(_g(xq), _g(xs), _g(wq), _g(ws), _g(cell["spine_codes"]),
                           _g(cell["spine_scale"]), _f16(cell["sc"]), _f16(cell["sh"]), _g(lut),
                           128, "int8", one_launch=True)
    assert _bits_eq(hq.cpu().numpy(), eq) and _bits_eq(hs.cpu().numpy(), es)
    # the two-launch form: the same outputs wherever the standalone GEMM does not split
    # K (its split parts are summed in order, the one launch never splits)
    args = (_g(xq), _g(xs), _g(wq), _g(ws), _g(cell["spine_codes"]), _g(cell["spine_scale"]),
            _f16(cell["sc"]), _f16(cell["sh"]), _g(lut), 128, "int8")
    hq2, hs2 = project_fused(*args, one_launch=False)
    if K < 2048:
        assert torch.equal(hq, hq2) and torch.equal(hs, hs2)
    # the default picks one of the two by shape, with the same outputs as the form it picks
    hq3, hs3 = project_fused(*args)
    pick = (hq, hs) if M <= 1024 and K < 2048 else (hq2, hs2)
    assert torch.equal(hq3, pick[0]) and torch.equal(hs3, pick[1])


# ---------------------------------------------------------------- VJP
def _check_vjp(out, value, coords, coef, sc, sh, raw_scale, raw_shift, group):
    dc, sums, dcoeff, dscale, dshift = ok.vjp(value, coords, coef, sc, sh, raw_scale, raw_shift)
    assert _bits_eq(out["dc"].cpu().numpy(), dc.astype(np.float16))
    eq, es = oq.quantize_last_dim(dc, group)
    assert _bits_eq(out["dc_codes"].cpu().numpy(), eq)
    assert _bits_eq(out["dc_scales"].cpu().numpy(), es)
    tq, ts = oq.quantize_last_dim(np.ascontiguousarray(dc.T), group)
    assert _bits_eq(out["dct_codes"].cpu().numpy(), tq)
    assert _bits_eq(out["dct_scales"].cpu().numpy(), ts)
    got = out["sums"].cpu().numpy()
    fin = np.isfinite(sums)
    assert np.array_equal(np.isfinite(got), fin)
    mag = np.where(fin, np.abs(sums), 0).max(axis=1, keepdims=True) + 1e-30
    assert (np.abs(got - sums) <= 2e-3 * np.abs(sums) + 1e-5 * mag)[fin].all()
    return dcoeff, dscale, dshift


@pytest.mark.parametrize("case", ["std1", "std8"])
def test_vjp_golden(gold, case):
    coef, sc, sh = ok.spine_params(gold["spine_codes"], gold["spine_scale"],
                                   gold["warp_scale_codes"], gold["warp_scale_scales"],
                                   gold["warp_shift_codes"], gold["warp_shift_scales"])
    value = gold[f"{case}/value"].astype(np.float32)
    coords = gold[f"{case}/coords"]
    out = K.ks3_vjp(_f16(value), _f16(coords), _g(gold["spine_codes"]), _g(gold["spine_scale"]),
                    _f16(sc), _f16(sh), _g(gold["master_raw_scale"]),
                    _g(gold["master_raw_shift"]), 128, want_dc=True, want_sums=True)
    assert _bits_eq(out["dc"].cpu().numpy(), gold[f"{case}/dc"].astype(np.float16))
    _check_vjp(out, value, coords, coef, sc, sh, gold["master_raw_scale"],
               gold["master_raw_shift"], 128)
    ref = gold[f"{case}/dcoeff"].reshape(-1, 6).astype(np.float32)
    np.testing.assert_allclose(out["dcoeff"].float().cpu().numpy(), ref, rtol=2e-3,
                               atol=1e-3 * np.abs(ref).max())
    for k in ("dscale", "dshift"):
        r = gold[f"{case}/{k}"].astype(np.float32)
        np.testing.assert_allclose(out[k].float().cpu().numpy(), r, rtol=2e-3,
                                   atol=1e-3 * np.abs(r).max() + 1e-12)


@pytest.mark.parametrize("M,Fn,group", [(256, 256, 128), (200, 384, 32), (77, 130, 64),
                                        (130, 257, 128), (300, 129, 32), (1, 6, 128)])
def test_vjp_random_shapes(M, Fn, group):
    cell = _random_cell(11 * M + Fn, Fn)
    coef = cell["coef"]
    coords = _random_coords(M + 5 * Fn, M, Fn, scale=3.0, saturated=False)
    rng = np.random.default_rng(M * Fn)
    value = ok.h((rng.standard_normal((M, Fn)) * 0.05).astype(np.float32))
    out = K.ks3_vjp(_f16(value), _f16(coords), _g(cell["spine_codes"]), _g(cell["spine_scale"]),
                    _f16(cell["sc"]), _f16(cell["sh"]), _g(cell["raw_scale"]),
                    _g(cell["raw_shift"]), group, want_dc=True, want_sums=True)
    dcoeff, dscale, dshift = _check_vjp(out, value, coords, coef, cell["sc"], cell["sh"],
                                        cell["raw_scale"], cell["raw_shift"], group)
    ref = np.concatenate([dcoeff.reshape(-1), dscale, dshift]).astype(np.float32)
    got = np.concatenate([out["dcoeff"].float().cpu().numpy().reshape(-1),
                          out["dscale"].float().cpu().numpy(), out["dshift"].float().cpu().numpy()])
    np.testing.assert_allclose(got, ref, rtol=4e-3, atol=2e-3 * np.abs(ref).max() + 1e-12)


def test_vjp_saturated_coordinates():
    """Coordinates at the +-65504 clamp overflow the fp16 VJP to inf/NaN, as in the
    reference: dc and its codes stay bit-exact (NaN groups: scale 0x7fff, codes 0) and the
    sums are non-finite exactly where the oracle's are."""
    M, Fn, group = 256, 256, 128
    cell = _random_cell(5, Fn)
    coords = _random_coords(6, M, Fn, scale=3.0, saturated=True)
    value = ok.h((np.random.default_rng(7).standard_normal((M, Fn)) * 0.05).astype(np.float32))
    out = K.ks3_vjp(_f16(value), _f16(coords), _g(cell["spine_codes"]), _g(cell["spine_scale"]),
                    _f16(cell["sc"]), _f16(cell["sh"]), _g(cell["raw_scale"]),
                    _g(cell["raw_shift"]), group, want_dc=True, want_sums=True)
    with np.errstate(all="ignore"):
        _check_vjp(out, value, coords, cell["coef"], cell["sc"], cell["sh"], cell["raw_scale"],
                   cell["raw_shift"], group)
    assert not np.isfinite(out["dc"].float().cpu().numpy()).all()


# ---------------------------------------------------------------- the trainable cell
class _Cell(nn.Module):
    """The attributes KS3Int8Cell reads from a torch KS3 (reference model/ks3.py:69-91)."""

    def __init__(self, gold):
        super().__init__()
        Fn, d = gold["master_down"].shape
        self.num_charts, self.subspace_rank = Fn, 1
        self.down = nn.Linear(d, Fn, bias=False)
        self.up = nn.Linear(Fn, d, bias=False)
        with torch.no_grad():
            self.down.weight.copy_(torch.from_numpy(gold["master_down"]))
            self.up.weight.copy_(torch.from_numpy(gold["master_up"]))
        self.coefficients = nn.Parameter(torch.from_numpy(gold["master_coefficients"].reshape(Fn, 6)))
        self.raw_scale = nn.Parameter(torch.from_numpy(gold["master_raw_scale"]))
        self.raw_shift = nn.Parameter(torch.from_numpy(gold["master_raw_shift"]))


def _oracle_cell_chain(gold, x, grad_out):
    """Forward and backward of the trainable cell from the oracle, with the ordered-group
    GEMM contract for every GEMM (ks3_int8.py:326-429)."""
    p = ok.pack_masters(gold["master_down"], gold["master_up"], gold["master_coefficients"],
                        gold["master_raw_scale"], gold["master_raw_shift"])
    sc, sh = ok.warp_scalars(p["warp_scale_codes"], p["warp_scale_scales"],
                             p["warp_shift_codes"], p["warp_shift_scales"])
    lut = ok.make_tanh_lut()
    xq, xs = oq.quantize_last_dim(x)
    coords = ok.coords_from_gemm(og.gemm_ordered(xq, xs, p["down_codes"], p["down_scales"]))
    h = ok.spine_features_int8(coords, p["spine_codes"], p["spine_scale"], sc, sh, lut)
    hq, hs = oq.quantize_last_dim(h)
    y = og.gemm_ordered(hq, hs, p["up_codes"], p["up_scales"])
    g16 = ok.h(grad_out)
    gq, gs = oq.quantize_last_dim(g16)
    upT = oq.requant_transpose(p["up_codes"], p["up_scales"])
    value = ok.h(og.gemm_ordered(gq, gs, *upT))
    coef, _, _ = ok.spine_params(p["spine_codes"], p["spine_scale"], p["warp_scale_codes"],
                                 p["warp_scale_scales"], p["warp_shift_codes"], p["warp_shift_scales"])
    dc, sums, dcoeff, dscale, dshift = ok.vjp(value, coords, coef, sc, sh,
                                              gold["master_raw_scale"], gold["master_raw_shift"])
    dcq, dcs = oq.quantize_last_dim(dc)
    dx = og.gemm_ordered(dcq, dcs, *oq.requant_transpose(p["down_codes"], p["down_scales"]))
    dtq, dts = oq.quantize_last_dim(np.ascontiguousarray(dc.T))
    ddown = og.gemm_ordered(dtq, dts, *oq.requant_transpose(xq, xs))
    gtq, gts = oq.quantize_last_dim(np.ascontiguousarray(g16.T))
    dup = og.gemm_ordered(gtq, gts, *oq.requant_transpose(hq, hs))
    return dict(y=y, value=value, dx=dx, ddown=ddown, dup=dup, dcoeff=dcoeff, dscale=dscale,
                dshift=dshift, packed=p)


@pytest.mark.parametrize("case", ["std1", "std8"])
def test_trainable_cell_forward_backward(gold, case):
    cell = K.KS3Int8Cell(_Cell(gold).to(DEV), group=128, nonlinear="int8", trainable=True)
    x = _g(gold[f"{case}/x"]).requires_grad_(True)
    grad_out = _g(gold[f"{case}/grad_out"])
    y = cell(x)
    y.backward(grad_out)
    ref = _oracle_cell_chain(gold, gold[f"{case}/x"], gold[f"{case}/grad_out"])
    p = ref["packed"]
    for k in ("spine_codes", "spine_scale", "down_codes", "down_scales", "up_codes", "up_scales",
              "warp_scale_codes", "warp_scale_scales", "warp_shift_codes", "warp_shift_scales"):
        assert _bits_eq(getattr(cell, k).cpu().numpy().reshape(p[k].shape), p[k]), k
    assert _bits_eq(y.detach().cpu().numpy(), ref["y"])
    assert _bits_eq(x.grad.cpu().numpy(), ref["dx"])
    # _grad_handoff: fp16 when that is finite, else fp32 (ks3_int8.py:75-84); autograd
    # stores the result in the fp32 masters' dtype
    def handoff(t):
        t16 = ok.h(t)
        return t16 if np.isfinite(t16).all() else t
    assert cell.master_down.grad.dtype == torch.float32
    assert _bits_eq(cell.master_down.grad.cpu().numpy(), handoff(ref["ddown"]))
    assert _bits_eq(cell.master_up.grad.cpu().numpy(), handoff(ref["dup"]))
    np.testing.assert_allclose(cell.master_coefficients.grad.float().cpu().numpy().reshape(-1, 6),
                               ref["dcoeff"], rtol=4e-3, atol=2e-3 * np.abs(ref["dcoeff"]).max())
    # against the reference's own CPU outputs (its GEMMs sum in another order)
    np.testing.assert_allclose(y.detach().cpu().numpy(), gold[f"{case}/y"], rtol=1e-2, atol=1e-3)
    for k, got in (("dx", x.grad), ("ddown", cell.master_down.grad), ("dup", cell.master_up.grad)):
        r = gold[f"{case}/{k}"].astype(np.float32)
        if not np.isfinite(r).all():
            continue  # the fixture holds the fp16 view; the reference handed off fp32 here
        g = got.float().cpu().numpy()
        cos = float((g * r).sum() / (np.linalg.norm(g) * np.linalg.norm(r)))
        assert cos > 0.99, (k, cos)


def test_eval_forward_fused_contract(gold):
    cell = K.KS3Int8Cell(_Cell(gold).to(DEV), group=128, nonlinear="int8").eval()
    x = gold["std1/x"]
    with torch.no_grad():
        y = cell(_g(x)).cpu().numpy()
    p = ok.pack_masters(gold["master_down"], gold["master_up"], gold["master_coefficients"],
                        gold["master_raw_scale"], gold["master_raw_shift"])
    sc, sh = ok.warp_scalars(p["warp_scale_codes"], p["warp_scale_scales"],
                             p["warp_shift_codes"], p["warp_shift_scales"])
    xq, xs = oq.quantize_last_dim(x)
    acc = og.gemm_ordered(xq, xs, p["down_codes"], p["down_scales"])
    hq, hs = ok.spine_fused_int8(acc, p["spine_codes"], p["spine_scale"], sc, sh, ok.make_tanh_lut())
    assert _bits_eq(y, og.gemm_ordered(hq, hs, p["up_codes"], p["up_scales"]))
    ref = gold["std1/y"]
    assert np.linalg.norm(y - ref) / np.linalg.norm(ref) < 0.05
    with torch.no_grad():
        yc = K.KS3Int8Cell._forward_composed(cell, _g(x)).cpu().numpy()
    assert _bits_eq(yc, _oracle_cell_chain(gold, x, np.zeros_like(x))["y"])


def test_project_and_spine_features_api(gold):
    cell = K.KS3Int8Cell(_Cell(gold).to(DEV), group=128).eval()
    x = gold["std8/x"]
    xq, xs = K.quantize_last_dim(_g(x))
    h, coords = cell._project(xq, xq, xs, cell.down_codes, cell.down_scales)
    assert coords.shape == (x.shape[0], cell.num_subspaces, 1) and coords.dtype == torch.float32
    exp = ok.spine_features_int8(coords.reshape(x.shape[0], -1).cpu().numpy(),
                                 cell.spine_codes.cpu().numpy(), cell.spine_scale.cpu().numpy(),
                                 *[t.float().cpu().numpy() for t in cell._warp_scalars(torch.float16)],
                                 cell.tanh_lut.cpu().numpy())
    assert _bits_eq(h.cpu().numpy(), exp)
    c = cell.spine_codes.reshape(-1, 1, 6)
    scale, shift = cell._warp_scalars(torch.float16)
    h2 = cell._spine_features(coords, coords, *(c[..., k] for k in range(6)),
                              cell.spine_scale, scale, shift)
    assert torch.equal(h2.reshape(h.shape), h)
    with pytest.raises(ValueError):
        K.KS3Int8Cell(_Cell(gold).to(DEV), nonlinear="bf16")


@pytest.mark.parametrize("case", ["finite", "overflow", "nan", "in_place"])
def test_grad_handoff_entry_point(case):
    """ksd_grad_handoff through the C ABI: fp32(fp16(t)) when every element is finite in
    fp16, else t unchanged (ks3_int8.py:75-84), with out separate from t or aliasing it."""
    from ksdraft_amd import _lib
    g = torch.Generator().manual_seed(7)
    t = torch.randn(3 * 2048 + 37, generator=g) * 100.0
    if case == "overflow":
        t[4001] = 70000.0
    if case == "nan":
        t[17] = float("nan")
    want = t.clone() if case in ("overflow", "nan") else t.half().float()
    td = t.to("cuda")
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    out = td if case == "in_place" else torch.full_like(td, -1.0)
    _lib.call("ksd_grad_handoff", td.data_ptr(), td.numel(), flag.data_ptr(), out.data_ptr(),
              _lib.stream_ptr(td.device))
    torch.cuda.synchronize()
    got = out.cpu()
    assert torch.equal(got.view(torch.int32), want.view(torch.int32)) or (
        case == "nan" and torch.equal(torch.nan_to_num(got), torch.nan_to_num(want)))
    assert int(flag.item()) == (1 if case in ("overflow", "nan") else 0)


def test_warp_scalars_follow_their_codes(gold):
    """The dequantized warp scale/shift are reused while their code and scale tensors are
    unchanged, and recomputed after a repack of the masters or an in-place edit."""
    from ksdraft_amd.kernels.quant import dequantize_last_dim
    cell = K.KS3Int8Cell(_Cell(gold).to(DEV), group=128, nonlinear="int8", trainable=True)

    def fresh():
        return (dequantize_last_dim(cell.warp_scale_codes, cell.warp_scale_scales, 128).reshape(-1).half(),
                dequantize_last_dim(cell.warp_shift_codes, cell.warp_shift_scales, 128).reshape(-1).half())

    s1, h1 = cell._warp_scalars(torch.float16)
    assert cell._warp_scalars(torch.float16)[0] is s1
    assert torch.equal(s1, fresh()[0]) and torch.equal(h1, fresh()[1])
    with torch.no_grad():
        cell.master_raw_scale.add_(0.5)
        cell.master_raw_shift.add_(0.25)
    cell._repack_masters()
    s2, h2 = cell._warp_scalars(torch.float16)
    assert torch.equal(s2, fresh()[0]) and torch.equal(h2, fresh()[1])
    assert not torch.equal(s2, s1)
    with torch.no_grad():
        cell.warp_shift_codes.neg_()
    s3, h3 = cell._warp_scalars(torch.float16)
    assert torch.equal(h3, fresh()[1]) and not torch.equal(h3, h2)


def test_cell_built_and_run_under_inference_mode(gold):
    """A cell built, converted and evaluated inside torch.inference_mode (whose tensors
    carry no version counter) gives the same output as one built outside it; the warp
    scalars are then dequantized every call instead of cached."""
    x = _g(gold["std1/x"])
    ref_cell = K.KS3Int8Cell(_Cell(gold).to(DEV), group=128, nonlinear="int8").eval()
    with torch.no_grad():
        ref = ref_cell(x)
    with torch.inference_mode():
        cell = K.KS3Int8Cell(_Cell(gold).to(DEV), group=128, nonlinear="int8").eval()
        y1 = cell(x)
        y2 = cell(x)
        yc = K.KS3Int8Cell._forward_composed(cell, x)
    assert torch.equal(y1, ref) and torch.equal(y2, ref)
    with torch.no_grad():
        assert torch.equal(yc, K.KS3Int8Cell._forward_composed(ref_cell, x))
