"""GPU parity at the BASELINE configs' full shapes (configs 2, 3 and 4).

Each test runs the product path at the shape bench.py times and checks it stage by stage
against the oracle: int8 codes, fp16 scales and GEMM outputs bit-exact (the GEMMs against
the ordered-group contract, oracle/gemm.py), every stage fed the previous stage's device
output once that output has itself been checked. Stages whose oracle is row-local are
checked on sampled rows (and, for the transposed operands, on whole sampled 128-row
groups); stages that reduce over the tokens are checked on sampled output rows with the
full device operands.

Configs: 2 = one W8A8 linear layer fwd + dX + dW at M = 8192, K = N = 1536;
3 = the LM head at M = 4096, K = 1536, N = 150144 with dY = softmax - onehot; 4 = the
trainable KS3 cell at d = 1536, F = 5888, B 4 x T 2048 and the Rosa step with 512 streams.
"""

import numpy as np
import pytest
import torch
from torch import nn

from ksdraft_amd import train as T
from ksdraft_amd.kernels import Int8Linear
from ksdraft_amd.kernels import gemm as kg
from ksdraft_amd.kernels import ks3_int8 as K
from ksdraft_amd.kernels import quant as kq
from ksdraft_amd.kernels import rosa as R
from ksdraft_amd.kernels.rosa_credit_gpu import HardRosaGPU
from oracle import gemm as og
from oracle import ks3 as ok
from oracle import quant as oq
from oracle import rosa as orr

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _np(t):
    return t.detach().cpu().numpy()


def _eq(a, b):
    a, b = np.asarray(a), np.asarray(b)
    assert a.shape == b.shape, (a.shape, b.shape)
    if a.dtype.kind == "f":
        u = np.uint16 if a.itemsize == 2 else np.uint32
        return np.array_equal(a.view(u), b.astype(a.dtype).view(u))
    return np.array_equal(a, b)


def _rows(n, k, seed):
    return np.sort(np.random.default_rng(seed).choice(n, k, replace=False))


# ------------------------------------------------------------------------------ config 2
def test_config2_linear_forward_backward_full_shape():
    """Int8Linear fwd + int8 dX + int8 dW at M = 8192, K = N = 1536 (X ~ N(0,1), W ~
    N(0,0.02), dY ~ N(0,1e-2), seed 0): every output element against the oracle chain of
    the recipe (dX = Q(dY) . requantT(W); dW = QT(dY) . requantT(Q(X)))."""
    M, Kd, N = 8192, 1536, 1536
    g = torch.Generator().manual_seed(0)
    x = torch.randn(M, Kd, generator=g)
    w = torch.randn(N, Kd, generator=g) * 0.02
    dy = torch.randn(M, N, generator=g) * 1e-2
    lin = Int8Linear(Kd, N, bias=False).to(DEV)
    with torch.no_grad():
        lin.weight.copy_(w)
    xd = x.to(DEV).requires_grad_(True)
    y = lin(xd)
    y.backward(dy.to(DEV))
    torch.cuda.synchronize()

    xq, xs = oq.quantize_last_dim(x.numpy())
    wq, ws = oq.quantize_last_dim(w.numpy())
    assert _eq(_np(lin.weight_codes), wq) and _eq(_np(lin.weight_scales), ws)
    assert _eq(_np(y), og.gemm_ordered(xq, xs, wq, ws))
    gq, gs = oq.quantize_last_dim(dy.numpy())
    assert _eq(_np(xd.grad), og.gemm_ordered(gq, gs, *oq.requant_transpose(wq, ws)))
    gtq, gts = oq.quantize_transpose(dy.numpy())
    assert _eq(_np(lin.weight.grad), og.gemm_ordered(gtq, gts, *oq.requant_transpose(xq, xs)))
    # the device operands themselves (one dual pass each for X and dY)
    c, s, ct, st = kq.quantize_dual(dy.to(DEV))
    assert _eq(_np(c), gq) and _eq(_np(s), gs) and _eq(_np(ct), gtq) and _eq(_np(st), gts)
    c, s, ct, st = kq.quantize_dual(x.to(DEV), t_from_codes=True)
    xtq, xts = oq.requant_transpose(xq, xs)
    assert _eq(_np(c), xq) and _eq(_np(ct), xtq) and _eq(_np(st), xts)


# ------------------------------------------------------------------------------ config 3
def test_config3_lm_head_full_shape():
    """The int8 LM head at M = 4096, K = 1536, N = 150144: fp32 logits, the fused
    cross-entropy gradient's two int8 layouts, dX (K = 150144 over 1173 groups) and dW
    (150144 rows over M = 4096), each on sampled rows against the oracle; the loss and
    dY against float64 torch on the device's logits."""
    M, Kd, N = 4096, 1536, 150144
    g = torch.Generator().manual_seed(0)
    x = torch.randn(M, Kd, generator=g).to(DEV)
    w = (torch.randn(N, Kd, generator=g) * 0.02).to(DEV)
    t = torch.randint(0, N, (M,), generator=g).to(DEV)
    wq, ws = kq.quantize_last_dim(w)
    rows_w = _rows(N, 64, 1)
    ewq, ews = oq.quantize_last_dim(_np(w[rows_w]))
    assert _eq(_np(wq[rows_w]), ewq) and _eq(_np(ws[rows_w]), ews)

    from ksdraft_amd.kernels.linear import w8a8_linear_forward_train
    y, xtq, xts = w8a8_linear_forward_train(x, wq, ws, None, 128, torch.float32)
    xq, xs = oq.quantize_last_dim(_np(x))
    rows = _rows(M, 32, 2)
    assert _eq(_np(y[rows]), og.gemm_ordered(xq[rows], xs[rows], _np(wq), _np(ws),
                                                     splits=og.splits_for(M, N, Kd)))
    exq, exs = oq.requant_transpose(xq, xs)
    assert _eq(_np(xtq), exq) and _eq(_np(xts), exs)

    loss, rmax, rinv, n = T.cross_entropy_stats(y, t)
    y64 = y.double()
    eloss = torch.nn.functional.cross_entropy(y64, t)
    assert abs(loss.item() - eloss.item()) <= 2e-5 * abs(eloss.item())
    gsc = torch.ones(1, device=DEV) / n
    (gq, gs, gtq, gts), dy = T.cross_entropy_grad_int8(y, t, rmax, rinv, gsc, return_dy=True)
    edy = torch.softmax(y64[rows], dim=1)
    edy[torch.arange(len(rows)), t[rows]] -= 1.0
    edy /= M
    assert (dy[rows].double() - edy).abs().max().item() <= 1e-5 / M
    dyr = _np(dy[rows])
    eq, es = oq.quantize_last_dim(dyr)
    assert _eq(_np(gq[rows]), eq) and _eq(_np(gs[rows]), es)
    vrows = _rows(N, 48, 3)  # vocabulary rows of dY^T (each quantized along all 4096 tokens)
    eq, es = oq.quantize_last_dim(np.ascontiguousarray(_np(dy[:, vrows]).T))
    assert _eq(_np(gtq[vrows]), eq) and _eq(_np(gts[vrows]), es)
    del dy, y64

    # dX = dY . W: W^T requantized along the vocabulary (1536 rows of 150144)
    wtq, wts = kq.requant_transpose(wq, ws)
    krows = _rows(Kd, 16, 4)
    real = _np(kq.dequantize_last_dim(wq, ws)[:, krows]).T  # (16, N)
    eq, es = oq.quantize_last_dim(np.ascontiguousarray(real))
    assert _eq(_np(wtq[krows]), eq) and _eq(_np(wts[krows]), es)
    dx = kg.w8a8_gemm(gq, gs, wtq, wts)
    assert _eq(_np(dx[rows]), og.gemm_ordered(_np(gq[rows]), _np(gs[rows]), _np(wtq), _np(wts),
                                                      splits=og.splits_for(M, Kd, N)))
    # dW = dY^T . X^T: 150144 output rows over the 4096 tokens
    dw = kg.w8a8_gemm(gtq, gts, xtq, xts)
    assert _eq(_np(dw[vrows]), og.gemm_ordered(_np(gtq[vrows]), _np(gts[vrows]), exq, exs,
                                                       splits=og.splits_for(N, Kd, M)))

    # the autograd function composes exactly these launches
    xg = x.clone().requires_grad_(True)
    wg = w.clone().requires_grad_(True)
    l2 = T.LinearCrossEntropyInt8.apply(xg, wg, wq, ws, t, T.IGNORE_INDEX, 128)
    l2.backward()
    assert torch.equal(l2, loss)
    assert torch.equal(xg.grad, dx) and torch.equal(wg.grad, dw)


# ------------------------------------------------------------------------------ config 4
class _Cell(nn.Module):
    """The attributes KS3Int8Cell reads from a torch KS3 (reference model/ks3.py:69-91)."""

    def __init__(self, down, up, coeffs, raw_scale, raw_shift):
        super().__init__()
        Fn, d = down.shape
        self.num_charts, self.subspace_rank = Fn, 1
        self.down = nn.Linear(d, Fn, bias=False)
        self.up = nn.Linear(Fn, d, bias=False)
        with torch.no_grad():
            self.down.weight.copy_(down)
            self.up.weight.copy_(up)
        self.coefficients = nn.Parameter(coeffs.clone())
        self.raw_scale = nn.Parameter(raw_scale.clone())
        self.raw_shift = nn.Parameter(raw_shift.clone())


def test_config4_ks3_cell_full_shape():
    """The trainable KS3 int8 cell at d = 1536, F = 5888, M = 4 x 2048 (x bf16 ~ N(0,1),
    down/up ~ N(0,0.02), coefficients ~ N(0,0.05), woken warp scalars): forward y and
    backward dx, ddown, dup bit-exact against the oracle chain, stage by stage."""
    B, Tn, d, Fn = 4, 2048, 1536, 5888
    M = B * Tn
    g = torch.Generator().manual_seed(0)
    x = torch.randn(B, Tn, d, generator=g).to(torch.bfloat16)
    down = torch.randn(Fn, d, generator=g) * 0.02
    up = torch.randn(d, Fn, generator=g) * 0.02
    coeffs = torch.randn(Fn, 6, generator=g) * 0.05
    raw_scale = 0.75 + torch.randn(Fn, generator=g) * 0.3
    raw_shift = torch.randn(Fn, generator=g) * 0.5
    grad = (torch.randn(B, Tn, d, generator=g) * 1e-2).to(torch.bfloat16)
    cell = K.KS3Int8Cell(_Cell(down, up, coeffs, raw_scale, raw_shift).to(DEV), trainable=True)
    xd = x.to(DEV).requires_grad_(True)
    y = cell(xd)
    y.backward(grad.to(DEV))
    torch.cuda.synchronize()

    p = ok.pack_masters(down.numpy(), up.numpy(), coeffs.numpy(), raw_scale.numpy(),
                        raw_shift.numpy())
    for k in ("down_codes", "down_scales", "up_codes", "up_scales", "spine_codes", "spine_scale"):
        assert _eq(_np(getattr(cell, k)).reshape(p[k].shape), p[k]), k
    sc, sh = ok.warp_scalars(p["warp_scale_codes"], p["warp_scale_scales"],
                             p["warp_shift_codes"], p["warp_shift_scales"])
    lut = ok.make_tanh_lut()
    coef, _, _ = ok.spine_params(p["spine_codes"], p["spine_scale"], p["warp_scale_codes"],
                                 p["warp_scale_scales"], p["warp_shift_codes"],
                                 p["warp_shift_scales"])

    # forward stages, replayed on the device with the cell's own kernels (deterministic)
    x2 = xd.detach().reshape(M, d)
    xq, xs = kq.quantize_last_dim(x2.float())
    hq, hs, coords16 = cell._project_codes(xq, xs)
    rows = _rows(M, 48, 5)
    x2n = _np(x2.float())
    exq, exs = oq.quantize_last_dim(x2n[rows])
    assert _eq(_np(xq[rows]), exq) and _eq(_np(xs[rows]), exs)
    coords = ok.coords_from_gemm(og.gemm_ordered(exq, exs, p["down_codes"], p["down_scales"],
                                                        splits=og.splits_for(M, Fn, d)))
    assert _eq(_np(coords16[rows]).astype(np.float32), coords)
    hfeat = ok.spine_features_int8(coords, p["spine_codes"], p["spine_scale"], sc, sh, lut)
    ehq, ehs = oq.quantize_last_dim(hfeat)
    assert _eq(_np(hq[rows]), ehq) and _eq(_np(hs[rows]), ehs)
    ey = og.gemm_ordered(ehq, ehs, p["up_codes"], p["up_scales"], splits=og.splits_for(M, d, Fn))
    assert torch.equal(y.detach().reshape(M, d)[rows].cpu(), torch.from_numpy(ey).to(torch.bfloat16))

    # backward stages
    g16 = grad.to(DEV).reshape(M, d).float().half()
    gq, gs = kq.quantize_last_dim(g16)
    upT = oq.requant_transpose(p["up_codes"], p["up_scales"])
    g16n = _np(g16).astype(np.float32)
    egq, egs = oq.quantize_last_dim(g16n[rows])
    assert _eq(_np(gq[rows]), egq)
    upTq, upTs = kq.requant_transpose(cell.up_codes, cell.up_scales)
    assert _eq(_np(upTq), upT[0]) and _eq(_np(upTs), upT[1])
    value = kg.w8a8_gemm_out(gq, gs, upTq, upTs, out_dtype=torch.float16)
    assert _eq(_np(value[rows]).astype(np.float32), ok.h(og.gemm_ordered(egq, egs, *upT,
                                                                                    splits=og.splits_for(M, Fn, d))))
    scale16, shift16 = cell._warp_scalars(torch.float16)
    v = K.ks3_vjp(value, coords16, cell.spine_codes, cell.spine_scale, scale16, shift16,
                  cell.warp_scale_raw, cell.warp_shift_raw)
    # dc: two whole 128-row groups, so both operand layouts are checked group-wise
    for grp in _rows(M // 128, 2, 6):
        r = np.arange(grp * 128, grp * 128 + 128)
        dc, _, _, _, _ = ok.vjp(_np(value[r]).astype(np.float32), _np(coords16[r]).astype(np.float32),
                                coef, sc, sh, raw_scale.numpy(), raw_shift.numpy())
        eq, es = oq.quantize_last_dim(dc)
        assert _eq(_np(v["dc_codes"][r]), eq) and _eq(_np(v["dc_scales"][r]), es)
        tq, ts = oq.quantize_last_dim(np.ascontiguousarray(dc.T))
        assert _eq(_np(v["dct_codes"][:, r]), tq) and _eq(_np(v["dct_scales"][:, grp:grp + 1]), ts)
    downT = oq.requant_transpose(p["down_codes"], p["down_scales"])
    edx = og.gemm_ordered(_np(v["dc_codes"][rows]), _np(v["dc_scales"][rows]), *downT,
                          splits=og.splits_for(M, d, Fn))
    assert torch.equal(xd.grad.reshape(M, d)[rows].cpu(), torch.from_numpy(edx).to(torch.bfloat16))
    xT = oq.requant_transpose(_np(xq), _np(xs))
    frows = _rows(Fn, 24, 7)
    eddown = og.gemm_ordered(_np(v["dct_codes"][frows]), _np(v["dct_scales"][frows]), *xT,
                             splits=og.splits_for(Fn, d, M))
    assert _eq(_np(cell.master_down.grad[frows]), ok.h(eddown))
    gT = oq.quantize_last_dim(np.ascontiguousarray(g16n.T))
    hT = oq.requant_transpose(_np(hq), _np(hs))
    drows = _rows(d, 24, 8)
    edup = og.gemm_ordered(gT[0][drows], gT[1][drows], *hT, splits=og.splits_for(d, Fn, M))
    assert _eq(_np(cell.master_up.grad[drows]), ok.h(edup))


def test_config4_project_fused_one_launch_full_shape():
    """project_fused 'int8' at config 4 (M = 8192, d = 1536, F = 5888): the one-launch
    kernel (spine in the GEMM's epilogue) equals the two-launch form everywhere (K = 1536
    is never split), and both equal the oracle chain (ordered GEMM, then the fused
    contract) on sampled rows."""
    from ksdraft_amd.kernels.ks3_triton import project_fused
    M, d, Fn = 8192, 1536, 5888
    g = torch.Generator().manual_seed(3)
    x = torch.randn(M, d, generator=g)
    down = torch.randn(Fn, d, generator=g) * 0.02
    up = torch.randn(d, Fn, generator=g) * 0.02
    coeffs = torch.randn(Fn, 6, generator=g) * 0.05
    raw_scale = 0.75 + torch.randn(Fn, generator=g) * 0.3
    raw_shift = torch.randn(Fn, generator=g) * 0.5
    cell = K.KS3Int8Cell(_Cell(down, up, coeffs, raw_scale, raw_shift).to(DEV)).eval()
    xq, xs = kq.quantize_last_dim(x.to(DEV))
    sc16, sh16 = cell._warp_scalars(torch.float16)
    args = (xq, xs, cell.down_codes, cell.down_scales, cell.spine_codes, cell.spine_scale,
            sc16, sh16, cell.tanh_lut, 128, "int8")
    hq1, hs1 = project_fused(*args, one_launch=True)
    hq2, hs2 = project_fused(*args, one_launch=False)
    assert torch.equal(hq1, hq2) and torch.equal(hs1, hs2)
    p = ok.pack_masters(down.numpy(), up.numpy(), coeffs.numpy(), raw_scale.numpy(),
                        raw_shift.numpy())
    sc, sh = ok.warp_scalars(p["warp_scale_codes"], p["warp_scale_scales"],
                             p["warp_shift_codes"], p["warp_shift_scales"])
    rows = _rows(M, 48, 9)
    acc = og.gemm_ordered(_np(xq[rows]), _np(xs[rows]), p["down_codes"], p["down_scales"])
    eq, es = ok.spine_fused_int8(acc, p["spine_codes"], p["spine_scale"], sc, sh,
                                 ok.make_tanh_lut(), 128)
    assert _eq(_np(hq1[rows]), eq) and _eq(_np(hs1[rows]), es)


def test_config4_rosa_step_full_shape():
    """The Rosa mixer step at B 4 x T 2048, d = 1536, 512 streams: the fused shift +
    quantize on sampled tokens, the hard match on sampled streams (pair brute force) and
    the exact credits on sampled flips (flip, re-match, dot), all against the oracle."""
    B, Tn, d, S = 4, 2048, 1536, 512
    g = torch.Generator().manual_seed(0)
    x = torch.randn(B, Tn, d, generator=g).to(torch.bfloat16).to(DEV)
    sigs = [torch.sigmoid(torch.randn(d, generator=g)).to(DEV) for _ in range(3)]
    out = R.shift_quantize(x, *sigs)
    xv = _np(x.float())
    toks = _rows(B * Tn, 24, 9)
    for (codes, scales), sg in zip(out, sigs):
        lerp = orr.shifted(xv, _np(sg), "bfloat16").reshape(B * Tn, d)[toks]
        ec, es = oq.quantize_last_dim(lerp)
        assert _eq(_np(codes[toks]), ec) and _eq(_np(scales[toks]), es)

    rng = np.random.default_rng(10)
    q, k, vv = (rng.standard_normal((B, Tn, S)).astype(np.float32) for _ in range(3))
    k[:, :, :8] = q[:, :, :8]  # streams with long matches past the 62 cap
    payload = (np.abs(rng.standard_normal(S)) + 0.5).astype(np.float32)
    go = rng.standard_normal((B, Tn, S)).astype(np.float32)
    tq, tk, tv = (torch.from_numpy(a).to(DEV).requires_grad_(True) for a in (q, k, vv))
    tp = torch.from_numpy(payload).to(DEV).requires_grad_(True)
    yh = HardRosaGPU.apply(tq, tk, tv, tp)
    yh.backward(torch.from_numpy(go).to(DEV))
    yh = _np(yh)
    streams = [(0, 0), (0, 3), (1, 200), (2, 511), (3, 7), (3, 300)]
    for b, s in streams:
        bits = [orr.bits_of(a[b, :, s])[None] for a in (q, k, vv)]
        sign, _, _ = orr.match(*bits)
        assert np.array_equal(yh[b, :, s], payload[s] * sign[0]), (b, s)
    gq_, gk_, gv_ = (_np(t.grad) for t in (tq, tk, tv))
    for b, s in streams[:3]:
        bits = [orr.bits_of(a[b, :, s])[None] for a in (q, k, vv)]
        base, _, _ = orr.match(*bits)
        gsign = (go[b, :, s] * payload[s]).astype(np.float64)
        for which, pre, grad in ((0, q, gq_), (1, k, gk_), (2, vv, gv_)):
            sig = orr.sigmoid32(pre[b, :, s])
            bern = (sig * (np.float32(1) - sig)).astype(np.float32)
            for pos in rng.choice(Tn, 6, replace=False):
                fl = [bb.copy() for bb in bits]
                fl[which][0, pos] ^= 1
                sp, _, _ = orr.match(*fl)
                cred = float(((sp[0] - base[0]) * gsign).sum())
                exp = np.float32(cred * (1.0 - 2.0 * bits[which][0, pos])) * bern[pos]
                assert abs(grad[b, pos, s] - exp) <= 1e-5 * max(1.0, abs(exp)), (which, b, s, pos)


# ------------------------------------------------------------------------------ config 5
def test_config5_draft_step_full_shape(monkeypatch):
    """One INT8 draft training step at config-5 dimensions (one layer: d 1536, 512 Rosa
    streams, 5888 KS3 charts, vocabulary 150144, B 4 x T 2048, teacher state bf16, every
    linear INT8, loss scale 2^12 so that every gradient group is live), checked on sampled
    rows against the oracle chains from the recorded surface inputs and the fp32 masters:
    the Rosa output projection (y with its fused residual, dX, dW), the KS3 cell (y, dx, and
    ddown / dup on sampled output rows from the device's replayed operands), the head's loss
    against float64 torch on logits whose sampled rows are bit-exact, and, after the
    optimizer step, the int8 codes of every registered surface against the oracle
    quantizer of its updated master."""
    from ksdraft_amd.config import baseline_config
    from ksdraft_amd.model import KSDraftModel, to_int8
    from ksdraft_amd.train.int8_step import Int8DraftTrainer
    from tests.test_gpu_draft import _Recorder

    cfg = baseline_config()
    cfg.layers = 1
    d, Fn, S, V = cfg.d_model, cfg.charts, cfg.rosa_streams, cfg.vocab_size
    B, Tn = 4, 2048
    M = B * Tn
    torch.manual_seed(0)
    fm = KSDraftModel(cfg, teacher_dim=d, device=DEV)
    with torch.no_grad():
        for name, p in fm.named_parameters():
            if name.endswith(("up.weight", "out_proj.weight", "teacher_proj.weight")):
                p.normal_(0, 0.02)
    model = to_int8(fm, trainable=True, int8_injection=True)
    del fm
    rec = _Recorder(model, monkeypatch)
    tr = Int8DraftTrainer(model, lr=3e-4, weight_decay=0.01, grad_clip=1.0, loss_scale=2.0 ** 12)
    g = torch.Generator(device=DEV).manual_seed(0)
    tokens = torch.randint(0, V, (B, Tn + 1), device=DEV, generator=g)
    teacher = torch.randn(B, Tn, d, device=DEV, generator=g).to(torch.bfloat16)
    masters = {n: p.detach().clone() for n, p in model.named_parameters()}
    model.train()
    loss, ce, ts = tr.loss(tokens, teacher)
    tr.backward(loss)
    torch.cuda.synchronize()
    assert torch.isfinite(loss)
    rows = _rows(M, 12, 20)
    mnp = lambda k: _np(masters[k]).astype(np.float32)  # noqa: E731

    # Rosa output projection: y = W8A8(x) + b + residual, dX, dW (K = 8192 tokens)
    r = rec.lin["blocks.0.rosa.out_proj"]
    mod = r["mod"]
    x = _np(r["x"]).reshape(M, S).astype(np.float32)
    gy = _np(r["g"]).reshape(M, d).astype(np.float32)
    wq, ws = oq.quantize_last_dim(mnp("blocks.0.rosa.out_proj.weight"))
    bias = mnp("blocks.0.rosa.out_proj.bias")
    xq, xs = oq.quantize_last_dim(x)
    ey = og.gemm_ordered(xq, xs, wq, ws, bias=bias, rows=rows, splits=og.splits_for(M, d, S))
    ey = (ey + _np(r["res"]).reshape(M, d)[rows]).astype(np.float32)
    assert _eq(_np(r["y"]).reshape(M, d)[rows], ey)
    gq, gs = oq.quantize_last_dim(gy[rows])
    edx = og.gemm_ordered(gq, gs, *oq.requant_transpose(wq, ws), splits=og.splits_for(M, S, d))
    assert _eq(_np(r["dx"]).reshape(M, S)[rows], edx)
    nrows = _rows(d, 8, 21)
    gtq, gts = oq.quantize_last_dim(np.ascontiguousarray(gy[:, nrows].T))
    edw = og.gemm_ordered(gtq, gts, *oq.requant_transpose(xq, xs), splits=og.splits_for(d, S, M))
    assert _eq(_np(mod.weight.grad)[nrows], edw)

    # KS3 cell, row-local chain: y and dx on sampled tokens
    r = rec.cell["blocks.0.ffn"]
    cell = r["mod"]
    mk = lambda k: mnp(f"blocks.0.ffn.master_{k}")  # noqa: E731
    p = ok.pack_masters(mk("down"), mk("up"), mk("coefficients"), mk("raw_scale"), mk("raw_shift"))
    sc, sh = ok.warp_scalars(p["warp_scale_codes"], p["warp_scale_scales"],
                             p["warp_shift_codes"], p["warp_shift_scales"])
    coef, _, _ = ok.spine_params(p["spine_codes"], p["spine_scale"], p["warp_scale_codes"],
                                 p["warp_scale_scales"], p["warp_shift_codes"], p["warp_shift_scales"])
    xc = _np(r["x"]).reshape(M, d).astype(np.float32)
    gc = _np(r["g"]).reshape(M, d).astype(np.float32)
    xq, xs = oq.quantize_last_dim(xc[rows])
    coords = ok.coords_from_gemm(og.gemm_ordered(xq, xs, p["down_codes"], p["down_scales"],
                                                 splits=og.splits_for(M, Fn, d)))
    hfeat = ok.spine_features_int8(coords, p["spine_codes"], p["spine_scale"], sc, sh, ok.make_tanh_lut())
    hq, hs = oq.quantize_last_dim(hfeat)
    ey = og.gemm_ordered(hq, hs, p["up_codes"], p["up_scales"], splits=og.splits_for(M, d, Fn))
    ey = (ey + _np(r["res"]).reshape(M, d)[rows]).astype(np.float32)
    assert _eq(_np(r["y"]).reshape(M, d)[rows], ey)
    g16 = ok.h(gc[rows])
    gq, gs = oq.quantize_last_dim(g16)
    value = ok.h(og.gemm_ordered(gq, gs, *oq.requant_transpose(p["up_codes"], p["up_scales"]),
                                 splits=og.splits_for(M, Fn, d)))
    dc, _, _, _, _ = ok.vjp(value, coords, coef, sc, sh, mk("raw_scale"), mk("raw_shift"))
    dcq, dcs = oq.quantize_last_dim(dc)
    edx = og.gemm_ordered(dcq, dcs, *oq.requant_transpose(p["down_codes"], p["down_scales"]),
                          splits=og.splits_for(M, d, Fn))
    assert _eq(_np(r["dx"]).reshape(M, d)[rows], edx)
    # ddown and dup reduce over the 8192 tokens: sampled output rows from the device's own
    # (replayed, deterministic) operands, each of which the row checks above pin
    xdev = r["x"].reshape(M, d).float()
    xq_d, xs_d = kq.quantize_last_dim(xdev)
    hq_d, hs_d, coords16 = cell._project_codes(xq_d, xs_d)
    gq_d, gs_d, gtq_d, gts_d = kq.quantize_dual(r["g"].reshape(M, d), round_fp16=True)
    assert _eq(_np(gq_d[rows]), gq)
    upTq, upTs = kq.requant_transpose(cell.up_codes, cell.up_scales)
    value_d = kg.w8a8_gemm_out(gq_d, gs_d, upTq, upTs, out_dtype=torch.float16)
    scale16, shift16 = cell._warp_scalars(torch.float16)
    v = K.ks3_vjp(value_d, coords16, cell.spine_codes, cell.spine_scale, scale16, shift16,
                  cell.warp_scale_raw, cell.warp_shift_raw)
    frows = _rows(Fn, 6, 22)
    eddown = og.gemm_ordered(_np(v["dct_codes"][frows]), _np(v["dct_scales"][frows]),
                             *oq.requant_transpose(_np(xq_d), _np(xs_d)), splits=og.splits_for(Fn, d, M))
    assert _eq(_np(cell.master_down.grad[frows]), ok.h(eddown))
    drows = _rows(d, 6, 23)
    edup = og.gemm_ordered(_np(gtq_d[drows]), _np(gts_d[drows]),
                           *oq.requant_transpose(_np(hq_d), _np(hs_d)), splits=og.splits_for(d, Fn, M))
    assert _eq(_np(cell.master_up.grad[drows]), ok.h(edup))
    del v, value_d, hq_d, coords16

    # the head: sampled logits rows bit-exact, the loss against float64 torch on the logits
    head = model.head
    with torch.no_grad():
        hn, _ = model.backbone(tokens[:, :-1], teacher)
        hn = hn.reshape(M, d).float()
        hxq, hxs = kq.quantize_last_dim(hn)
        logits = kg.w8a8_gemm(hxq, hxs, head.weight_codes, head.weight_scales)
    vrows = _rows(V, 64, 26)
    ewq, ews = oq.quantize_last_dim(mnp("embedding.weight")[vrows])
    assert _eq(_np(head.weight_codes[vrows]), ewq) and _eq(_np(head.weight_scales[vrows]), ews)
    lrows = rows[:4]
    el = og.gemm_ordered(_np(hxq), _np(hxs), _np(head.weight_codes), _np(head.weight_scales),
                         rows=lrows, splits=og.splits_for(M, V, d))
    assert _eq(_np(logits[lrows]), el)
    eref = torch.nn.functional.cross_entropy(logits.double(), tokens[:, 1:].reshape(-1))
    assert abs(ce.item() - eref.item()) <= 2e-5 * abs(eref.item())
    del logits

    # the optimizer step: every registered surface's codes from its updated master
    tr.optimizer_step()
    torch.cuda.synchronize()
    for name, mod in model.named_modules():
        if isinstance(mod, Int8Linear):
            n = mod.weight.shape[0]
            sel = _rows(n, min(n, 16), 24)
            eq, es = oq.quantize_last_dim(_np(mod.weight[sel]).astype(np.float32))
            assert _eq(_np(mod.weight_codes[sel]), eq) and _eq(_np(mod.weight_scales[sel]), es), name
    for nm in ("down", "up"):
        w = getattr(cell, "master_" + nm)
        sel = _rows(w.shape[0], 16, 25)
        eq, es = oq.quantize_last_dim(_np(w[sel]).astype(np.float32))
        assert _eq(_np(getattr(cell, nm + "_codes")[sel]), eq), nm
        assert _eq(_np(getattr(cell, nm + "_scales")[sel]), es), nm
