"""GPU parity of the INT8 draft training step (at a small shape).

A 2-layer draft (d 256, 64 Rosa streams, 384 KS3 charts, vocabulary 512, B 2 x T 48, a
bf16 teacher state on the teacher_proj seam) is converted with to_int8(trainable=True)
and trained through Int8DraftTrainer. Every INT8 surface of the step is checked stage by
stage: hooks capture each surface's device inputs and upstream gradients, and the oracle
chains (tests/chains.py) recompute its outputs and gradients from those inputs and the
fp32 masters.

Bars: Int8Linear (Rosa q/k/v/out, teacher_proj) y, dX, dW bit-exact (q/k/v through the
fused shift + dual quantization, whose input gradient is within fp32 summation order of
the oracle's float64 shift backward); KS3Int8Cell y, dx,
ddown, dup bit-exact, dcoeff/dscale/dshift within the VJP-reduction tolerance; the Rosa
hard output bit-exact and its credits within 1e-5; the head's loss within 2e-5 of float64
torch; after the optimizer step, every registered layer's int8 codes bit-exact against the
oracle quantizer of its updated master.
"""

import numpy as np
import pytest
import torch

import ksdraft_amd.kernels.rosa as krosa
import ksdraft_amd.kernels.rosa_credit_gpu as rcg
from ksdraft_amd.config import KSDraftConfig
from ksdraft_amd.kernels.ks3_int8 import KS3Int8Cell
from ksdraft_amd.kernels.linear import Int8Linear
from ksdraft_amd.model import KSDraftModel, to_int8
from ksdraft_amd.train.int8_step import Int8DraftTrainer, clip_coefficient
from oracle import gemm as og
from oracle import quant as oq
from oracle import rosa as orr
from tests import chains

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _np(t):
    return t.detach().float().cpu().numpy()


def _bits(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    assert a.shape == b.shape, (a.shape, b.shape)
    return np.array_equal(a.view(np.uint32), b.view(np.uint32))


def _model(int8_injection=False):
    torch.manual_seed(0)
    cfg = KSDraftConfig(vocab_size=512, layers=2, d_model=256, rosa_streams=64, ks3_charts=384)
    m = KSDraftModel(cfg, teacher_dim=256).to(DEV)
    with torch.no_grad():
        # zero-init surfaces woken as the reference's conversion tests do
        # (tests/test_int8_convert.py:17-25): otherwise the parity checks see zeros
        for name, p in m.named_parameters():
            if name.endswith(("up.weight", "out_proj.weight", "teacher_proj.weight",
                              "embedding.weight")):
                p.normal_(0, 0.02)
    return to_int8(m, trainable=True, int8_injection=int8_injection)


class _Recorder:
    def __init__(self, model, monkeypatch):
        self.lin, self.cell, self.rosa = {}, {}, []
        for name, mod in model.named_modules():
            if isinstance(mod, Int8Linear) and mod is not model.head:
                self._hook(name, mod, self.lin)
            elif isinstance(mod, KS3Int8Cell):
                self._hook(name, mod, self.cell)
        orig = rcg.HardRosaGPU
        rec = self.rosa

        class Recording:
            @staticmethod
            def apply(q, k, v, payload):
                out = orig.apply(q, k, v, payload)
                r = {n: t.detach().clone() for n, t in (("q", q), ("k", k), ("v", v),
                                                         ("p", payload), ("out", out))}
                for n, t in (("q", q), ("k", k), ("v", v), ("out", out)):
                    if t.requires_grad:
                        t.register_hook(lambda g, n=n: r.__setitem__("g" + n, g.detach().clone()))
                rec.append(r)
                return out
        monkeypatch.setattr(rcg, "HardRosaGPU", Recording)

        # the Rosa q/k/v projections in training: shift + dual quantization + 3 GEMMs
        orig_shift = krosa.ShiftedInt8Projections
        shift = self.shift = []

        class RecordingShift:
            @staticmethod
            def apply(x, sq, sk, sv, *args):
                outs = orig_shift.apply(x, sq, sk, sv, *args)
                r = {"x": x.detach().clone(), "sig": [t.detach().clone() for t in (sq, sk, sv)],
                     "out": [o.detach().clone() for o in outs]}
                for i, o in enumerate(outs):
                    o.register_hook(lambda g, i=i: r.__setitem__(f"g{i}", g.detach().clone()))
                x.register_hook(lambda g: r.__setitem__("dx", g.detach().clone()))
                shift.append(r)
                return outs
        monkeypatch.setattr(krosa, "ShiftedInt8Projections", RecordingShift)

    @staticmethod
    def _hook(name, mod, store):
        r = store.setdefault(name, {"mod": mod})

        def fwd(m, inp, kwargs, out):
            r["x"] = inp[0].detach().clone()
            r["y"] = out.detach().clone()
            res = kwargs.get("residual")
            r["res"] = None if res is None else res.detach().clone()

        def bwd(m, gin, gout):
            r["g"] = gout[0].detach().clone()
            r["dx"] = None if gin[0] is None else gin[0].detach().clone()
        mod.register_forward_hook(fwd, with_kwargs=True)
        mod.register_full_backward_hook(bwd)


@pytest.mark.parametrize("int8_injection", [False, True])
def test_int8_draft_step_stagewise_bit_exact(monkeypatch, int8_injection):
    model = _model(int8_injection)
    rec = _Recorder(model, monkeypatch)
    trainer = Int8DraftTrainer(model, lr=1e-3)
    g = torch.Generator().manual_seed(1)
    tokens = torch.randint(0, 512, (2, 49), generator=g).to(DEV)
    teacher = torch.randn(2, 48, 256, generator=g).to(torch.bfloat16).to(DEV)
    masters = {n: p.detach().clone() for n, p in model.named_parameters()}

    loss, ce, ts = trainer.loss(tokens, teacher)
    trainer.opt.zero_grad(set_to_none=True)
    loss.backward()
    torch.cuda.synchronize()
    assert torch.isfinite(loss)

    # Int8Linear surfaces: Rosa q/k/v/out of both blocks and the teacher seam (and the
    # DSpine injection's eight low-rank maps per block)
    assert len(rec.lin) == 2 * 4 + 1 + (2 * 8 if int8_injection else 0)
    for name, r in rec.lin.items():
        mod = r["mod"]
        if "x" not in r:  # the fused shift + q/k/v path runs instead of the module's forward
            assert name.endswith(("rosa.q_proj", "rosa.k_proj", "rosa.v_proj")), name
            continue
        x = _np(r["x"]).reshape(-1, mod.in_features)
        gy = _np(r["g"]).reshape(-1, mod.out_features)
        w = _np(masters[name + ".weight"])
        b = None if mod.bias is None else _np(masters[name + ".bias"])
        exp = chains.linear_chain(x, w, b, gy)
        ey = exp["y"]
        if r["res"] is not None:  # the block's residual add, fused in the store
            ey = (_np(r["res"]).reshape(ey.shape) + ey).astype(np.float32)
        assert _bits(_np(r["y"]).reshape(ey.shape), ey), name
        if r["dx"] is not None:
            assert _bits(_np(r["dx"]).reshape(exp["dx"].shape), exp["dx"]), name
        assert _bits(_np(mod.weight.grad), exp["dw"]), name

    assert sum(r.get("res") is not None for r in rec.lin.values()) == 2  # both out_proj

    # Rosa q/k/v: the fused shift + projections against the oracle shift and linear chain
    assert len(rec.shift) == 2
    for blk, r in enumerate(rec.shift):
        x = _np(r["x"])
        d = x.shape[-1]
        dxs = []
        for m, proj in enumerate(("q_proj", "k_proj", "v_proj")):
            name = f"blocks.{blk}.rosa.{proj}"
            lerp = orr.shifted(x, _np(r["sig"][m]), "float32").reshape(-1, d)
            gy = _np(r[f"g{m}"]).reshape(lerp.shape[0], -1)
            exp = chains.linear_chain(lerp, _np(masters[name + ".weight"]),
                                      _np(masters[name + ".bias"]), gy)
            assert _bits(_np(r["out"][m]).reshape(exp["y"].shape), exp["y"]), name
            assert _bits(_np(model.get_submodule(name).weight.grad), exp["dw"]), name
            dxs.append(exp["dx"].reshape(x.shape))
        edx, _ = orr.shifted_backward(x, np.stack([_np(t) for t in r["sig"]]), dxs)
        np.testing.assert_allclose(_np(r["dx"]), edx, rtol=1e-5, atol=1e-6 * np.abs(edx).max())
    # KS3 cells
    assert len(rec.cell) == 2
    assert all(r["res"] is not None for r in rec.cell.values())
    for name, r in rec.cell.items():
        mod = r["mod"]
        mk = lambda k: _np(masters[f"{name}.master_{k}"])  # noqa: E731
        x = _np(r["x"]).reshape(-1, mod.in_features)
        exp = chains.ks3_cell_chain(mk("down"), mk("up"), mk("coefficients"), mk("raw_scale"),
                                    mk("raw_shift"), x, _np(r["g"]).reshape(x.shape[0], -1))
        ey = exp["y"]
        if r["res"] is not None:
            ey = (_np(r["res"]).reshape(ey.shape) + ey).astype(np.float32)
        assert _bits(_np(r["y"]).reshape(ey.shape), ey), name
        assert _bits(_np(r["dx"]).reshape(exp["dx"].shape), exp["dx"]), name
        assert _bits(_np(mod.master_down.grad), chains.handoff(exp["ddown"])), name
        assert _bits(_np(mod.master_up.grad), chains.handoff(exp["dup"])), name
        ref = exp["dcoeff"].reshape(-1)
        np.testing.assert_allclose(_np(mod.master_coefficients.grad).reshape(-1), ref,
                                   rtol=4e-3, atol=2e-3 * np.abs(ref).max() + 1e-12)

    # Rosa hard match and credits
    assert len(rec.rosa) == 2
    for r in rec.rosa:
        q, k, v, p = (_np(r[n]) for n in ("q", "k", "v", "p"))
        ey, _ = orr.hard_rosa_forward(q, k, v, p)
        assert _bits(_np(r["out"]), ey)
        for got, exp in zip((r["gq"], r["gk"], r["gv"]),
                            orr.hard_rosa_backward(q, k, v, p, _np(r["gout"]))[:3]):
            got = _np(got)
            np.testing.assert_allclose(got, exp, rtol=1e-5, atol=1e-5 * (np.abs(exp).max() + 1e-30))

    # the head: fp32 loss against float64 torch on the device's normed stream
    with torch.no_grad():
        hn, _ = model.backbone(tokens[:, :-1], teacher)
        wq, ws = oq.quantize_last_dim(_np(masters["embedding.weight"]))
        xq, xs = oq.quantize_last_dim(_np(hn).reshape(-1, 256))
        logits = torch.from_numpy(og.gemm_ordered(xq, xs, wq, ws)).double()
        eref = torch.nn.functional.cross_entropy(logits, tokens[:, 1:].reshape(-1).cpu())
    assert abs(ce.item() - eref.item()) <= 2e-5 * abs(eref.item())

    # the optimizer writes every registered layer's codes from its updated master
    coef = clip_coefficient(model.parameters(), 1.0)
    trainer.opt.step(clip_coef=coef)
    torch.cuda.synchronize()
    for mod in [r["mod"] for r in rec.lin.values()] + [model.head]:
        eq, es = oq.quantize_last_dim(_np(mod.weight))
        assert np.array_equal(mod.weight_codes.cpu().numpy(), eq)
        assert np.array_equal(mod.weight_scales.cpu().numpy().view(np.uint16), es.view(np.uint16))
    for r in rec.cell.values():  # the KS3 cells' down/up codes come from the optimizer too
        cell = r["mod"]
        for name in ("down", "up"):
            assert cell._master_codes_current(name)
            eq, es = oq.quantize_last_dim(_np(getattr(cell, "master_" + name)))
            assert np.array_equal(getattr(cell, name + "_codes").cpu().numpy(), eq)
            assert np.array_equal(getattr(cell, name + "_scales").cpu().numpy().view(np.uint16),
                                  es.view(np.uint16))
    # and a full second step runs on the optimizer's codes
    l2, _, _ = trainer.step(tokens, teacher)
    assert torch.isfinite(l2)


def test_clip_coefficient_matches_torch():
    torch.manual_seed(3)
    ps = [torch.nn.Parameter(torch.randn(n, device=DEV)) for n in (10, 300, 7)]
    for p in ps:
        p.grad = torch.randn_like(p) * 3
    coef = clip_coefficient(ps, 1.0)
    grads = [p.grad.clone() for p in ps]
    torch.nn.utils.clip_grad_norm_(ps, 1.0)
    for g0, p in zip(grads, ps):
        torch.testing.assert_close(g0 * coef, p.grad, rtol=1e-6, atol=1e-7)


def test_training_step_gradients_are_deterministic():
    """Two backward passes of the INT8 draft step from the same state give bit-identical
    gradients for every parameter (the Rosa credits are exact fixed-point sums, every other
    reduction has a fixed order)."""
    model = _model(int8_injection=True)
    trainer = Int8DraftTrainer(model, lr=1e-3, loss_scale=2.0 ** 12)
    g = torch.Generator().manual_seed(5)
    tokens = torch.randint(0, 512, (2, 97), generator=g).to(DEV)
    teacher = torch.randn(2, 96, 256, generator=g).to(torch.bfloat16).to(DEV)
    runs = []
    for _ in range(3):
        model.train()
        loss, _, _ = trainer.loss(tokens, teacher)
        trainer.backward(loss)
        torch.cuda.synchronize()
        runs.append({n: p.grad.detach().clone() for n, p in model.named_parameters()
                     if p.grad is not None})
    assert len(runs[0]) > 50
    for r in runs[1:]:
        assert r.keys() == runs[0].keys()
        for n, t in r.items():
            assert torch.equal(t, runs[0][n]), n
    assert any(float(t.abs().max()) > 0 for n, t in runs[0].items() if "rosa.q_proj" in n)


def test_clip_coefficient_with_loss_scale():
    """Gradients of a power-of-two scaled loss: the factor returned for them applies the
    clip and the unscaling at once, bit for bit the unscaled gradients' clip."""
    torch.manual_seed(4)
    S = 2.0 ** 12
    for spread in (3.0, 1e-3):  # clipping active, and inactive
        ps = [torch.nn.Parameter(torch.randn(n, device=DEV)) for n in (10, 300, 7)]
        grads = [torch.randn_like(p) * spread for p in ps]
        for p, g in zip(ps, grads):
            p.grad = g.clone()
        coef = clip_coefficient(ps, 1.0)
        for p, g in zip(ps, grads):
            p.grad = g * S
        coef_s = clip_coefficient(ps, 1.0, loss_scale=S)
        for p, g in zip(ps, grads):
            assert torch.equal(p.grad * coef_s, g * coef)


def test_int8_draft_step_with_int8_embedding():
    """to_int8(int8_embedding=True): the lookup reads the tied head's codes; the looked-up
    rows equal the oracle dequantization of Q(master)[ids], and training steps run."""
    torch.manual_seed(0)
    cfg = KSDraftConfig(vocab_size=512, layers=1, d_model=256, rosa_streams=64, ks3_charts=384)
    m = KSDraftModel(cfg).to(DEV)
    with torch.no_grad():
        m.embedding.weight.normal_(0, 0.02)
    model = to_int8(m, trainable=True, int8_embedding=True)
    assert model.embedding.weight is model.head.weight and model.embedding.codes_from is model.head
    seen = {}
    model.embedding.register_forward_hook(lambda mod, i, o: seen.__setitem__("y", o.detach().clone()))
    trainer = Int8DraftTrainer(model, lr=1e-3)
    tokens = torch.randint(0, 512, (2, 33), generator=torch.Generator().manual_seed(2)).to(DEV)
    for step in range(2):
        master = _np(model.embedding.weight)
        loss, _, _ = trainer.step(tokens)
        assert torch.isfinite(loss)
        ec, es = oq.quantize_last_dim(master)
        ids = tokens[:, :-1].reshape(-1).cpu().numpy()
        exp = oq.dequantize_last_dim(ec[ids], es[ids])
        assert _bits(_np(seen["y"]).reshape(exp.shape), exp), step
    assert model.head._codes_current()  # the optimizer's codes feed the next lookup
