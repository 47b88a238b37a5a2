"""GPU checks of the fused float surfaces of the draft step (kernels/draft.py) against the
torch composition that restates the reference.

  TransferSpaceLoss   reference ksdraft/train/__init__.py:79-85, in float64 on the CPU
  FusedInjection      reference ksdraft/model/spine.py:38-68 (AdjacentInjection with
                      ``fused = False``: torch ops on the same weights, fp32, GPU)

Bars (fp32, different summation orders): the transfer loss within 1e-6 relative and its
gradients within 1e-5; the injection's outputs and every gradient within 1e-4 relative to
the largest entry.
"""

import copy

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from ksdraft_amd.model.spine import AdjacentInjection
from ksdraft_amd.train.int8_step import transfer_space_loss

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _ref_transfer(features, emb, tgt):
    """train/__init__.py:79-85 in float64."""
    tgt_emb = F.normalize(emb[tgt].double(), dim=-1)
    ts = 0.0
    for f in features:
        fn = F.normalize(f.double(), dim=-1)
        ts = ts + (1 - (fn * tgt_emb).sum(-1)).mean()
    return ts / max(1, len(features))


@pytest.mark.parametrize("d", [256, 258])
def test_transfer_space_loss_matches_reference(d):
    g = torch.Generator().manual_seed(d)
    B, T, V, L = 2, 37, 100, 3
    emb = torch.randn(V, d, generator=g)
    tgt = torch.randint(0, V, (B, T), generator=g)
    feats = [torch.randn(B, T, d, generator=g) * (i + 1) for i in range(L)]
    feats[1][0, 3] = 0.0  # a zero feature row: F.normalize divides by eps there
    fg = [f.to(DEV).requires_grad_(True) for f in feats]
    eg = emb.to(DEV).requires_grad_(True)
    ts = transfer_space_loss(fg, eg, tgt.to(DEV))
    ts.backward()
    fr = [f.double().requires_grad_(True) for f in feats]
    er = emb.double().requires_grad_(True)
    tr = _ref_transfer(fr, er, tgt)
    tr.backward()
    assert abs(ts.item() - tr.item()) <= 1e-6 * abs(tr.item())
    for a, b in zip(fg, fr):
        a, b = a.grad.double().cpu(), b.grad
        torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-5 * b.abs().max().item())
    torch.testing.assert_close(eg.grad.double().cpu(), er.grad, rtol=1e-5,
                               atol=1e-5 * er.grad.abs().max().item())


def _injection(d, seed):
    torch.manual_seed(seed)
    m = AdjacentInjection(d)
    with torch.no_grad():
        for p in m.parameters():
            p.normal_(0, 0.05)
    return m.to(DEV)


@pytest.mark.parametrize("with_prev", [False, True])
@pytest.mark.parametrize("B,T,d", [(2, 40, 256), (3, 17, 200)])
def test_fused_injection_matches_composition(with_prev, B, T, d):
    m1 = _injection(d, B * T + d)
    m2 = copy.deepcopy(m1)
    m2.fused = False
    g = torch.Generator().manual_seed(7)
    z0 = torch.randn(B, T, d, generator=g)
    prev0 = torch.randn(B, T, d, generator=g) if with_prev else None
    gout = torch.randn(B, T, d, generator=g)
    gp = torch.randn(B, T, d, generator=g)
    res = []
    for m in (m1, m2):
        z = z0.to(DEV).requires_grad_(True)
        prev = prev0.to(DEV).requires_grad_(True) if with_prev else None
        assert m._use_fused(z) == m.fused
        out, p = m(z, prev)
        torch.autograd.backward([out, p], [gout.to(DEV), gp.to(DEV)])
        grads = {n: q.grad.clone() for n, q in m.named_parameters()}
        res.append((out.detach(), p.detach(), z.grad, None if prev is None else prev.grad, grads))

    def close(a, b, name):
        torch.testing.assert_close(a, b, rtol=1e-4, atol=1e-4 * b.abs().max().item() + 1e-12,
                                   msg=name)
    (o1, p1, z1, v1, g1), (o2, p2, z2, v2, g2) = res
    close(o1, o2, "out")
    close(p1, p2, "p")
    close(z1, z2, "dz")
    if with_prev:
        close(v1, v2, "dprev")
    for n in g2:
        close(g1[n], g2[n], n)


@pytest.mark.parametrize("d,M", [(1536, 300), (256, 17), (512, 64)])
@pytest.mark.parametrize("with_res", [True, False])
def test_residual_layer_norm_matches_torch(d, M, with_res):
    """ResidualLayerNorm: the forward is torch's; dx = LN_backward(dy) + dres, dweight and
    dbias against torch's LayerNorm + residual add (fp32, rtol 1e-5)."""
    from ksdraft_amd.kernels.draft import ResidualLayerNorm
    g = torch.Generator().manual_seed(d + M)
    x0 = torch.randn(2, M, d, generator=g) * 2 + 0.5
    w0 = torch.randn(d, generator=g) * 0.3 + 1
    b0 = torch.randn(d, generator=g) * 0.1
    gy = torch.randn(2, M, d, generator=g)
    gr = torch.randn(2, M, d, generator=g)
    outs = []
    for fused in (True, False):
        x = x0.to(DEV).requires_grad_(True)
        w = w0.to(DEV).requires_grad_(True)
        b = b0.to(DEV).requires_grad_(True)
        if fused:
            y, res = ResidualLayerNorm.apply(x, w, b, 1e-5)
        else:
            y, res = F.layer_norm(x, (d,), w, b, 1e-5), x
        grads = [gy.to(DEV)] + ([gr.to(DEV)] if with_res else [])
        torch.autograd.backward([y, res] if with_res else [y], grads)
        outs.append((y.detach(), x.grad, w.grad, b.grad))
    (y1, dx1, dw1, db1), (y2, dx2, dw2, db2) = outs
    assert torch.equal(y1, y2)
    for a, b_, n in ((dx1, dx2, "dx"), (dw1, dw2, "dw"), (db1, db2, "db")):
        torch.testing.assert_close(a, b_, rtol=1e-5, atol=1e-5 * b_.abs().max().item(), msg=n)
