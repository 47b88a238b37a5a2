"""The float-tier model around the INT8 tier (CPU only): shapes, parameter counts against
the reference's formulas (config.py:71-91), the tie of head and embedding after a device
move (draft.py:49-51), identity-block init (block.py docstring), and the Horner spine
against the explicit Hermite / Chebyshev basis (reference tests/test_ks3.py:15-37)."""

import pytest
import torch

from ksdraft_amd.config import KSDraftConfig, baseline_config
from ksdraft_amd.model import KSDraftModel, spine_horner
from ksdraft_amd.model.spine import AdjacentInjection


def test_baseline_config_counts():
    cfg = baseline_config()
    assert cfg.charts == 5888 and cfg.d_model == 1536 and cfg.rosa_streams == 512
    # the counts the reference's formulas give for this config (ksdraft/config.py:71-95)
    assert cfg.ks3_params() == 18_135_040
    assert cfg.rosa_params() == 3_153_920
    assert cfg.total_params() == 741_556_224
    with pytest.raises(ValueError):
        KSDraftConfig(dtype="fp8")


def test_model_tie_and_identity_init():
    cfg = KSDraftConfig(vocab_size=97, layers=2, d_model=128, rosa_streams=16, ks3_charts=64)
    m = KSDraftModel(cfg, teacher_dim=32)
    assert m.head.weight is m.embedding.weight
    core = cfg.layers * cfg.layer_params() + cfg.embedding_params()
    assert m.param_counts()["core"] == core
    # every additive update starts at zero: the blocks' residual branches vanish
    x = torch.randn(2, 5, 128)
    for blk in m.blocks:
        h, p = blk.injection(x)
        assert torch.equal(h, x)
        assert torch.equal(blk.ffn(x), torch.zeros_like(x))


def test_spine_horner_matches_basis():
    g = torch.Generator().manual_seed(0)
    t = torch.randn(50, 7, 1, generator=g)
    z = torch.randn(50, 7, 1, generator=g)
    c = torch.randn(7, 6, generator=g)
    s, w = spine_horner(t, z, c)
    p0, p1, p2, p3, p4, p5 = c.unbind(-1)
    t2, t3 = t * t, t * t * t
    sb = (p0 * (2 * t3 - 3 * t2 + 1) + p1 * (-2 * t3 + 3 * t2) + p2 * (t3 - 2 * t2 + t)
          + p3 * (t3 - t2))
    wb = p4 * (2 * z * z - 1) + p5 * (4 * z * z * z - 3 * z)
    torch.testing.assert_close(s, sb, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(w, wb, rtol=1e-5, atol=1e-5)


def test_injection_seeds_position_zero_from_previous_layer():
    torch.manual_seed(1)
    inj = AdjacentInjection(32, rank=4, feature_rank=8)
    for lr in (inj.gate_q, inj.gate_p, inj.inject):
        torch.nn.init.normal_(lr.up.weight, std=0.1)
    z = torch.randn(2, 6, 32)
    prev = torch.randn(2, 6, 32)
    out0, p = inj(z)
    out1, _ = inj(z, prev)
    assert torch.equal(out0[:, 1:], out1[:, 1:])      # only position 0 takes the seed
    assert not torch.equal(out0[:, 0], out1[:, 0])
    torch.testing.assert_close(p, inj.feature_up(inj.feature_down(z)))


def test_injection_stacked_gemms_equal_the_reference_composition():
    """AdjacentInjection's stacked low-rank GEMMs compute spine.py:62-68's sums."""
    import torch.nn.functional as F
    torch.manual_seed(4)
    inj = AdjacentInjection(48, rank=6, feature_rank=10)
    for lr in (inj.gate_q, inj.gate_p, inj.inject):
        torch.nn.init.normal_(lr.up.weight, std=0.2)
    torch.nn.init.normal_(inj.gate_bias, std=0.1)
    z = torch.randn(3, 9, 48, dtype=torch.float64)
    prev = torch.randn(3, 9, 48, dtype=torch.float64)
    inj = inj.double()
    for pl in (None, prev):
        got, p = inj(z, pl)
        pr = inj.feature_up(inj.feature_down(z))
        pp = F.pad(pr, (0, 0, 1, 0))[:, :-1, :]
        if pl is not None:
            pp = torch.cat([pl[:, :1, :], pp[:, 1:, :]], dim=1)
        gate = torch.sigmoid(inj.gate_q(z) + inj.gate_p(pp) + inj.gate_bias)
        ref = z + gate * inj.inject(pp)
        torch.testing.assert_close(got, ref, rtol=1e-12, atol=1e-12)
        torch.testing.assert_close(p, pr, rtol=1e-12, atol=1e-12)


def test_sparse_row_gather_gradient_equals_the_dense_embedding_gradient():
    """The trainer's gathers from the tied weight return sparse row-sum gradients, which
    autograd adds into the head's dense gradient. The weight's .grad must equal the dense
    embedding backward's accumulation (duplicate ids included); torch.autograd.grad with a
    preset .grad must return the lookup's own gradient and leave .grad untouched."""
    import torch.nn.functional as F
    from ksdraft_amd.kernels.embedding import gather_rows_sparse_grad
    torch.manual_seed(0)
    w = torch.randn(50, 8, requires_grad=True)
    ids = torch.tensor([[3, 7, 3], [49, 0, 7], [3, 3, 12]])
    ids2 = torch.tensor([[0, 0, 5], [7, 7, 7], [49, 1, 2]])
    g, g2 = torch.randn(3, 3, 8), torch.randn(3, 3, 8)
    x, gh = torch.randn(6, 8), torch.randn(6, 50)
    out = gather_rows_sparse_grad(w, ids)
    assert torch.equal(out, F.embedding(ids, w))

    def step(gather):
        w.grad = None
        loss = ((x @ w.t()) * gh).sum() + (gather(ids, w) * g).sum() + (gather(ids2, w) * g2).sum()
        loss.backward()
        return w.grad
    got = step(lambda i, ww: gather_rows_sparse_grad(ww, i))
    assert got.layout == torch.strided and got.shape == w.shape
    exp = step(F.embedding)
    torch.testing.assert_close(got, exp, rtol=1e-6, atol=1e-6)

    # one gather beside the head: the same two additions per element, bit for bit
    w.grad = None
    ((x @ w.t()) * gh).sum().add((gather_rows_sparse_grad(w, ids) * g).sum()).backward()
    one = w.grad.clone()
    w.grad = None
    ((x @ w.t()) * gh).sum().add((F.embedding(ids, w) * g).sum()).backward()
    assert torch.equal(one, w.grad)

    # autograd.grad with .grad already set: no side effects, the lookup's own gradient
    preset = torch.randn(50, 8)
    w.grad = preset.clone()
    (gr,) = torch.autograd.grad((gather_rows_sparse_grad(w, ids) * g).sum(), w)
    (ge,) = torch.autograd.grad((F.embedding(ids, w) * g).sum(), w)
    assert torch.equal(gr.to_dense(), ge)
    assert torch.equal(w.grad, preset)


def test_loss_scale_must_be_a_power_of_two():
    from ksdraft_amd.train.int8_step import _check_loss_scale
    assert _check_loss_scale(1) == 1.0 and _check_loss_scale(4096.0) == 4096.0
    assert _check_loss_scale(2.0 ** -3) == 0.125
    for bad in (0, -2.0, 3.0, 1000.0, float("inf"), float("nan")):
        with pytest.raises(ValueError):
            _check_loss_scale(bad)
