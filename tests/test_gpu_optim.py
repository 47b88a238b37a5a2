"""GPU parity: the fused AdamW step + int8 repack (ksdraft_amd/train) against
torch.optim.AdamW and the oracle quantizer.

Bars:
- Masters and both moments are TOL against torch.optim.AdamW, the reference's optimizer
  (ksdraft/train/__init__.py:114-116, 166; its single-tensor update order), on the same
  device in fp32: rtol 2e-6 with an absolute floor of 2e-6 of the tensor's largest
  magnitude, after each of three steps. torch's elementwise kernels may contract a*b + c
  into one rounding (its lerp does, judging by the results), and this build does not, so
  moments that cancel to tiny values differ in their last bits.
- The int8 codes and fp16 scales are bit-exact against oracle/quant.py's
  quantize_last_dim of the kernel's own updated master.
"""

import numpy as np
import pytest
import torch

from ksdraft_amd import train as T
from ksdraft_amd.kernels import Int8Linear
from oracle import quant as oq

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _codes_match(p, res):
    codes, scales = (a.cpu().numpy() for a in res)
    ec, es = oq.quantize_last_dim(p.detach().cpu().numpy(), 128)
    assert np.array_equal(codes, ec)
    assert np.array_equal(scales.view(np.uint16), es.view(np.uint16))


@pytest.mark.parametrize("shape", [(256, 384), (130, 200), (1, 1536), (64, 1000), (7, 13)])
@pytest.mark.parametrize("wd,clip", [(0.1, None), (0.0, 0.5)])
def test_adamw_requant_matches_torch(shape, wd, clip):
    g = torch.Generator().manual_seed(hash((shape, wd)) % 2**31)
    p0 = (torch.randn(*shape, generator=g) * 0.02).to(DEV)
    ref = p0.clone().requires_grad_(True)
    opt = torch.optim.AdamW([ref], lr=3e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=wd,
                            foreach=False)
    p = p0.clone()
    m = torch.zeros_like(p)
    v = torch.zeros_like(p)
    cc = None if clip is None else torch.tensor([clip], device=DEV)
    for step in range(1, 4):
        grad = (torch.randn(*shape, generator=g) * 0.01).to(DEV)
        ref.grad = grad * clip if clip is not None else grad.clone()
        opt.step()
        res = T.adamw_requant_(p, grad, m, v, step, 3e-3, (0.9, 0.95), 1e-8, wd, clip_coef=cc)
        torch.cuda.synchronize()
        st = opt.state[ref]
        for got, exp in ((p, ref.detach()), (m, st["exp_avg"]), (v, st["exp_avg_sq"])):
            torch.testing.assert_close(got, exp, rtol=2e-6, atol=2e-6 * exp.abs().max().item())
        _codes_match(p, res)


@pytest.mark.parametrize("clip", [None, 0.7])
def test_adamw_requant_multi_equals_one_call_per_master(clip):
    """ksd_adamw_requant_multi over 60 masters (more than one launch batch: ragged K, 1-D
    and 3-D shapes, with and without the int8 repack, different step counts, misaligned
    views) gives the bits of one ksd_adamw_requant call per master."""
    g = torch.Generator().manual_seed(11 if clip is None else 12)
    shapes = [(256, 384), (130, 200), (1536,), (7, 13), (3, 5, 136), (64, 1000), (1, 1)] * 8
    shapes = shapes[:60]
    cc = None if clip is None else torch.tensor([clip], device=DEV)
    items, ref = [], []
    for i, sh in enumerate(shapes):
        p0 = (torch.randn(*sh, generator=g) * 0.02).to(DEV)
        grad = (torch.randn(*sh, generator=g) * 0.01).to(DEV)
        m0 = (torch.randn(*sh, generator=g) * 1e-3).to(DEV)
        v0 = (torch.rand(*sh, generator=g) * 1e-5).to(DEV)
        step = 1 + i % 5
        quant = i % 3 != 2

        def param_copy():
            if i % 9 != 4:
                return p0.clone()
            buf = torch.zeros(p0.numel() + 1, device=DEV)  # misaligned, contiguous: unvectorised
            buf[1:] = p0.reshape(-1)
            return buf[1:].view(sh)
        items.append((param_copy(), grad, m0.clone(), v0.clone(), step, quant))
        ref.append((param_copy(), grad, m0.clone(), v0.clone(), step, quant))
    got = T.adamw_requant_multi_(items, 3e-3, (0.9, 0.95), 1e-8, 0.05, clip_coef=cc)
    exp = [T.adamw_requant_(p, gr, m, v, st, 3e-3, (0.9, 0.95), 1e-8, 0.05, clip_coef=cc, quantize=q)
           for p, gr, m, v, st, q in ref]
    torch.cuda.synchronize()
    for a, b, ra, rb in zip(items, ref, got, exp):
        for x, y in zip(a[:4], b[:4]):
            assert torch.equal(x.view(torch.int32), y.view(torch.int32))
        assert (ra is None) == (rb is None)
        if ra is not None:
            assert torch.equal(ra[0], rb[0]) and torch.equal(ra[1].view(torch.int16), rb[1].view(torch.int16))


def test_requant_transpose_multi_equals_one_call_per_tensor():
    """ksd_requant_transpose_multi over 70 tensors (more than two launch batches; ragged R
    and C, one-row and one-column tensors, an unaligned view) gives the bits of one
    ksd_requant_transpose call per tensor."""
    from ksdraft_amd.kernels.quant import quantize_last_dim, requant_transpose, requant_transpose_multi
    g = torch.Generator().manual_seed(5)
    shapes = [(1536, 1536), (200, 130), (1, 384), (384, 1), (129, 257), (64, 96), (300, 1000)] * 10
    pairs = []
    for i, sh in enumerate(shapes):
        x = (torch.randn(*sh, generator=g) * (0.02 + i)).to(DEV)
        c, s = quantize_last_dim(x)
        if i % 11 == 3:  # codes at an odd address: the unvectorised loads
            buf = torch.empty(c.numel() + 1, dtype=torch.int8, device=DEV)
            buf[1:] = c.reshape(-1)
            c = buf[1:].view(sh)
        pairs.append((c, s))
    got = requant_transpose_multi(pairs)
    for (c, s), (ct, st) in zip(pairs, got):
        ec, es = requant_transpose(c, s)
        assert torch.equal(ct, ec) and torch.equal(st.view(torch.int16), es.view(torch.int16))


def test_optimizer_hands_over_current_transposes():
    """After AdamWRequant.step, every registered Int8Linear in training mode holds the
    transposed codes of its new codes (dX's operand), equal to requant_transpose of them;
    an eval-mode module gets none, and a forward that requantizes drops the stale ones."""
    from ksdraft_amd.kernels.quant import requant_transpose
    torch.manual_seed(3)
    mods = [Int8Linear(256, 384).to(DEV), Int8Linear(384, 128, bias=False).to(DEV),
            Int8Linear(128, 256).to(DEV)]
    mods[2].eval()
    opt = T.AdamWRequant([p for m in mods for p in m.parameters()], lr=1e-3)
    for m in mods:
        opt.register_int8(m)
    x = torch.randn(64, 256, device=DEV)
    y = mods[1](mods[0](x))
    y.square().mean().backward()
    mods[2].weight.grad = torch.randn_like(mods[2].weight)
    opt.step()
    for m in mods[:2]:
        wt = m.current_transpose()
        assert wt is not None
        ec, es = requant_transpose(m.weight_codes, m.weight_scales)
        assert torch.equal(wt[0], ec) and torch.equal(wt[1].view(torch.int16), es.view(torch.int16))
    assert mods[2].current_transpose() is None
    with torch.no_grad():
        mods[0].weight.add_(1e-3)  # versioned write: the next forward requantizes
    mods[0](x)
    wt = mods[0].current_transpose()
    ec, es = requant_transpose(mods[0].weight_codes, mods[0].weight_scales)
    assert wt is None or (torch.equal(wt[0], ec) and torch.equal(wt[1].view(torch.int16), es.view(torch.int16)))


def test_adamw_requant_optimizer_drives_int8linear():
    """AdamWRequant on an Int8Linear: after the step the module's codes are those of the
    updated master, and the next forward uses them without rebuilding them."""
    torch.manual_seed(0)
    lin = Int8Linear(256, 384).to(DEV)
    with torch.no_grad():
        lin.weight.normal_(0, 0.02)
    lin_ref = Int8Linear(256, 384).to(DEV)
    lin_ref.load_state_dict(lin.state_dict())
    opt = T.AdamWRequant(lin.parameters(), lr=1e-3, weight_decay=0.01)
    opt.register_int8(lin)
    opt_ref = torch.optim.AdamW(lin_ref.parameters(), lr=1e-3, weight_decay=0.01, foreach=False)
    x = torch.randn(64, 256, device=DEV)
    for _ in range(2):
        for mod, o in ((lin, opt), (lin_ref, opt_ref)):
            o.zero_grad()
            mod(x).square().mean().backward()
            o.step()
        _codes_match(lin.weight, (lin.weight_codes, lin.weight_scales))
        codes = lin.weight_codes
        y = lin(x)  # no requant: the optimizer's codes are current
        assert lin.weight_codes is codes
        torch.testing.assert_close(lin.weight, lin_ref.weight, rtol=2e-6,
                                   atol=2e-6 * lin_ref.weight.abs().max().item())
        torch.testing.assert_close(y, lin_ref(x), rtol=1e-3, atol=1e-4)
    # a torch-side change of the master makes the next forward requantize
    with torch.no_grad():
        lin.weight.mul_(2.0)
    lin(x)
    assert lin.weight_codes is not codes
    _codes_match(lin.weight, (lin.weight_codes, lin.weight_scales))


@pytest.mark.parametrize("betas", [(0.3, 0.999), (0.5, 0.9)])
def test_adamw_requant_small_beta1_uses_torchs_second_lerp_form(betas):
    """beta1 <= 0.5 puts the lerp weight 1 - beta1 at or above 0.5, where torch's lerp
    switches to end - (end - self) * (1 - w); the kernel switches with it."""
    g = torch.Generator().manual_seed(11)
    shape = (96, 384)
    p0 = (torch.randn(*shape, generator=g) * 0.02).to(DEV)
    ref = p0.clone().requires_grad_(True)
    opt = torch.optim.AdamW([ref], lr=3e-3, betas=betas, eps=1e-8, weight_decay=0.01,
                            foreach=False)
    p, m, v = p0.clone(), torch.zeros_like(p0), torch.zeros_like(p0)
    for step in range(1, 4):
        grad = (torch.randn(*shape, generator=g) * 0.01).to(DEV)
        ref.grad = grad.clone()
        opt.step()
        res = T.adamw_requant_(p, grad, m, v, step, 3e-3, betas, 1e-8, 0.01)
        torch.cuda.synchronize()
        st = opt.state[ref]
        for got, exp in ((p, ref.detach()), (m, st["exp_avg"]), (v, st["exp_avg_sq"])):
            torch.testing.assert_close(got, exp, rtol=2e-6, atol=2e-6 * exp.abs().max().item())
        _codes_match(p, res)


def test_registered_int8linear_after_unversioned_write():
    """A write through .data after the step is invisible to torch's version counter: the
    module requantizes once invalidate_codes() is called, and after load_state_dict."""
    torch.manual_seed(1)
    lin = Int8Linear(256, 128).to(DEV)
    with torch.no_grad():
        lin.weight.normal_(0, 0.02)
    opt = T.AdamWRequant(lin.parameters(), lr=1e-3)
    opt.register_int8(lin)
    x = torch.randn(32, 256, device=DEV)
    lin(x).square().mean().backward()
    opt.step()
    lin.weight.data.copy_(torch.randn(128, 256, device=DEV) * 0.05)
    lin.invalidate_codes()
    lin(x)
    _codes_match(lin.weight, (lin.weight_codes, lin.weight_scales))
    sd = {k: v.clone() * 0.5 for k, v in lin.state_dict().items()}
    lin.load_state_dict(sd)
    with torch.no_grad():
        lin(x)
    _codes_match(lin.weight, (lin.weight_codes, lin.weight_scales))


def test_int8linear_accepts_float64_like_the_reference():
    """The reference quantizes x2.float() (linear.py:69) and casts y back to x's dtype."""
    torch.manual_seed(2)
    lin = Int8Linear(256, 64).to(DEV)
    with torch.no_grad():
        lin.weight.normal_(0, 0.02)
        x = torch.randn(16, 256, device=DEV, dtype=torch.float64)
        y = lin(x)
        assert y.dtype == torch.float64
        torch.testing.assert_close(y, lin(x.float()).double(), rtol=0, atol=0)
    xg = x.clone().requires_grad_(True)
    y = lin(xg)
    y.sum().backward()
    assert y.dtype == torch.float64 and xg.grad.dtype == torch.float64


def test_int8_embedding_gather_and_ste_backward():
    """The int8 lookup equals the oracle dequantization of the looked-up rows, bit-exact,
    for every output dtype and group; its gradient is nn.Embedding's (scatter-add)."""
    from ksdraft_amd.kernels.embedding import Int8Embedding, embedding_gather_int8
    from ksdraft_amd.kernels import quant as kq
    g = torch.Generator().manual_seed(13)
    V, d = 1000, 1536
    w = torch.randn(V, d, generator=g) * 0.05
    ids = torch.randint(0, V, (3, 77), generator=g)
    for group in (128, 64, 32):
        codes, scales = kq.quantize_last_dim(w.to(DEV), group)
        ec, es = oq.quantize_last_dim(w.numpy(), group)
        exp = oq.dequantize_last_dim(ec[ids.numpy().reshape(-1)], es[ids.numpy().reshape(-1)], group)
        for dt in (torch.float32, torch.bfloat16, torch.float16):
            got = embedding_gather_int8(codes, scales, ids.to(DEV), group, dt)
            assert got.shape == (3, 77, d)
            assert torch.equal(got.reshape(-1, d).cpu(), torch.from_numpy(exp).to(dt)), (group, dt)
    with pytest.raises(IndexError):
        embedding_gather_int8(codes, scales, torch.tensor([V], device=DEV), 32)
    # ragged d (not a multiple of 8) takes the scalar path
    w2 = torch.randn(50, 300, generator=g)
    c2, s2 = kq.quantize_last_dim(w2.to(DEV))
    i2 = torch.tensor([0, 49, 7, 7], device=DEV)
    e2 = oq.dequantize_last_dim(*oq.quantize_last_dim(w2.numpy()))[[0, 49, 7, 7]]
    assert torch.equal(embedding_gather_int8(c2, s2, i2).cpu(), torch.from_numpy(e2))
    # module: forward from the master's codes, backward = nn.Embedding's scatter-add
    emb = Int8Embedding(V, d).to(DEV)
    with torch.no_grad():
        emb.weight.copy_(w.to(DEV))
    y = emb(ids.to(DEV))
    gy = torch.randn(3, 77, d, generator=g).to(DEV)
    y.backward(gy)
    ref = torch.nn.Embedding(V, d).to(DEV)
    with torch.no_grad():
        ref.weight.copy_(w.to(DEV))
    ref(ids.to(DEV)).backward(gy)
    assert torch.equal(emb.weight.grad, ref.weight.grad)
