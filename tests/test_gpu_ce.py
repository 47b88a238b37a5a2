"""GPU parity: the fused cross-entropy gradient (ksdraft_amd/train) against torch and the
oracle quantizer.

Bars:
- The loss and dY are TOL against torch's F.cross_entropy in float64 on the CPU, the
  reference's own call (ksdraft/train/__init__.py:77). The kernel's exp and its sum order
  are its own, so only a tolerance applies: rtol 2e-5 on the loss, and on dY an absolute
  1e-5 of the gradient scale per element (dY is (softmax - onehot) * grad_scale).
- Given the kernel's own dY (returned on request), the int8 codes and fp16 scales of both
  layouts are bit-exact against oracle/quant.py's quantize_last_dim of dY and of dY^T.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from ksdraft_amd import train as T
from ksdraft_amd.kernels import quant as kq
from oracle import quant as oq

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(R, C, seed, spread=4.0, ignore_frac=0.1):
    g = torch.Generator().manual_seed(seed)
    y = torch.randn(R, C, generator=g) * spread
    if R > 2:  # one row with a dominant logit, one with -inf entries (masked classes)
        y[0, C // 3] += 40.0
        y[1, : C // 2] = -float("inf")
    t = torch.randint(0, C, (R,), generator=g)
    if R > 2:
        t[1] = C - 1  # the masked row's target is a live class
    t[torch.rand(R, generator=g) < ignore_frac] = T.IGNORE_INDEX
    if R > 3:
        t[3] = T.IGNORE_INDEX
    return y, t


def _torch_ref(y, t, grad_output=1.0):
    y64 = y.double().requires_grad_(True)
    loss = F.cross_entropy(y64, t, ignore_index=T.IGNORE_INDEX)
    loss.backward(torch.tensor(grad_output, dtype=torch.float64))
    return loss.item(), y64.grad.numpy()


def _check_codes(dy, ops):
    codes, scales, codes_t, scales_t = (a.cpu().numpy() for a in ops)
    ec, es = oq.quantize_last_dim(dy, 128)
    assert np.array_equal(codes, ec)
    assert np.array_equal(scales.view(np.uint16), es.view(np.uint16))
    etc, ets = oq.quantize_last_dim(np.ascontiguousarray(dy.T), 128)
    assert np.array_equal(codes_t, etc)
    assert np.array_equal(scales_t.view(np.uint16), ets.view(np.uint16))


@pytest.mark.parametrize("R,C", [(300, 1000), (256, 2048), (130, 389), (1, 128), (129, 1544),
                                 (64, 4096)])
def test_cross_entropy_int8_matches_torch_and_oracle(R, C):
    y, t = _case(R, C, seed=R * 7 + C)
    loss, ops, dy = T.cross_entropy_int8(y.to(DEV), t.to(DEV), grad_output=0.75, return_dy=True)
    torch.cuda.synchronize()
    eloss, edy = _torch_ref(y, t, 0.75)
    assert abs(loss.item() - eloss) <= 2e-5 * abs(eloss)
    dy = dy.cpu().numpy()
    n = int((t != T.IGNORE_INDEX).sum())
    gscale = 0.75 / n
    assert np.all(np.abs(dy - edy) <= 1e-5 * gscale), float(np.abs(dy - edy).max() / gscale)
    assert np.all(dy[(t == T.IGNORE_INDEX).numpy()] == 0.0)
    _check_codes(dy, ops)
    # without the fp32 copy the fused kernel gives the same operands
    if C % 8 == 0:
        loss2, ops2 = T.cross_entropy_int8(y.to(DEV), t.to(DEV), grad_output=0.75)
        for a, b in zip(ops, ops2):
            assert torch.equal(a, b)
        assert torch.equal(loss, loss2)


def test_cross_entropy_stats_rows():
    y, t = _case(200, 777, seed=5)
    loss, rmax, rinv, n = T.cross_entropy_stats(y.to(DEV), t.to(DEV))
    torch.cuda.synchronize()
    y64 = y.double()
    assert torch.equal(rmax.cpu(), y.max(dim=1).values)
    esum = torch.exp(y64 - y64.max(dim=1, keepdim=True).values).sum(dim=1)
    np.testing.assert_allclose(1.0 / rinv.cpu().double().numpy(), esum.numpy(), rtol=1e-5)
    assert int(n.item()) == int((t != T.IGNORE_INDEX).sum())


def test_cross_entropy_int8_all_ignored_and_bad_targets():
    y = torch.randn(16, 256)
    t = torch.full((16,), T.IGNORE_INDEX)
    loss, ops, dy = T.cross_entropy_int8(y.to(DEV), t.to(DEV), return_dy=True)
    assert torch.isnan(loss).item()  # 0 / 0, as torch's mean gives
    assert torch.count_nonzero(dy).item() == 0 and torch.count_nonzero(ops[0]).item() == 0
    with pytest.raises(IndexError):
        T.cross_entropy_int8(y.to(DEV), torch.full((16,), 256).to(DEV))
    with pytest.raises(IndexError):
        T.cross_entropy_int8(y.to(DEV), torch.full((16,), -3).to(DEV))


def test_cross_entropy_int8_matches_composed_quantization():
    """The fused operands equal quantize_dual of the kernel's dY on the device too."""
    y, t = _case(384, 3072, seed=3)
    _, ops, dy = T.cross_entropy_int8(y.to(DEV), t.to(DEV), return_dy=True)
    ref = kq.quantize_dual(dy)
    for a, b in zip(ops, ref):
        assert torch.equal(a, b)


@pytest.mark.parametrize("xdtype", [torch.float32, torch.bfloat16])
def test_linear_cross_entropy_int8_autograd(xdtype):
    """The int8 head + CE autograd function against the composed int8 path (W8A8 linear,
    torch cross entropy, int8 backward of the torch dY): same loss, gradients within the
    tolerance their one-ulp dY differences allow."""
    from ksdraft_amd.kernels.linear import W8A8LinearFunction

    g = torch.Generator().manual_seed(0)
    M, K, V = 192, 256, 1000
    x = torch.randn(M, K, generator=g).to(DEV, xdtype)
    w = (torch.randn(V, K, generator=g) * 0.02).to(DEV)
    t = torch.randint(0, V, (M,), generator=g).to(DEV)
    t[5] = T.IGNORE_INDEX
    wq, ws = kq.quantize_last_dim(w)

    xa = x.clone().requires_grad_(True)
    wa = w.clone().requires_grad_(True)
    loss = T.LinearCrossEntropyInt8.apply(xa, wa, wq, ws, t, T.IGNORE_INDEX, 128)
    loss.backward()

    xb = x.float().clone().requires_grad_(True)  # fp32 logits on both sides (same codes)
    wb = w.clone().requires_grad_(True)
    yb = W8A8LinearFunction.apply(xb, wb, None, wq, ws, 128).float()
    lb = F.cross_entropy(yb, t, ignore_index=T.IGNORE_INDEX)
    lb.backward()

    assert abs(loss.item() - lb.item()) <= 2e-5 * abs(lb.item())
    assert xa.grad.dtype == xdtype and xa.grad.shape == x.shape
    for ga, gb in ((xa.grad.float(), xb.grad.float()), (wa.grad, wb.grad)):
        err = (ga - gb).abs().max().item()
        assert err <= 2e-2 * gb.abs().max().item(), (err, gb.abs().max().item())


def test_unchecked_out_of_range_targets_count_as_ignored_rows():
    """check_targets=False (graph capture) treats an out-of-range target as an ignored row
    in the kernels; the mean's denominator counts the same rows, so loss and dY equal those
    of the same batch with those targets set to ignore_index."""
    y, t = _case(64, 512, seed=17, ignore_frac=0.0)
    bad = t.clone()
    bad[5], bad[9], bad[20] = 512, -7, 10_000
    fixed = bad.clone()
    fixed[5] = fixed[9] = fixed[20] = T.IGNORE_INDEX
    yd = y.to(DEV)
    loss_b, rmax, rinv, n_b = T.cross_entropy_stats(yd, bad.to(DEV), check_targets=False)
    loss_f, _, _, n_f = T.cross_entropy_stats(yd, fixed.to(DEV))
    n_exp = int((fixed != T.IGNORE_INDEX).sum())
    assert n_b.item() == n_f.item() == n_exp
    assert torch.equal(loss_b, loss_f)
    eloss, edy = _torch_ref(y, fixed)
    assert abs(loss_b.item() - eloss) <= 2e-5 * abs(eloss)
    gsc = torch.ones(1, device=DEV) / n_b
    _, dy = T.cross_entropy_grad_int8(yd, bad.to(DEV), rmax, rinv, gsc, return_dy=True)
    dy = dy.cpu().numpy()
    assert np.all(np.abs(dy - edy) <= 1e-5 / n_exp)
