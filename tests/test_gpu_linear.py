"""GPU parity: Int8Linear (eval W8A8 path) and the int8-native training autograd.

The backward recipe follows reference ksdraft/kernels/ks3_int8.py:403-424 (the only
int8-operand backward in the reference): dX = quant_N(dY) . requant_N(W)^T and
dW = quant_M(dY)^T . requant_M(dequant(quant(X)))^T. Operands are checked bit-exactly
against the oracle, outputs bit-exactly against the ordered-group contract and within
rtol/atol 1e-3 of the reference CPU GEMM on the same operands.
"""

import numpy as np
import pytest
import torch

from ksdraft_amd.kernels import Int8Linear
from ksdraft_amd.kernels.linear import W8A8LinearFunction
from oracle import gemm as og
from oracle import quant as oq

pytestmark = pytest.mark.gpu
DEV = "cuda"


def test_int8_linear_matches_fp32_within_int8_tolerance():
    # reference tests/test_int8.py:43-55, on the GPU path
    g = torch.Generator().manual_seed(1)
    for M, K, N in ((8, 256, 128), (33, 128, 64), (4, 384, 96)):
        ref = torch.nn.Linear(K, N, bias=True)
        with torch.no_grad():
            ref.weight.normal_(0, 0.1, generator=g)
            ref.bias.normal_(0, 0.1, generator=g)
        lin = Int8Linear.from_float(ref.to(DEV))
        x = torch.randn(M, K, generator=g)
        with torch.no_grad():
            y = lin(x.to(DEV)).cpu()
            y_ref = ref.cpu()(x)
        assert ((y - y_ref).norm() / y_ref.norm()).item() < 0.05


def test_eval_forward_bit_exact():
    g = torch.Generator().manual_seed(4)
    ref = torch.nn.Linear(256, 128, bias=True)
    with torch.no_grad():
        ref.weight.normal_(0, 0.05, generator=g)
        ref.bias.normal_(0, 0.1, generator=g)
    lin = Int8Linear.from_float(ref.to(DEV))
    x = torch.randn(48, 256, generator=g)
    with torch.no_grad():
        y = lin(x.to(DEV)).cpu().numpy()
    xq, xs = oq.quantize_last_dim(x.numpy())
    wq, ws = oq.quantize_last_dim(ref.weight.detach().cpu().numpy())
    exp = og.gemm_ordered(xq, xs, wq, ws, bias=ref.bias.detach().cpu().numpy())
    assert np.array_equal(y, exp)
    np.testing.assert_allclose(y, og.gemm_reference(xq, xs, wq, ws) + ref.bias.detach().cpu().numpy(),
                               rtol=1e-4, atol=1e-3)


def _recipe(x, w, gy, group=128):
    """Oracle for one int8 training step of a linear layer (bias omitted)."""
    xq, xs = oq.quantize_last_dim(x, group)
    wq, ws = oq.quantize_last_dim(w, group)
    y = og.gemm_ordered(xq, xs, wq, ws, group)
    gq, gs = oq.quantize_last_dim(gy, group)
    wtq, wts = oq.requant_transpose(wq, ws, group, group)
    dx = og.gemm_ordered(gq, gs, wtq, wts, group)
    dx_ref = og.gemm_reference(gq, gs, wtq, wts, group)
    gtq, gts = oq.quantize_transpose(gy, group)
    xtq, xts = oq.requant_transpose(xq, xs, group, group)
    dw = og.gemm_ordered(gtq, gts, xtq, xts, group)
    dw_ref = og.gemm_reference(gtq, gts, xtq, xts, group)
    return y, dx, dx_ref, dw, dw_ref


@pytest.mark.parametrize("M,K,N", [(256, 384, 256), (33, 256, 96), (200, 128, 520)])
def test_training_step_matches_recipe(M, K, N):
    g = torch.Generator().manual_seed(M + K + N)
    x = torch.randn(M, K, generator=g)
    w = torch.randn(N, K, generator=g) * 0.02
    b = torch.randn(N, generator=g) * 0.1
    gy = torch.randn(M, N, generator=g) * 1e-2
    lin = Int8Linear(K, N, bias=True).to(DEV)
    with torch.no_grad():
        lin.weight.copy_(w)
        lin.bias.copy_(b)
    xd = x.to(DEV).requires_grad_(True)
    y = lin(xd)
    # training quantizes W and dX's W^T operand in one dual pass (no requant in backward)
    assert lin._wt is not None and lin._wt_src is lin.weight_codes
    y.backward(gy.to(DEV))
    ey, edx, edx_ref, edw, edw_ref = _recipe(x.numpy(), w.numpy(), gy.numpy())
    assert np.array_equal(y.detach().cpu().numpy(), (ey + b.numpy()).astype(np.float32))
    dx = xd.grad.cpu().numpy()
    dw = lin.weight.grad.cpu().numpy()
    assert np.array_equal(dx, edx)
    assert np.array_equal(dw, edw)
    np.testing.assert_allclose(dx, edx_ref, rtol=1e-3, atol=1e-3)
    np.testing.assert_allclose(dw, edw_ref, rtol=1e-3, atol=1e-3)
    np.testing.assert_allclose(lin.bias.grad.cpu().numpy(), gy.numpy().sum(0), rtol=1e-4, atol=1e-5)


def test_training_grads_track_fp32_reference():
    """The int8 backward stays close to fp32 autograd of the same layer (sanity)."""
    g = torch.Generator().manual_seed(0)
    M, K, N = 512, 512, 384
    x = torch.randn(M, K, generator=g)
    w = torch.randn(N, K, generator=g) * 0.02
    gy = torch.randn(M, N, generator=g) * 1e-2
    lin = Int8Linear(K, N, bias=False).to(DEV)
    with torch.no_grad():
        lin.weight.copy_(w)
    xd = x.to(DEV).requires_grad_(True)
    lin(xd).backward(gy.to(DEV))
    xr = x.clone().requires_grad_(True)
    wr = w.clone().requires_grad_(True)
    (xr @ wr.T).backward(gy)
    cos = torch.nn.functional.cosine_similarity
    assert cos(xd.grad.cpu().flatten(), xr.grad.flatten(), dim=0) > 0.99
    assert cos(lin.weight.grad.cpu().flatten(), wr.grad.flatten(), dim=0) > 0.99


def test_bf16_activations_round_trip_dtype():
    lin = Int8Linear(256, 128).to(DEV)
    with torch.no_grad():
        lin.weight.normal_(0, 0.02)
    x = torch.randn(4, 7, 256, device=DEV, dtype=torch.bfloat16, requires_grad=True)
    y = lin(x)
    assert y.dtype == torch.bfloat16 and y.shape == (4, 7, 128)
    y.float().square().mean().backward()
    assert x.grad.dtype == torch.bfloat16 and torch.isfinite(x.grad.float()).all()
    assert lin.weight.grad.dtype == torch.float32


def test_ste_training_keeps_reference_behaviour():
    # reference tests/test_int8.py:58-66 (fake_quant_forward STE grads)
    torch.manual_seed(2)
    lin = Int8Linear.from_float(torch.nn.Linear(64, 32, bias=True).to(DEV))
    x = torch.randn(4, 64, device=DEV, requires_grad=True)
    y = lin.fake_quant_forward(x)
    y.square().mean().backward()
    assert x.grad is not None and torch.isfinite(x.grad).all()
    assert lin.weight.grad is not None and torch.isfinite(lin.weight.grad).all()
    assert W8A8LinearFunction is not None
