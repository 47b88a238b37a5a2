"""GPU parity: the fused LayerNorm + GS128 quantization (ksdraft_amd.kernels.quant.
layer_norm_quantize) against torch's LayerNorm and the oracle quantizer.

The path it replaces is nn.LayerNorm (reference ksdraft/model/block.py:27-41) followed by
quantize_last_dim of its output (kernels/linear.py:69).

Bars:
- y is TOL against F.layer_norm in float64 on the CPU. The kernel's mean/variance sum
  order is its own: for fp32 output an absolute 1e-4 (the inputs are O(1) to O(30)); for
  bf16/fp16 output, the dtype's rounding of the float64 result within one ulp.
- Given the kernel's own y (returned on request), codes and fp16 scales are bit-exact
  against oracle/quant.py's quantize_last_dim of y, and the call without the y copy gives
  the same operands.
- mean and rstd are TOL against float64 (1e-5 relative).
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from ksdraft_amd.kernels import quant as kq
from oracle import quant as oq

pytestmark = pytest.mark.gpu
DEV = "cuda"
ULP = {torch.bfloat16: 2.0 ** -7, torch.float16: 2.0 ** -10}


def _case(R, d, seed, offset=0.0, affine=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(R, d, generator=g) * 2.0 + offset
    if R > 2:
        x[1] = 0.5  # a constant row: mean exact, variance 0, y = bias
        x[2] *= 1e-3
    w = (1.0 + 0.3 * torch.randn(d, generator=g)) if affine else None
    b = (0.2 * torch.randn(d, generator=g)) if affine else None
    return x, w, b


def _ref(x, w, b, eps):
    x64 = x.double()
    y = F.layer_norm(x64, (x.shape[-1],), None if w is None else w.double(),
                     None if b is None else b.double(), eps)
    mean = x64.mean(dim=-1)
    rstd = 1.0 / torch.sqrt(x64.var(dim=-1, unbiased=False) + eps)
    return y, mean, rstd


def _check_codes(y, codes, scales):
    ec, es = oq.quantize_last_dim(y.float().cpu().numpy(), 128)
    assert np.array_equal(codes.cpu().numpy(), ec)
    assert np.array_equal(scales.cpu().numpy().view(np.uint16), es.view(np.uint16))


@pytest.mark.parametrize("R,d", [(300, 1536), (64, 4096), (130, 200), (1, 128), (257, 1000),
                                 (33, 129)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_layer_norm_quantize_matches_torch_and_oracle(R, d, dtype):
    x, w, b = _case(R, d, seed=R * 31 + d)
    xd = x.to(dtype)
    eps = 1e-5
    codes, scales, y, mean, rstd = kq.layer_norm_quantize(
        xd.to(DEV), w.to(DEV), b.to(DEV), eps, return_y=True, return_stats=True)
    torch.cuda.synchronize()
    assert y.dtype == dtype and codes.shape == (R, d) and scales.shape == (R, -(-d // 128))
    ey, em, er = _ref(xd.float(), w, b, eps)
    yk = y.double().cpu()
    if dtype == torch.float32:
        assert (yk - ey).abs().max().item() <= 1e-4
    else:
        assert torch.all((yk - ey).abs() <= ULP[dtype] * ey.abs().clamp_min(1e-3)), \
            float(((yk - ey).abs() / ey.abs().clamp_min(1e-3)).max())
    torch.testing.assert_close(mean.double().cpu(), em, rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(rstd.double().cpu(), er, rtol=1e-5, atol=0.0)
    _check_codes(y, codes, scales)
    # the constant row: y is the bias exactly
    if R > 2 and dtype == torch.float32:
        assert torch.equal(y[1].cpu(), b)
    # without the y copy (and the stats) the kernel gives the same operands
    c2, s2 = kq.layer_norm_quantize(xd.to(DEV), w.to(DEV), b.to(DEV), eps)
    assert torch.equal(c2, codes) and torch.equal(s2, scales)
    # and they are quantize_last_dim of y on the device too
    c3, s3 = kq.quantize_last_dim(y)
    assert torch.equal(c3, codes) and torch.equal(s3, scales)


def test_layer_norm_quantize_no_affine_offset_and_strided():
    x, _, _ = _case(96, 1536, seed=7, offset=30.0, affine=False)
    wide = torch.zeros(96, 1600)
    wide[:, :1536] = x
    xv = wide.to(DEV)[:, :1536]  # row stride 1600
    codes, scales, y = kq.layer_norm_quantize(xv, eps=1e-6, return_y=True)
    ey, _, _ = _ref(x, None, None, 1e-6)
    assert (y.double().cpu() - ey).abs().max().item() <= 1e-4
    _check_codes(y, codes, scales)
    # against torch's own fp32 LayerNorm on the device, then the library quantizer
    yt = F.layer_norm(xv, (1536,), eps=1e-6)
    assert (yt - y).abs().max().item() <= 1e-4
    # leading dims are kept
    c4, s4 = kq.layer_norm_quantize(x.to(DEV).reshape(4, 24, 1536), eps=1e-6)
    assert c4.shape == (4, 24, 1536) and s4.shape == (4, 24, 12)
    assert torch.equal(c4.reshape(96, 1536), codes)


def test_layer_norm_quantize_rejects_bad_input():
    with pytest.raises(ValueError):
        kq.layer_norm_quantize(torch.randn(4, 4097, device=DEV))
    with pytest.raises(ValueError):
        kq.layer_norm_quantize(torch.randn(4, 256, device=DEV), torch.ones(255, device=DEV))
    with pytest.raises(ValueError):
        kq.layer_norm_quantize(torch.randn(4, 256, device=DEV), group=64)
    with pytest.raises(RuntimeError):
        kq.layer_norm_quantize(torch.randn(4, 256))
