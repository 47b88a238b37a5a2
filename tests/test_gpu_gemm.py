"""GPU parity: the W8A8 GEMM kernel.

Bars: int32 group partials bit-exact (brute force oracle); fp32 output bit-exact vs the
ordered-group contract oracle; within rtol/atol 1e-3 of the reference CPU path
(dequantize + fp32 matmul, gemm.py:76-82) — the reference's own GPU test uses rtol 1e-4 /
atol 1e-3 (tests/test_int8.py:80), which is asserted too.
"""

import numpy as np
import pytest
import torch

from ksdraft_amd.kernels import gemm as kg
from ksdraft_amd.kernels import quant as kq
from oracle import gemm as og
from oracle import quant as oq

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _operands(seed, M, K, N, wscale=0.1, group=128):
    g = torch.Generator().manual_seed(seed)
    a = torch.randn(M, K, generator=g)
    w = torch.randn(N, K, generator=g) * wscale
    aq, as_ = oq.quantize_last_dim(a.numpy(), group)
    wq, ws = oq.quantize_last_dim(w.numpy(), group)
    return aq, as_, wq, ws


def _gpu(*arrs):
    return [torch.from_numpy(np.ascontiguousarray(a)).to(DEV) for a in arrs]


# the reference's own GPU parity shapes, tests/test_int8.py:73
REF_SHAPES = [(16, 256, 128), (64, 128, 96), (33, 384, 64), (128, 128, 128)]


@pytest.mark.parametrize("M,K,N", REF_SHAPES + [(256, 1536, 1536), (1, 128, 1), (200, 640, 260)])
def test_gemm_bit_exact_and_within_reference_tolerance(M, K, N):
    aq, as_, wq, ws = _operands(3 + M, M, K, N)
    y = kg.w8a8_gemm(*_gpu(aq, as_, wq, ws)).cpu().numpy()
    ordered = og.gemm_ordered(aq, as_, wq, ws)
    assert np.array_equal(y.view(np.uint32), ordered.view(np.uint32))
    ref = og.gemm_reference(aq, as_, wq, ws)
    np.testing.assert_allclose(y, ref, rtol=1e-4, atol=1e-3)


@pytest.mark.parametrize("group", [32, 64, 128])
@pytest.mark.parametrize("M,K,N", [(64, 256, 96), (40, 384, 130)])
def test_group_partials_bit_exact(M, K, N, group):
    aq, _, wq, _ = _operands(7, M, K, N, group=group)
    p = kg.w8a8_group_partials(*_gpu(aq, wq), group=group).cpu().numpy()
    assert np.array_equal(p, og.group_partials(aq, wq, group))


@pytest.mark.parametrize("group", [32, 64])
def test_small_groups(group):
    aq, as_, wq, ws = _operands(9, 48, 320, 72, group=group)
    y = kg.w8a8_gemm(*_gpu(aq, as_, wq, ws), group=group).cpu().numpy()
    assert np.array_equal(y, og.gemm_ordered(aq, as_, wq, ws, group))
    np.testing.assert_allclose(y, og.gemm_reference(aq, as_, wq, ws, group), rtol=1e-4, atol=1e-3)


def test_ragged_k_is_zero_padded():
    g = torch.Generator().manual_seed(1)
    a = torch.randn(5, 100, generator=g)
    w = torch.randn(6, 100, generator=g)
    aq, as_ = oq.quantize_last_dim(a.numpy())
    wq, ws = oq.quantize_last_dim(w.numpy())
    y = kg.w8a8_gemm(*_gpu(aq, as_, wq, ws)).cpu().numpy()
    assert np.array_equal(y, og.gemm_ordered(aq, as_, wq, ws))


def test_epilogue_bias_and_output_dtypes():
    aq, as_, wq, ws = _operands(11, 70, 512, 300)
    bias = torch.randn(300, generator=torch.Generator().manual_seed(2))
    ta = _gpu(aq, as_, wq, ws)
    exp = torch.from_numpy(og.gemm_ordered(aq, as_, wq, ws, bias=bias.numpy()))
    y32 = kg.w8a8_gemm_out(*ta, bias=bias.to(DEV)).cpu()
    torch.testing.assert_close(y32, exp, rtol=0, atol=0)
    ybf = kg.w8a8_gemm_out(*ta, bias=bias.to(DEV), out_dtype=torch.bfloat16).cpu()
    torch.testing.assert_close(ybf, exp.to(torch.bfloat16), rtol=0, atol=0)
    y16 = kg.w8a8_gemm_out(*ta, out_dtype=torch.float16).cpu()
    torch.testing.assert_close(y16, torch.from_numpy(og.gemm_ordered(aq, as_, wq, ws)).half(),
                               rtol=0, atol=0)


def test_fp16_saturating_output():
    # coords = fp16(acc).clamp(+-65504) (ks3_int8.py:241-242)
    a = np.full((4, 128), 127, np.int8)
    w = np.full((4, 128), 127, np.int8)
    sa = np.full((4, 1), 2.0, np.float16)
    sw = np.array([[1.0], [-1.0], [1e-3], [0.5]], np.float16)
    y = kg.w8a8_gemm_out(*_gpu(a, sa, w, sw), fp16_saturate=True).cpu()
    ref = torch.from_numpy(og.gemm_ordered(a, sa, w, sw)).half().clamp(-65504, 65504)
    assert torch.equal(y, ref)
    assert y[0, 0].item() == 65504.0 and y[0, 1].item() == -65504.0


def test_config1_forward_full_oracle():
    """M=256, K=N=1536, X~N(0,1), W~N(0,0.02), seed 0, fp32 out."""
    g = torch.Generator().manual_seed(0)
    x = torch.randn(256, 1536, generator=g)
    w = torch.randn(1536, 1536, generator=g) * 0.02
    xq, xs = kq.quantize_last_dim(x.to(DEV))
    wq, ws = kq.quantize_last_dim(w.to(DEV))
    y = kg.w8a8_gemm(xq, xs, wq, ws).cpu().numpy()
    exq, exs = oq.quantize_last_dim(x.numpy())
    ewq, ews = oq.quantize_last_dim(w.numpy())
    assert np.array_equal(xq.cpu().numpy(), exq) and np.array_equal(wq.cpu().numpy(), ewq)
    assert np.array_equal(y, og.gemm_ordered(exq, exs, ewq, ews))
    np.testing.assert_allclose(y, og.gemm_reference(exq, exs, ewq, ews), rtol=1e-3, atol=1e-3)


def test_config2_forward_sampled_rows():
    """BASELINE config 2 forward at full size (M=8192, K=N=1536): 96 sampled rows checked
    bit-exactly against the ordered oracle; partials of 8 rows bit-exact."""
    g = torch.Generator().manual_seed(0)
    x = torch.randn(8192, 1536, generator=g)
    w = torch.randn(1536, 1536, generator=g) * 0.02
    xq, xs = kq.quantize_last_dim(x.to(DEV))
    wq, ws = kq.quantize_last_dim(w.to(DEV))
    y = kg.w8a8_gemm(xq, xs, wq, ws)
    rows = np.sort(np.random.default_rng(0).choice(8192, 96, replace=False))
    hq, hs, hwq, hws = (t.cpu().numpy() for t in (xq, xs, wq, ws))
    exp = og.gemm_ordered(hq, hs, hwq, hws, rows=rows)
    assert np.array_equal(y.cpu().numpy()[rows], exp)
    p = kg.w8a8_group_partials(xq[:128], wq).cpu().numpy()
    assert np.array_equal(p[:, :8], og.group_partials(hq[:8], hwq))


@pytest.mark.parametrize("mag", [1e-4, 3e-7])
def test_subnormal_fp16_scales(mag):
    """Inputs this small give fp16-subnormal group scales (amax/127 < 6.1e-5)."""
    g = torch.Generator().manual_seed(21)
    a = torch.randn(96, 384, generator=g) * mag
    w = torch.randn(160, 384, generator=g) * mag
    aq, as_ = oq.quantize_last_dim(a.numpy())
    wq, ws = oq.quantize_last_dim(w.numpy())
    assert (np.abs(as_.astype(np.float32)) < 6.1e-5).all()
    y = kg.w8a8_gemm(*_gpu(aq, as_, wq, ws)).cpu().numpy()
    assert np.array_equal(y, og.gemm_ordered(aq, as_, wq, ws))


def test_many_tiles_persistent_chunks():
    """More tiles than CUs and an odd K-step count per tile (KT=5)."""
    aq, as_, wq, ws = _operands(23, 2304, 640, 1920)
    y = kg.w8a8_gemm(*_gpu(aq, as_, wq, ws)).cpu().numpy()
    rows = np.arange(0, 2304, 37)
    assert np.array_equal(y[rows], og.gemm_ordered(aq, as_, wq, ws, rows=rows))


@pytest.mark.parametrize("M,K,N", [(512, 8192, 1536), (1536, 8192, 512), (256, 2048, 256),
                                   (200, 4096, 130), (64, 16384, 96)])
def test_split_k_shapes_bit_exact(M, K, N):
    """Shapes with few output tiles run split into K parts (the dW of narrow layers, e.g.
    the Rosa projections at 8192 tokens): bit-exact against the split contract, for every
    output type and with bias."""
    S = og.splits_for(M, N, K)
    assert S > 1 and kg.gemm_splits(M, N, K) == S
    aq, as_, wq, ws = _operands(31 + M, M, K, N)
    ta = _gpu(aq, as_, wq, ws)
    y = kg.w8a8_gemm(*ta).cpu().numpy()
    assert np.array_equal(y.view(np.uint32), og.gemm_ordered(aq, as_, wq, ws).view(np.uint32))
    bias = torch.randn(N, generator=torch.Generator().manual_seed(M))
    exp = torch.from_numpy(og.gemm_ordered(aq, as_, wq, ws, bias=bias.numpy()))
    for dt in (torch.float32, torch.bfloat16, torch.float16):
        got = kg.w8a8_gemm_out(*ta, bias=bias.to(DEV), out_dtype=dt).cpu()
        assert torch.equal(got, exp.to(dt)), dt
    np.testing.assert_allclose(y, og.gemm_reference(aq, as_, wq, ws), rtol=1e-4, atol=1e-3)


@pytest.mark.parametrize("M,K,N", [(200, 640, 260), (256, 2048, 256)])
def test_residual_store(M, K, N):
    """y = out(out(gemm + bias) + r): the residual add of `x + linear(x')` in the output
    dtype, fused in the store, bit-exact against the oracle GEMM followed by torch's add
    in that dtype; also in place (y aliasing r) and on a split-K shape."""
    aq, as_, wq, ws = _operands(41 + M, M, K, N)
    ta = _gpu(aq, as_, wq, ws)
    g = torch.Generator().manual_seed(K)
    bias = torch.randn(N, generator=g)
    base = torch.from_numpy(og.gemm_ordered(aq, as_, wq, ws, bias=bias.numpy()))
    for dt in (torch.float32, torch.bfloat16, torch.float16):
        r = (torch.randn(M, N, generator=g) * 3).to(dt)
        exp = r + base.to(dt)
        got = kg.w8a8_gemm_out(*ta, bias=bias.to(DEV), out_dtype=dt, residual=r.to(DEV)).cpu()
        assert torch.equal(got, exp), dt
        rd = r.to(DEV)
        kg.w8a8_gemm_out(*ta, bias=bias.to(DEV), out_dtype=dt, residual=rd, out=rd)
        assert torch.equal(rd.cpu(), exp), dt
    with pytest.raises(ValueError):
        kg.w8a8_gemm_out(*ta, residual=torch.zeros(M, N, device=DEV), fp16_saturate=True)


def test_int8linear_residual_autograd():
    """Int8Linear(x, residual=r) = r + Int8Linear(x), forward and backward (r's gradient is
    the upstream gradient), in training and eval."""
    from ksdraft_amd.kernels import Int8Linear
    torch.manual_seed(9)
    lin = Int8Linear(256, 384).to(DEV)
    with torch.no_grad():
        lin.weight.normal_(0, 0.05)
        lin.bias.normal_(0, 0.1)
    x = torch.randn(3, 40, 256, device=DEV)
    r = torch.randn(3, 40, 384, device=DEV)
    xa, ra = x.clone().requires_grad_(True), r.clone().requires_grad_(True)
    xb, rb = x.clone().requires_grad_(True), r.clone().requires_grad_(True)
    ya = lin(xa, residual=ra)
    yb = rb + lin(xb)
    assert torch.equal(ya, yb)
    g = torch.randn_like(ya)
    ya.backward(g)
    wga = lin.weight.grad.clone()
    lin.weight.grad = None
    yb.backward(g)
    assert torch.equal(xa.grad, xb.grad) and torch.equal(ra.grad, rb.grad)
    assert torch.equal(wga, lin.weight.grad)
    with torch.no_grad():
        assert torch.equal(lin(x, residual=r), r + lin(x))
