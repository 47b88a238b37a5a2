"""GPU parity: quantization kernels vs the oracle, bit-exact codes and fp16 scales."""

import numpy as np
import pytest
import torch

from ksdraft_amd.kernels import quant as kq
from oracle import quant as oq
from tests.test_oracle_quant import _adversarial_rows

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _check(x_cpu, group=128):
    x = x_cpu.to(DEV)
    codes, scales = kq.quantize_last_dim(x, group)
    torch.cuda.synchronize()
    ec, es = oq.quantize_last_dim(x_cpu.float().numpy(), group)
    assert codes.dtype == torch.int8 and scales.dtype == torch.float16
    assert np.array_equal(codes.cpu().numpy(), ec)
    assert np.array_equal(scales.cpu().numpy().view(np.uint16), es.view(np.uint16))


@pytest.mark.parametrize("group", [32, 64, 128])
@pytest.mark.parametrize("shape", [(64, 256), (4, 100), (33, 1536), (3, 7), (1, 1), (5, 136)])
def test_quantize_matches_oracle(shape, group):
    g = torch.Generator().manual_seed(hash((shape, group)) % 2**31)
    _check(torch.randn(*shape, generator=g) * 3, group)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_quantize_half_inputs(dtype):
    g = torch.Generator().manual_seed(11)
    _check((torch.randn(17, 384, generator=g) * 2).to(dtype))


@pytest.mark.parametrize("group", [32, 128])
def test_quantize_adversarial_rounding(group):
    x = _adversarial_rows(np.random.default_rng(99 + group), group)
    _check(torch.from_numpy(x), group)


def test_zero_row_and_extremes():
    _check(torch.zeros(2, 128))
    _check(torch.tensor([[1e-30] * 128, [3e38] * 128, [-7e-8] * 128]))


def test_quantize_leading_dims_and_strided_rows():
    g = torch.Generator().manual_seed(5)
    x = torch.randn(2, 3, 256, generator=g).to(DEV)
    c, s = kq.quantize_last_dim(x)
    assert c.shape == (2, 3, 256) and s.shape == (2, 3, 2)
    ec, es = oq.quantize_last_dim(x.cpu().numpy())
    assert np.array_equal(c.cpu().numpy(), ec)
    big = torch.randn(8, 512, generator=g).to(DEV)
    view = big[:, 128:384]  # rows strided by 512
    c, s = kq.quantize_last_dim(view)
    ec, es = oq.quantize_last_dim(view.cpu().numpy())
    assert np.array_equal(c.cpu().numpy(), ec) and np.array_equal(s.cpu().numpy(), es)


def test_dither_matches_oracle_with_same_draws():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(8, 256, generator=g) * 3
    noise = torch.rand(8, 256, generator=g)
    codes, scales = kq._quantize(x.to(DEV), 128, noise.to(DEV), 0.5)
    ec, es = oq.quantize_last_dim(x.numpy(), 128, noise=noise.numpy(), dither=0.5)
    assert np.array_equal(codes.cpu().numpy(), ec) and np.array_equal(scales.cpu().numpy(), es)
    c0, s0 = kq.quantize_last_dim_dithered(x.to(DEV), 128, 0.0)
    ce, se = kq.quantize_last_dim(x.to(DEV), 128)
    assert torch.equal(c0, ce) and torch.equal(s0, se)


@pytest.mark.parametrize("K,nsc", [(256, 2), (100, 1), (6, 1), (256, 8)])
def test_dequantize_matches_oracle(K, nsc):
    g = torch.Generator().manual_seed(K)
    codes = torch.randint(-127, 128, (9, K), generator=g, dtype=torch.int8)
    scales = (torch.rand(9, nsc, generator=g) * 0.1).half()
    out = kq.dequantize_last_dim(codes.to(DEV), scales.to(DEV))
    ref = oq.dequantize_last_dim(codes.numpy(), scales.numpy())
    assert np.array_equal(out.cpu().numpy(), ref)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("R,C", [(256, 192), (33, 70), (8192, 64), (130, 1)])
def test_quantize_transpose_matches_oracle(R, C, dtype):
    g = torch.Generator().manual_seed(R * 7 + C)
    x = (torch.randn(R, C, generator=g) * 1e-2).to(dtype)
    codes, scales = kq.quantize_transpose(x.to(DEV))
    ec, es = oq.quantize_transpose(x.float().numpy())
    assert np.array_equal(codes.cpu().numpy(), ec)
    assert np.array_equal(scales.cpu().numpy(), es)


@pytest.mark.parametrize("group_in,group", [(128, 128), (128, 32), (32, 128)])
@pytest.mark.parametrize("R,C", [(200, 96), (1536, 1536), (64, 300)])
def test_requant_transpose_matches_oracle(R, C, group_in, group):
    g = torch.Generator().manual_seed(R + C)
    w = torch.randn(R, C, generator=g) * 0.02
    wq, ws = oq.quantize_last_dim(w.numpy(), group_in)
    tq, ts = kq.requant_transpose(torch.from_numpy(wq).to(DEV), torch.from_numpy(ws).to(DEV),
                                  group_in, group)
    eq, es = oq.requant_transpose(wq, ws, group_in, group)
    assert np.array_equal(tq.cpu().numpy(), eq)
    assert np.array_equal(ts.cpu().numpy(), es)


@pytest.mark.parametrize("group", [32, 128])
def test_quantize_transpose_adversarial_rounding(group):
    """Half-integer quotients and their fp32 neighbours, grouped along R (transposed)."""
    x = _adversarial_rows(np.random.default_rng(7 + group), group).T.copy()  # (2*group, rows)
    codes, scales = kq.quantize_transpose(torch.from_numpy(x).to(DEV), group)
    ec, es = oq.quantize_transpose(x, group)
    assert np.array_equal(codes.cpu().numpy(), ec)
    assert np.array_equal(scales.cpu().numpy().view(np.uint16), es.view(np.uint16))


@pytest.mark.parametrize("group", [32, 128])
def test_requant_transpose_rounding_ties(group):
    """Rows whose input scale is half the group's output scale give half-integer quotients
    (odd codes), the exact ties of the requantization; neighbouring scales give near-ties."""
    rng = np.random.default_rng(31 + group)
    R, C = 2 * group, 64
    S = np.float16(0.0078125)
    codes = rng.integers(-127, 128, (R, C)).astype(np.int8)
    codes[::group, :] = 127  # each column group's amax row: 127 * S, so the new scale is S
    scales = np.empty((R, 1), np.float16)
    scales[:, 0] = np.float16(S / np.float16(2))
    scales[::group, 0] = S
    scales[1::4, 0] = np.nextafter(np.float16(S / np.float16(2)), np.float16(1))
    scales[2::4, 0] = np.nextafter(np.float16(S / np.float16(2)), np.float16(0))
    scales[::group, 0] = S
    tq, ts = kq.requant_transpose(torch.from_numpy(codes).to(DEV), torch.from_numpy(scales).to(DEV),
                                  C, group)
    eq, es = oq.requant_transpose(codes, scales, C, group)
    assert np.array_equal(tq.cpu().numpy(), eq)
    assert np.array_equal(ts.cpu().numpy().view(np.uint16), es.view(np.uint16))


@pytest.mark.parametrize("t_from_codes", [False, True])
@pytest.mark.parametrize("shape,dtype,group", [
    ((256, 384), torch.float32, 128),      # whole tiles (dual kernel)
    ((300, 136), torch.float32, 128),      # ragged rows and columns (dual kernel)
    ((129, 1024), torch.bfloat16, 128),
    ((64, 200), torch.float16, 128),
    ((100, 96), torch.float32, 64),        # other groups: the single-layout kernels
    ((70, 13), torch.float32, 128),        # C % 8 != 0: the single-layout kernels
])
def test_quantize_dual_matches_oracle(shape, dtype, group, t_from_codes):
    """quantize_dual = quantize_last_dim plus quantize_transpose (dY) or plus
    requant_transpose of the row codes (X^T's double quantization), bit-exact."""
    g = torch.Generator().manual_seed(hash((shape, group, t_from_codes)) % 2**31)
    x_cpu = (torch.randn(*shape, generator=g) * 2).to(dtype)
    c, s, ct, st = kq.quantize_dual(x_cpu.to(DEV), group, t_from_codes=t_from_codes)
    xf = x_cpu.float().numpy()
    ec, es = oq.quantize_last_dim(xf, group)
    if t_from_codes:
        ect, est = oq.requant_transpose(ec, es, group, group)
    else:
        ect, est = oq.quantize_transpose(xf, group)
    assert np.array_equal(c.cpu().numpy(), ec)
    assert np.array_equal(s.cpu().numpy().view(np.uint16), es.view(np.uint16))
    assert np.array_equal(ct.cpu().numpy(), ect)
    assert np.array_equal(st.cpu().numpy().view(np.uint16), est.view(np.uint16))


@pytest.mark.parametrize("t_from_codes", [False, True])
def test_quantize_dual_adversarial_rounding(t_from_codes):
    """Quotients on and next to half-integers through both layouts of the dual kernel."""
    x = _adversarial_rows(np.random.default_rng(5), 128)            # (rows, 256)
    x = np.concatenate([x, x[::-1] * np.float32(0.5)], 0)            # more rows, two tiles
    c, s, ct, st = kq.quantize_dual(torch.from_numpy(x).to(DEV), 128, t_from_codes=t_from_codes)
    ec, es = oq.quantize_last_dim(x, 128)
    ect, est = (oq.requant_transpose(ec, es, 128, 128) if t_from_codes
                else oq.quantize_transpose(x, 128))
    assert np.array_equal(c.cpu().numpy(), ec)
    assert np.array_equal(s.cpu().numpy().view(np.uint16), es.view(np.uint16))
    assert np.array_equal(ct.cpu().numpy(), ect)
    assert np.array_equal(st.cpu().numpy().view(np.uint16), est.view(np.uint16))


@pytest.mark.parametrize("shape,dtype", [
    ((256, 384), torch.float32),      # whole tiles
    ((300, 136), torch.float32),      # ragged rows (zeros past R) and columns
    ((8192, 512), torch.float32),     # a Rosa projection's dY at config 4/5
    ((129, 1024), torch.bfloat16),
    ((64, 200), torch.float16),
    ((70, 13), torch.float32),        # C % 8 != 0: quantize_dual + torch's sum
])
def test_quantize_dual_colsum(shape, dtype):
    """The bias-gradient column sums formed in the dual quantization's pass: the codes equal
    quantize_dual's (bit-exact against the oracle), the sums equal the float64 column sums
    of the same values within fp32 summation error (the reference's db is torch's fp32
    g.float().sum(0), another order). Inputs include a NaN-free wide range and exact zeros."""
    g = torch.Generator().manual_seed(hash(shape) % 2**31)
    x_cpu = (torch.randn(*shape, generator=g) * 2).to(dtype)
    x_cpu[:, ::7] = 0
    c, s, ct, st, cs = kq.quantize_dual_colsum(x_cpu.to(DEV))
    xf = x_cpu.float().numpy()
    ec, es = oq.quantize_last_dim(xf, 128)
    ect, est = oq.quantize_transpose(xf, 128)
    assert np.array_equal(c.cpu().numpy(), ec)
    assert np.array_equal(s.cpu().numpy().view(np.uint16), es.view(np.uint16))
    assert np.array_equal(ct.cpu().numpy(), ect)
    assert np.array_equal(st.cpu().numpy().view(np.uint16), est.view(np.uint16))
    want = xf.astype(np.float64).sum(0)
    bound = np.abs(xf).astype(np.float64).sum(0) * shape[0] * 2.0 ** -24 + 1e-30
    err = np.abs(cs.cpu().numpy().astype(np.float64) - want)
    assert (err <= bound).all(), float((err / bound).max())
    assert np.array_equal(cs.cpu().numpy()[::7], np.zeros_like(want[::7], dtype=np.float32))
    # torch's fp32 sum (the reference's db) sits within the same bound of the exact sum
    terr = np.abs(x_cpu.float().sum(0).numpy().astype(np.float64) - cs.cpu().numpy())
    assert (terr <= 2 * bound).all()


@pytest.mark.parametrize("sa,sb,dtype", [
    ((1536, 1536), (8192, 1536), torch.float32),   # config 2's W and X
    ((300, 136), (129, 1024), torch.float32),      # ragged tiles in both
    ((64, 200), (256, 384), torch.bfloat16),
    ((70, 13), (64, 256), torch.float32),          # C % 8 != 0: two launches
])
def test_quantize_dual2_equals_two_duals(sa, sb, dtype):
    """Two X operands in one launch = quantize_dual(t_from_codes=True) of each, bit for bit."""
    g = torch.Generator().manual_seed(hash((sa, sb)) % 2**31)
    a = (torch.randn(*sa, generator=g) * 2).to(dtype).to(DEV)
    b = torch.randn(*sb, generator=g).to(dtype).to(DEV)
    ra, rb = kq.quantize_dual2(a, b)
    for got, x in ((ra, a), (rb, b)):
        want = kq.quantize_dual(x, 128, t_from_codes=True)
        for u, v in zip(got, want):
            assert torch.equal(u.view(torch.int8) if u.dtype == torch.int8 else u.view(torch.int16),
                               v.view(torch.int8) if v.dtype == torch.int8 else v.view(torch.int16))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("R,C", [(256, 1536), (200, 136), (8192, 1536), (33, 24)])
def test_quantize_dual_fp16_rounding_mode(dtype, R, C):
    """round_fp16: both layouts of x.to(float16) from one pass, bit-exact against the oracle
    quantizer of the fp16-rounded values (rows scaled over 16 binades: fp16 subnormals and
    values that round to zero included)."""
    from ksdraft_amd.kernels.quant import quantize_dual
    rng = np.random.default_rng(R + C)
    x = (rng.standard_normal((R, C)) * np.exp(rng.uniform(-12, 4, (R, 1)))).astype(np.float32)
    x[::7, ::5] *= 1e-3
    xd = torch.from_numpy(x).to("cuda").to(dtype)
    c, s, ct, st = quantize_dual(xd, round_fp16=True)
    x16 = xd.float().cpu().numpy().astype(np.float16).astype(np.float32)
    ec, es = oq.quantize_last_dim(x16)
    et, ets = oq.quantize_last_dim(np.ascontiguousarray(x16.T))
    assert np.array_equal(c.cpu().numpy(), ec) and np.array_equal(s.cpu().numpy().view(np.uint16), es.view(np.uint16))
    assert np.array_equal(ct.cpu().numpy(), et) and np.array_equal(st.cpu().numpy().view(np.uint16), ets.view(np.uint16))
