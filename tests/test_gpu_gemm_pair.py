"""GPU parity: two GEMMs in one persistent launch (ksd_w8a8_gemm_pair).

Each problem of a paired launch keeps the numeric contract of its own launch (the ordered
per-group fmaf contract, and its K split when the shape splits), so both outputs must be
bit-identical to two separate w8a8_gemm_out calls, which the GEMM tests pin to the oracle.
The outputs are pre-filled with NaN and called through the C ABI, so a tile that the
balanced work split skipped, or stored twice from the wrong problem, cannot pass. One case
is also checked against the oracle directly.
"""

import numpy as np
import pytest
import torch

from ksdraft_amd import _lib
from ksdraft_amd.kernels import gemm as kg
from ksdraft_amd.kernels import quant as kq
from oracle import gemm as og
from oracle import quant as oq

pytestmark = pytest.mark.gpu
DEV = "cuda"
_CODE = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16, torch.float16: _lib.F16}


def _problem(seed, M, K, N, wscale=0.1):
    g = torch.Generator().manual_seed(seed)
    a = torch.randn(M, K, generator=g).to(DEV)
    w = (torch.randn(N, K, generator=g) * wscale).to(DEV)
    aq, as_ = kq.quantize_last_dim(a)
    wq, ws = kq.quantize_last_dim(w)
    return aq, as_, wq, ws


def _pair_abi(p0, p1):
    """Call the C ABI directly with NaN-filled outputs and an exactly sized workspace."""
    outs, args, need = [], [], 0
    for (aq, as_, wq, ws, dt) in (p0, p1):
        M, K = aq.shape
        N = wq.shape[0]
        y = torch.full((M, N), float("nan"), dtype=dt, device=DEV)
        outs.append(y)
        args += [aq.data_ptr(), as_.data_ptr(), wq.data_ptr(), ws.data_ptr(), M, N, K, y.data_ptr(),
                 _CODE[dt]]
        s = kg.gemm_splits(M, N, K)
        if s > 1:
            need += s * M * N
    work = torch.full((max(need, 4),), float("nan"), device=DEV)
    _lib.call("ksd_w8a8_gemm_pair", *args, work.data_ptr(), need * 4, _lib.stream_ptr(torch.device(DEV)))
    torch.cuda.synchronize()
    return outs


def _bits(t):
    return t.view(torch.int32 if t.dtype == torch.float32 else torch.int16)


CASES = [
    # config 2's backward: dX (8192 x 1536, K 1536) beside dW (1536 x 1536, K 8192)
    ("c2_dx_dw", (8192, 1536, 1536, torch.float32), (1536, 8192, 1536, torch.float32)),
    # the Rosa projection's backward: dX (K 512) beside a split dW (512 x 1536, K 8192)
    ("rosa_dx_dw_split", (8192, 512, 1536, torch.bfloat16), (512, 8192, 1536, torch.float32)),
    # the KS3 backward's value GEMM (fp16 out) beside dup (K = tokens)
    ("ks3_value_dup", (2048, 1536, 5888, torch.float16), (1536, 2048, 5888, torch.float32)),
    # ragged shapes, fewer tiles than CUs
    ("ragged_small", (300, 384, 200, torch.float32), (130, 1024, 70, torch.bfloat16)),
    # both problems split K
    ("both_split", (256, 4096, 384, torch.float32), (384, 8192, 256, torch.float16)),
    # equal unit lengths
    ("same_cost", (1024, 640, 512, torch.float32), (512, 640, 1024, torch.float32)),
]


@pytest.mark.parametrize("name,s0,s1", CASES, ids=[c[0] for c in CASES])
def test_pair_bit_identical_to_two_launches(name, s0, s1):
    probs = []
    for i, (M, K, N, dt) in enumerate((s0, s1)):
        aq, as_, wq, ws = _problem(11 + i, M, K, N)
        probs.append((aq, as_, wq, ws, dt))
    print(f"pair case {name}: {s0[:3]} + {s1[:3]}", flush=True)
    got = _pair_abi(*probs)
    for (aq, as_, wq, ws, dt), y in zip(probs, got):
        ref = kg.w8a8_gemm_out(aq, as_, wq, ws, out_dtype=dt)
        assert torch.equal(_bits(y), _bits(ref)), name
    # the Python wrapper returns the same
    w0, w1 = kg.w8a8_gemm_pair(probs[0], probs[1])
    assert torch.equal(_bits(w0), _bits(got[0])) and torch.equal(_bits(w1), _bits(got[1]))


def test_pair_against_oracle():
    g = torch.Generator().manual_seed(5)
    a0 = torch.randn(320, 512, generator=g)
    w0 = torch.randn(96, 512, generator=g) * 0.05
    a1 = torch.randn(96, 2048, generator=g)
    w1 = torch.randn(200, 2048, generator=g) * 0.05
    ops = []
    for a, w in ((a0, w0), (a1, w1)):
        aq, as_ = oq.quantize_last_dim(a.numpy())
        wq, ws = oq.quantize_last_dim(w.numpy())
        ops.append((aq, as_, wq, ws))
    dev = [tuple(torch.from_numpy(np.ascontiguousarray(x)).to(DEV) for x in o) for o in ops]
    y0, y1 = _pair_abi(dev[0] + (torch.float32,), dev[1] + (torch.float32,))
    for y, (aq, as_, wq, ws) in zip((y0, y1), ops):
        M, K = aq.shape
        N = wq.shape[0]
        s = og.splits_for(M, N, K)
        want = og.gemm_ordered(aq, as_, wq, ws, splits=s)
        assert np.array_equal(y.cpu().numpy().view(np.uint32), want.view(np.uint32))


def test_pair_one_empty_problem():
    aq, as_, wq, ws = _problem(3, 64, 256, 96)
    e = torch.empty(0, 256, dtype=torch.int8, device=DEV)
    es = torch.empty(0, 2, dtype=torch.float16, device=DEV)
    y0, y1 = kg.w8a8_gemm_pair((aq, as_, wq, ws, torch.float32), (e, es, wq, ws, torch.float32))
    assert y1.shape == (0, 96)
    assert torch.equal(_bits(y0), _bits(kg.w8a8_gemm_out(aq, as_, wq, ws)))
