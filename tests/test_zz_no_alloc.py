"""The no-allocation KS3 spine entry point (ksd_ks3_spine_fwd_noalloc) against the
allocating one (ksd_ks3_spine_fwd, which takes the table workspace from its caller).

Both are called through the C ABI with the same inputs and caller-owned outputs. The
features and their int8 codes and fp16 scales must be bit-identical, and bit-exact against
the oracle; two calls in a row, the second with fewer rows and charts, check that the
library's table array keeps no state between calls that matters."""

import ctypes

import numpy as np
import pytest
import torch

from ksdraft_amd import _lib
from oracle import ks3 as ok
from oracle import quant as oq

DEV = "cuda"


def _inputs(seed, M, Fn):
    rng = np.random.default_rng(seed)
    coeffs = (rng.standard_normal((Fn, 6)) * 0.3).astype(np.float32)
    sq, ss = oq.quantize_last_dim(coeffs)
    ss = ss.reshape(-1)
    sc = ok.h((0.5 + np.abs(rng.standard_normal(Fn))).astype(np.float32))
    sh = ok.h((rng.standard_normal(Fn) * 0.3).astype(np.float32))
    coords = ok.h((rng.standard_normal((M, Fn)) * 2.5).astype(np.float32))
    return coords, sq, ss, sc, sh


def _run(name, coords, sq, ss, sc, sh, group):
    M, Fn = coords.shape
    g = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)  # noqa: E731
    c16 = g(coords.astype(np.float16))
    lut = g(ok.make_tanh_lut())
    ins = [g(sq), g(ss.astype(np.float16)), g(sc.astype(np.float16)), g(sh.astype(np.float16))]
    h = torch.empty((M, Fn), dtype=torch.float32, device=DEV)
    hq = torch.empty((M, Fn), dtype=torch.int8, device=DEV)
    hs = torch.empty((M, -(-Fn // group)), dtype=torch.float16, device=DEV)
    args = [c16.data_ptr(), M, Fn] + [t.data_ptr() for t in ins] + [lut.data_ptr(), group,
                                                                     h.data_ptr(), hq.data_ptr(),
                                                                     hs.data_ptr()]
    if name == "ksd_ks3_spine_fwd":
        table = torch.empty((Fn, 256), dtype=torch.float16, device=DEV)
        args.append(table.data_ptr())
    args.append(torch.cuda.current_stream().cuda_stream)
    _lib.call(name, *args)
    torch.cuda.synchronize()
    return h.cpu().numpy(), hq.cpu().numpy(), hs.cpu().numpy()


@pytest.mark.gpu
@pytest.mark.parametrize("group", [128, 32])
def test_noalloc_spine_matches_allocating_entry_point(group):
    torch.cuda.set_device(0)
    for seed, M, Fn in ((1, 512, 5888), (2, 70, 300)):   # the second call is smaller
        ins = _inputs(seed + group, M, Fn)
        a = _run("ksd_ks3_spine_fwd", *ins, group)
        b = _run("ksd_ks3_spine_fwd_noalloc", *ins, group)
        for x, y in zip(a, b):
            assert np.array_equal(x.view(np.uint8), y.view(np.uint8))
        coords, sq, ss, sc, sh = ins
        feat = ok.spine_features_int8(coords, sq, ss, sc, sh, ok.make_tanh_lut())
        assert np.array_equal(b[0].view(np.uint32), feat.view(np.uint32))
        eq, es = oq.quantize_last_dim(feat, group)
        assert np.array_equal(b[1], eq) and np.array_equal(b[2].view(np.uint16), es.view(np.uint16))


@pytest.mark.gpu
def test_noalloc_spine_rejects_more_charts_than_its_table():
    with pytest.raises(ValueError, match="scratch table"):
        _lib.call("ksd_ks3_spine_fwd_noalloc", 0, 16, 8193, 0, 0, 0, 0, 0, 128, 0, 0, 0,
                  torch.cuda.current_stream().cuda_stream)
