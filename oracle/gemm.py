"""CPU restatement of the W8A8 GS GEMM (test infrastructure only).

Three views of reference ksdraft/kernels/gemm.py:
  * ``group_partials``  — the exact int32 per-group dot products (gemm.py:42), in C.
  * ``gemm_ordered``    — the ordered per-group fp32 contract the GPU kernel implements
                          (acc = fmaf(P_g, sa*sw, acc), g ascending; gemm.py:34-45), in C;
                          shapes with few output tiles split the groups into contiguous
                          parts summed that way and added in order (``splits_for``).
  * ``gemm_reference``  — the reference's CPU path: dequantize both operands, fp32
                          matmul (gemm.py:76-82), in numpy/BLAS. Outputs of the GPU kernel
                          are held to rtol/atol 1e-3 of this path.

Pinned by tests/test_oracle_gemm.py: partials against numpy int64 matmuls per group;
the ordered contract against exact rational arithmetic (fractions.Fraction) rounded
once per group; gemm_reference against float64 products of the dequantized operands.
"""

from __future__ import annotations

import numpy as np

from . import _clib
from .quant import dequantize_last_dim


def _pad_k(a_codes, w_codes, n_groups, group):
    K = a_codes.shape[1]
    Kp = n_groups * group
    if Kp < K:
        raise ValueError(f"K {K} exceeds the scales' padded length {Kp}")
    if K < Kp:
        a_codes = np.pad(a_codes, ((0, 0), (0, Kp - K)))
        w_codes = np.pad(w_codes, ((0, 0), (0, Kp - K)))
    return np.ascontiguousarray(a_codes, np.int8), np.ascontiguousarray(w_codes, np.int8), Kp


def group_partials(a_codes, w_codes, group: int = 128):
    """(M,K) x (N,K) -> int32 (K/group, M, N)."""
    a = np.ascontiguousarray(a_codes, np.int8)
    w = np.ascontiguousarray(w_codes, np.int8)
    M, K = a.shape
    N = w.shape[0]
    out = np.empty((K // group, M, N), np.int32)
    _clib.lib().ksd_oracle_partials(_clib.ptr(a), _clib.ptr(w), M, N, K, group, _clib.ptr(out))
    return out


def splits_for(M: int, N: int, K: int, group: int = 128) -> int:
    """K parts of the GS128 contract for a shape: 1 when there are at least 192 output
    tiles of 128 x 128, else min(256 // tiles, (K // 128) // 8, 8), at least 1 (groups
    other than 128 are never split). K is the 128-padded reduction length."""
    if group != 128:
        return 1
    tiles = -(-M // 128) * -(-N // 128)
    if tiles <= 0 or tiles >= 192:
        return 1
    return max(1, min(256 // tiles, (K // 128) // 8, 8))


def gemm_ordered(a_codes, a_scales, w_codes, w_scales, group: int = 128, bias=None,
                 rows=None, splits=None):
    """Ordered-group fp32 contract; rows: optional subset of row indices to evaluate.

    splits: K parts (default: splits_for the full shape). Part q sums the groups
    [q*G//S, (q+1)*G//S) from zero in order; the parts are added in ascending order, then
    the bias."""
    a, w, K = _pad_k(np.asarray(a_codes), np.asarray(w_codes), a_scales.shape[-1], group)
    M = a.shape[0]
    N = w.shape[0]
    if splits is None:
        splits = splits_for(M, N, -(-K // 128) * 128, group)
    as_ = np.ascontiguousarray(a_scales, np.float16).view(np.uint16)
    ws_ = np.ascontiguousarray(w_scales, np.float16).view(np.uint16)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    if rows is None:
        r = None
        nr = M
    else:
        r = np.ascontiguousarray(rows, np.int64)
        nr = r.shape[0]
    y = np.empty((nr, N), np.float32)
    _clib.lib().ksd_oracle_gemm_ordered(
        _clib.ptr(a), _clib.ptr(as_), _clib.ptr(w), _clib.ptr(ws_), M, N, K, group,
        _clib.ptr(b), _clib.ptr(r), nr, int(splits), _clib.ptr(y))
    return y


def gemm_reference(a_codes, a_scales, w_codes, w_scales, group: int = 128):
    """gemm.py:76-82: dequantize then fp32 matmul."""
    a, w, K = _pad_k(np.asarray(a_codes), np.asarray(w_codes), a_scales.shape[-1], group)
    ad = dequantize_last_dim(a, a_scales, group)
    wd = dequantize_last_dim(w, w_scales, group)
    return ad @ wd.T
