"""CPU restatement of the Rosa mixer step (test infrastructure only).

Follows reference ksdraft/model/rosa.py and ksdraft/kernels/rosa_credit_gpu.py:
  * default_max_match_len              rosa.py:50-55
  * match_payload_sign_loops           rosa.py:40-98, the length loop, numpy (small T)
  * match                              the same decision by brute force over (t, j)
                                       pairs in C (ksd_oracle.c), for large T
  * shifted                            RosaMixer._shifted, rosa.py:128-133
  * hard_rosa_forward / _backward      HardRosaGPU, rosa_credit_gpu.py:54-112
  * credits                            _chunk_credits by its definition (flip one bit,
                                       redo the match, dot with the gradient), C

Pinned by the reference's own known-answer tests (tests/test_rosa.py:25-36 hand case,
:52-57 no-match case), its brute-force _sign (:7-22) restated in tests and compared on
random streams, and the length loop against the pair brute force
(tests/test_oracle_rosa.py).
"""

from __future__ import annotations

import numpy as np

from ._clib import lib, ptr


def default_max_match_len(T: int, max_match_len: int | None = None) -> int:
    """rosa.py:50-55."""
    if max_match_len is None:
        return max(1, min(62, T - 1)) if T > 1 else 0
    return min(max_match_len, T - 1)


def match_payload_sign_loops(q, k, v, max_match_len=None):
    """rosa.py:40-98: rolling exact codes, lengths searched longest first; the latest
    endpoint j in [L-1, t-1] with equal codes decides. (..., T) {0,1} -> (..., T) +-1."""
    q = np.asarray(q, np.int64)
    k = np.asarray(k, np.int64)
    v = np.asarray(v, np.int64)
    *lead, T = q.shape
    L = default_max_match_len(T, max_match_len)
    sign = np.full(q.shape, -1.0, np.float32)
    if L < 1:
        return sign
    codes = []
    qc = np.zeros(q.shape, np.int64)
    kc = np.zeros(q.shape, np.int64)
    for _ in range(L):
        qc = np.concatenate([np.zeros(lead + [1], np.int64), 2 * qc[..., :-1]], -1) + q
        kc = np.concatenate([np.zeros(lead + [1], np.int64), 2 * kc[..., :-1]], -1) + k
        codes.append((qc, kc))
    decided = np.zeros(q.shape, bool)
    idx = np.arange(T)
    for length in range(L, 0, -1):
        qc, kc = codes[length - 1]
        eq = qc[..., :, None] == kc[..., None, :]
        valid = (idx[None, :] >= length - 1) & (idx[None, :] < idx[:, None])
        cand = eq & valid & ~decided[..., :, None]
        take = cand.any(-1) & ~decided
        if take.any():
            latest = np.where(cand, idx, -1).max(-1)
            succ = np.clip(latest, 0, None) + 1
            vs = np.where(np.take_along_axis(v, np.minimum(succ, T - 1), -1) > 0, 1.0, -1.0)
            sign = np.where(take, vs, sign).astype(np.float32)
            decided |= take
        if decided.all():
            break
    return sign


def match(q, k, v, max_match_len=None):
    """Pair brute force (C). q/k/v (streams, T) {0,1}. Returns (sign float32, j int32,
    length int32), each (streams, T); j = -1 and length 0 where nothing matches."""
    q = np.ascontiguousarray(q, np.uint8)
    k = np.ascontiguousarray(k, np.uint8)
    v = np.ascontiguousarray(v, np.uint8)
    S, T = q.shape
    L = default_max_match_len(T, max_match_len)
    sign = np.empty((S, T), np.float32)
    mj = np.empty((S, T), np.int32)
    ml = np.empty((S, T), np.int32)
    if L < 1:
        sign[:] = -1.0
        mj[:] = -1
        ml[:] = 0
        return sign, mj, ml
    lib().ksd_oracle_rosa_match(ptr(q), ptr(k), ptr(v), S, T, L, ptr(sign), ptr(mj), ptr(ml))
    return sign, mj, ml


def credits(q, k, v, grad_sign, max_match_len=None):
    """First-order credits by definition (C): (streams, 3, T) float64."""
    q = np.ascontiguousarray(q, np.uint8)
    k = np.ascontiguousarray(k, np.uint8)
    v = np.ascontiguousarray(v, np.uint8)
    g = np.ascontiguousarray(grad_sign, np.float32)
    S, T = q.shape
    L = default_max_match_len(T, max_match_len)
    out = np.zeros((S, 3, T), np.float64)
    if L >= 1:
        lib().ksd_oracle_rosa_credits(ptr(q), ptr(k), ptr(v), ptr(g), S, T, L, ptr(out))
    return out


def sigmoid32(x):
    return (1.0 / (1.0 + np.exp(-np.asarray(x, np.float64)))).astype(np.float32)


def _bf16_round(a):
    """fp32 -> bf16 (round to nearest even) -> fp32."""
    u = np.asarray(a, np.float32).view(np.uint32).astype(np.uint64)
    u = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return u.astype(np.uint32).view(np.float32)


def shifted(x, sig, dtype="float32"):
    """rosa.py:128-133: prev + (x - prev) * sig, sig = sigmoid(time_mix) as fp32.

    x (B, T, d) holds values of `dtype` ("float32", "bfloat16", "float16"): x - prev is a
    tensor op in that dtype (fp32 then rounded), the rest fp32 (type promotion against the
    fp32 sigmoid)."""
    x = np.asarray(x, np.float32)
    prev = np.concatenate([np.zeros_like(x[:, :1]), x[:, :-1]], 1)
    diff = (x - prev).astype(np.float32)
    if dtype == "bfloat16":
        diff = _bf16_round(diff)
    elif dtype == "float16":
        diff = diff.astype(np.float16).astype(np.float32)
    return (prev + (diff * np.asarray(sig, np.float32)).astype(np.float32)).astype(np.float32)


def shifted_backward(x, sig, grads, dtype="float32"):
    """Backward of the three lerps of rosa.py:128-133, in float64 (the gradient the
    autograd of _shifted computes, without its intermediate roundings).

    x (B, T, d) values of `dtype`; sig (3, d) the fp32 sigmoids of time_mix_q/k/v; grads
    the three dL/d(m_in), (B, T, d). m_in = prev + (x - prev) * s_m, prev = x shifted one
    token (0 at t = 0), x - prev rounded to `dtype` as the forward rounds it. Returns
    (dx (B, T, d) float64, dsig (3, d) float64)."""
    x = np.asarray(x, np.float32)
    prev = np.concatenate([np.zeros_like(x[:, :1]), x[:, :-1]], 1)
    diff = (x - prev).astype(np.float32)
    if dtype == "bfloat16":
        diff = _bf16_round(diff)
    elif dtype == "float16":
        diff = diff.astype(np.float16).astype(np.float32)
    diff = diff.astype(np.float64)
    dx = np.zeros(x.shape, np.float64)
    dsig = np.zeros((3, x.shape[-1]), np.float64)
    for m, g in enumerate(grads):
        g = np.asarray(g, np.float64)
        s = np.asarray(sig[m], np.float64)
        dx += g * s                          # through x - prev, into x[t]
        dx[:, :-1] += (g * (1.0 - s))[:, 1:]  # through prev (+ and - terms), into x[t - 1]
        dsig[m] = (g * diff).sum(axis=(0, 1))
    return dx, dsig


def bits_of(x):
    """(x > 0) as uint8 (rosa.py:156-158, rosa_credit_gpu.py:68-70)."""
    return (np.asarray(x) > 0).astype(np.uint8)


def hard_rosa_forward(q, k, v, payload):
    """HardRosaGPU.forward (rosa_credit_gpu.py:62-75): (B, T, S) -> (B, T, S) fp32 and the
    (B, S, T) sign."""
    q, k, v = (np.asarray(a, np.float32) for a in (q, k, v))
    B, T, S = q.shape
    tb = lambda a: np.ascontiguousarray(bits_of(a).transpose(0, 2, 1)).reshape(B * S, T)  # noqa: E731
    sign, _, _ = match(tb(q), tb(k), tb(v))
    sign = sign.reshape(B, S, T)
    out = (np.asarray(payload, np.float32)[None, :, None] * sign).transpose(0, 2, 1)
    return np.ascontiguousarray(out), sign


def hard_rosa_backward(q, k, v, payload, grad_out):
    """HardRosaGPU.backward (rosa_credit_gpu.py:78-112): exact first-order credits with
    the Bernoulli logit map. Returns (gq, gk, gv (B, T, S) float32, gp (S,) float32)."""
    q, k, v = (np.asarray(a, np.float32) for a in (q, k, v))
    B, T, S = q.shape
    payload = np.asarray(payload, np.float32)
    _, sign = hard_rosa_forward(q, k, v, payload)
    grad_hard = np.asarray(grad_out, np.float32).transpose(0, 2, 1)
    grad_sign = (grad_hard * payload[None, :, None]).astype(np.float32)
    tb = lambda a: np.ascontiguousarray(bits_of(a).transpose(0, 2, 1)).reshape(B * S, T)  # noqa: E731
    qb, kb, vb = tb(q), tb(k), tb(v)
    cr = credits(qb, kb, vb, grad_sign.reshape(B * S, T)).reshape(B, S, 3, T)
    outs = []
    for which, bits, pre in ((0, qb, q), (1, kb, k), (2, vb, v)):
        delta = (cr[:, :, which, :] * (1.0 - 2.0 * bits.reshape(B, S, T))).astype(np.float32)
        s = sigmoid32(pre)
        bern = (s * (np.float32(1.0) - s)).astype(np.float32)
        outs.append((delta.transpose(0, 2, 1) * bern).astype(np.float32))
    gp = (grad_hard.astype(np.float64) * sign).sum(axis=(0, 2)).astype(np.float32)
    return outs[0], outs[1], outs[2], gp
