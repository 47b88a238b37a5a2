"""Pins the Rosa oracle (oracle/rosa.py) — CPU only.

The reference's own known answers (tests/test_rosa.py:25-36, 52-57), its brute-force
_sign (tests/test_rosa.py:7-22, restated below as a test helper) on random streams, the
length-loop restatement against the pair brute force on long structured streams (matches
past the 62-bit cap), and the credits against a second, independent restatement of
_chunk_credits (rosa_credit_gpu.py:28-51) plus the closed form of v-flip credits."""

import numpy as np
import pytest

from oracle import rosa as orr


def _sign_bruteforce(q, k, v):
    """tests/test_rosa.py:7-22: longest suffix, latest endpoint, successor bit."""
    T = len(q)
    out = [-1.0] * T
    for t in range(T):
        for L in range(min(t, T - 1), 0, -1):
            pat = q[t - L + 1: t + 1]
            best = -1
            for j in range(t - 1, L - 2, -1):
                if k[j - L + 1: j + 1] == pat:
                    best = j
                    break
            if best >= 0:
                out[t] = 1.0 if v[best + 1] else -1.0
                break
    return out


def test_hand_case():
    q, k, v = [0, 1, 1, 1], [1, 0, 1, 1], [1, 0, 0, 1]
    exp = [-1.0, -1.0, -1.0, 1.0]
    assert orr.match_payload_sign_loops([q], [k], [v])[0].tolist() == exp
    assert orr.match([q], [k], [v])[0][0].tolist() == exp


def test_no_match():
    q, k, v = [[1, 1, 1]], [[0, 0, 0]], [[1, 1, 1]]
    assert orr.match_payload_sign_loops(q, k, v)[0].tolist() == [-1.0] * 3
    assert orr.match(q, k, v)[0][0].tolist() == [-1.0] * 3


def test_single_position_and_lmax_rule():
    assert orr.default_max_match_len(1) == 0
    assert orr.default_max_match_len(2) == 1
    assert orr.default_max_match_len(2048) == 62
    assert orr.default_max_match_len(100, 5) == 5
    assert orr.match([[1]], [[1]], [[1]])[0].tolist() == [[-1.0]]


def test_vs_reference_bruteforce_random():
    rng = np.random.default_rng(7)
    for _ in range(60):
        T = int(rng.integers(2, 24))
        q, k, v = (rng.integers(0, 2, T).tolist() for _ in range(3))
        exp = _sign_bruteforce(q, k, v)
        assert orr.match_payload_sign_loops([q], [k], [v])[0].tolist() == exp
        assert orr.match([q], [k], [v])[0][0].tolist() == exp


def _structured(rng, S, T):
    rows = [np.zeros(T, np.uint8), np.ones(T, np.uint8), np.arange(T) % 2,
            (np.arange(T) // 3) % 2, (np.arange(T) % 7 == 0)]
    out = [np.asarray(r, np.uint8) for r in rows]
    while len(out) < S:
        p = rng.uniform(0.05, 0.95)
        out.append((rng.uniform(size=T) < p).astype(np.uint8))
    return np.stack(out[:S])


@pytest.mark.parametrize("T", [70, 130])
def test_loops_vs_pair_bruteforce_long_streams(T):
    """Streams longer than the 62-bit cap, including constant and periodic ones whose
    matches exceed the cap (the latest endpoint among capped ties must win)."""
    rng = np.random.default_rng(T)
    q = _structured(rng, 8, T)
    k = np.concatenate([q[:4], _structured(rng, 4, T)])
    v = _structured(rng, 8, T)[::-1].copy()
    exp = orr.match_payload_sign_loops(q, k, v)
    got, mj, ml = orr.match(q, k, v)
    assert np.array_equal(got, exp)
    assert (ml <= 62).all() and (ml[:, 63:] == 62).any()
    # the endpoint's successor bit is the sign
    has = mj >= 0
    succ = np.take_along_axis(v, np.where(has, mj + 1, 0), 1)
    assert np.array_equal(np.where(has, np.where(succ > 0, 1.0, -1.0), -1.0), got)


def test_explicit_max_match_len():
    rng = np.random.default_rng(3)
    q, k, v = (rng.integers(0, 2, (6, 40)) for _ in range(3))
    for L in (1, 3, 8):
        assert np.array_equal(orr.match(q, k, v, L)[0], orr.match_payload_sign_loops(q, k, v, L))


def _credits_by_loops(q, k, v, g):
    """A second restatement of _chunk_credits (rosa_credit_gpu.py:28-51): every single-bit
    perturbation matched at once through the length loop."""
    S, T = q.shape
    base = orr.match_payload_sign_loops(q, k, v)
    out = np.zeros((S, 3, T))
    for s in range(S):
        pert = np.broadcast_to(np.stack([q[s], k[s], v[s]]), (3 * T, 3, T)).copy()
        for n in range(3 * T):
            pert[n, n // T, n % T] ^= 1
        sp = orr.match_payload_sign_loops(pert[:, 0], pert[:, 1], pert[:, 2])
        out[s] = ((sp - base[s]) * g[s]).sum(-1).reshape(3, T)
    return out


def test_credits_two_restatements_agree():
    rng = np.random.default_rng(11)
    S, T = 4, 18
    q, k, v = (rng.integers(0, 2, (S, T)).astype(np.uint8) for _ in range(3))
    g = rng.standard_normal((S, T)).astype(np.float32)
    np.testing.assert_allclose(orr.credits(q, k, v, g), _credits_by_loops(q, k, v, g),
                               rtol=1e-6, atol=1e-6)


def test_v_credits_closed_form():
    """Flipping v[p] only changes the sign at the t whose endpoint is p - 1, by -2*sign."""
    rng = np.random.default_rng(5)
    S, T = 5, 90
    q, k, v = (rng.integers(0, 2, (S, T)).astype(np.uint8) for _ in range(3))
    g = rng.standard_normal((S, T)).astype(np.float32)
    sign, mj, _ = orr.match(q, k, v)
    exp = np.zeros((S, T))
    for s in range(S):
        for t in range(T):
            if mj[s, t] >= 0:
                exp[s, mj[s, t] + 1] += -2.0 * sign[s, t] * g[s, t]
    np.testing.assert_allclose(orr.credits(q, k, v, g)[:, 2], exp, rtol=1e-9, atol=1e-9)
