"""GPU parity: the Rosa mixer step kernels against the oracle (oracle/rosa.py).

Bars: packed bits, match signs and endpoints bit-exact (pair brute force in C), including
T = 2048 and streams whose matches pass the 62-bit cap; the fused time shift + quantize
bit-exact against quantize_last_dim of the oracle's shift (same fp32 sigmoid values); the
credits' flip decisions exact and their fp32 sums within 1e-5 relative (the reference's
own sum order is torch's), the projection gradients after the Bernoulli map likewise.
"""

import numpy as np
import pytest
import torch

from ksdraft_amd.kernels import rosa as R
from ksdraft_amd.kernels.rosa_credit_gpu import HardRosaGPU
from ksdraft_amd.model.rosa import RosaMixer, _match_payload_sign
from oracle import quant as oq
from oracle import rosa as orr

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _g(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _streams(rng, n, T):
    """Random streams of varied density plus constant / periodic ones (long matches)."""
    rows = [np.zeros(T), np.ones(T), np.arange(T) % 2, (np.arange(T) // 5) % 2]
    while len(rows) < n:
        rows.append(rng.uniform(size=T) < rng.uniform(0.1, 0.9))
    return np.stack(rows[:n]).astype(np.uint8)


def _bits_to_proj(bits, rng):
    """(n, T) bits -> signed projection values whose (x > 0) bits are `bits`."""
    mag = rng.uniform(0.1, 2.0, bits.shape).astype(np.float32)
    return np.where(bits > 0, mag, -mag).astype(np.float32)


@pytest.mark.parametrize("T", [2, 5, 33, 63, 64, 100, 300])
def test_match_vs_pair_bruteforce(T):
    rng = np.random.default_rng(T)
    n = 24
    q = _streams(rng, n, T)
    k = np.concatenate([q[:6], _streams(rng, n - 6, T)])
    v = _streams(rng, n, T)[::-1].copy()
    proj = [_bits_to_proj(b, rng).T[None] for b in (q, k, v)]  # (1, T, n)
    packed = [R.pack_bits(_g(p)) for p in proj]
    sign, mj = R.match_packed(*(p.reshape(n, -1) for p in packed), T, want_j=True)
    es, ej, _ = orr.match(q, k, v)
    assert np.array_equal(sign.cpu().numpy().astype(np.float32), es)
    assert np.array_equal(mj.cpu().numpy(), ej)


@pytest.mark.parametrize("lmax", [1, 2, 3, 5, 7, 63])
@pytest.mark.parametrize("T", [100, 300])
def test_match_explicit_max_match_len(T, lmax):
    """Caps below and above the default (every residue of the walk's four-length steps and
    its two/one-length tail, and the 63-bit maximum) against the pair brute force."""
    rng = np.random.default_rng(T * 64 + lmax)
    n = 16
    q = _streams(rng, n, T)
    k = np.concatenate([q[:6], _streams(rng, n - 6, T)])
    v = _streams(rng, n, T)
    proj = [_bits_to_proj(b, rng).T[None] for b in (q, k, v)]
    packed = [R.pack_bits(_g(p)) for p in proj]
    sign, mj = R.match_packed(*(p.reshape(n, -1) for p in packed), T, max_match_len=lmax,
                              want_j=True)
    es, ej, el = orr.match(q, k, v, max_match_len=lmax)
    assert el.max() == min(lmax, T - 1)
    assert np.array_equal(sign.cpu().numpy().astype(np.float32), es)
    assert np.array_equal(mj.cpu().numpy(), ej)


def test_match_t2048_sampled_streams():
    rng = np.random.default_rng(2048)
    n, T = 12, 2048
    q = _streams(rng, n, T)
    k = np.concatenate([q[:4], _streams(rng, n - 4, T)])
    v = _streams(rng, n, T)
    proj = [_bits_to_proj(b, rng).T[None] for b in (q, k, v)]
    packed = [R.pack_bits(_g(p)) for p in proj]
    sign, mj = R.match_packed(*(p.reshape(n, -1) for p in packed), T, want_j=True)
    es, ej, el = orr.match(q, k, v)
    assert (el == 62).any()
    assert np.array_equal(sign.cpu().numpy().astype(np.float32), es)
    assert np.array_equal(mj.cpu().numpy(), ej)


def test_pack_bits_dtypes():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((2, 70, 37)).astype(np.float32)
    x[0, 3, 4] = 0.0
    x[1, 5, 6] = -0.0
    for dt in (torch.float32, torch.bfloat16, torch.float16):
        xt = _g(x).to(dt)
        words = R.pack_bits(xt).cpu().numpy().view(np.uint32)
        bits = orr.bits_of(xt.float().cpu().numpy()).transpose(0, 2, 1)  # (B, S, T)
        for t in range(70):
            got = (words[..., t // 32] >> (t % 32)) & 1
            assert np.array_equal(got, bits[..., t]), (dt, t)


@pytest.mark.parametrize("shape", [(2, 70, 37), (1, 2048, 512), (3, 64, 64), (1, 5, 3)])
def test_pack_bits3_equals_three_packs(shape):
    """One launch for q, k and v gives each projection's pack_bits words."""
    rng = np.random.default_rng(sum(shape))
    xs = [_g(rng.standard_normal(shape).astype(np.float32)) for _ in range(3)]
    got = R.pack_bits3(*xs)
    for g, x in zip(got, xs):
        assert torch.equal(g, R.pack_bits(x))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("B,S,T", [(2, 37, 70), (1, 512, 2048), (3, 64, 64), (1, 3, 5), (2, 130, 66)])
def test_hard_out_matches_payload_times_sign(B, S, T, dtype):
    """hard_out = (payload[s] * sign[b, s, t]) transposed to (B, T, S) in the output dtype
    (rosa_credit_gpu.py:75), including tiles cut by S and T (whole-word and byte loads,
    vector and scalar stores)."""
    rng = np.random.default_rng(B * 1000 + S + T)
    sign = np.where(rng.random((B, S, T)) < 0.5, -1, 1).astype(np.int8)
    pay = rng.standard_normal(S).astype(np.float32)
    out = R.hard_out(_g(sign), _g(pay), dtype)
    want = torch.from_numpy((pay[None, :, None] * sign.astype(np.float32)).transpose(0, 2, 1).copy()).to(dtype)
    assert out.shape == (B, T, S)
    assert torch.equal(out.cpu(), want)


def test_match_payload_sign_api_kats():
    q, k, v = [[0, 1, 1, 1]], [[1, 0, 1, 1]], [[1, 0, 0, 1]]
    got = _match_payload_sign(_g(np.array(q, np.int8)), _g(np.array(k, np.int8)),
                              _g(np.array(v, np.int8)))
    assert got.cpu().tolist() == [[-1.0, -1.0, -1.0, 1.0]]
    got = _match_payload_sign(*(_g(np.array(a, np.int8)) for a in ([[1, 1, 1]], [[0, 0, 0]], [[1, 1, 1]])))
    assert got.cpu().tolist() == [[-1.0, -1.0, -1.0]]
    rng = np.random.default_rng(4)
    q, k, v = (rng.integers(0, 2, (3, 5, 40)).astype(np.int8) for _ in range(3))
    got = _match_payload_sign(_g(q), _g(k), _g(v), max_match_len=6).cpu().numpy()
    assert np.array_equal(got, orr.match_payload_sign_loops(q, k, v, 6))


@pytest.mark.parametrize("dtype", ["float32", "bfloat16", "float16"])
@pytest.mark.parametrize("B,T,d,group", [(2, 33, 320, 128), (1, 17, 301, 128), (3, 5, 1536, 64),
                                         (2, 9, 72, 32), (1, 1, 8, 128)])
def test_shift_quantize(dtype, B, T, d, group):
    rng = np.random.default_rng(9 + d)
    x = rng.standard_normal((B, T, d)).astype(np.float32) * 2
    tdt = getattr(torch, dtype)
    xt = _g(x).to(tdt)
    mixes = [_g(rng.standard_normal(d).astype(np.float32)) for _ in range(3)]
    sigs = [torch.sigmoid(m) for m in mixes]
    out = R.shift_quantize(xt, *sigs, group=group)
    xv = xt.float().cpu().numpy()
    for (codes, scales), sg in zip(out, sigs):
        lerp = orr.shifted(xv, sg.cpu().numpy(), dtype).reshape(B * T, d)
        ec, es = oq.quantize_last_dim(lerp, group)
        assert np.array_equal(codes.cpu().numpy(), ec)
        assert np.array_equal(scales.cpu().numpy(), es)


@pytest.mark.parametrize("group", [32, 128])
def test_shift_quantize_adversarial_rounding(group):
    """Quotients on and next to half-integers (the codes' rounding ties) through the fused
    shift: with T = 1 the previous token is zero, so q_in = x * sigmoid, and sigmoid values
    1 and 0.5 keep every quotient of the quantize-time rows exactly where it was."""
    from tests.test_oracle_quant import _adversarial_rows
    x = _adversarial_rows(np.random.default_rng(7 + group), group)
    n, d = x.shape
    sigs = [torch.full((d,), v, dtype=torch.float32, device=DEV) for v in (1.0, 0.5, 1.0)]
    out = R.shift_quantize(_g(x.reshape(n, 1, d)), *sigs, group=group)
    for (codes, scales), sg in zip(out, sigs):
        lerp = orr.shifted(x.reshape(n, 1, d), sg.cpu().numpy(), "float32").reshape(n, d)
        ec, es = oq.quantize_last_dim(lerp, group)
        assert np.array_equal(codes.cpu().numpy(), ec)
        assert np.array_equal(scales.cpu().numpy().view(np.uint16), es.view(np.uint16))


def _hard_case(seed, B, T, S):
    rng = np.random.default_rng(seed)
    q, k, v = (rng.standard_normal((B, T, S)).astype(np.float32) * 2 for _ in range(3))
    # a few streams with long matches: constant and copied patterns
    q[:, :, 0] = 1.0
    k[:, :, 0] = 1.0
    k[:, :, 1] = q[:, :, 1]
    payload = (np.abs(rng.standard_normal(S)) + 0.5).astype(np.float32)
    g = rng.standard_normal((B, T, S)).astype(np.float32)
    return q, k, v, payload, g


@pytest.mark.parametrize("B,T,S", [(2, 16, 8), (1, 63, 6), (2, 70, 5), (1, 150, 4)])
def test_hard_rosa_forward_backward(B, T, S):
    q, k, v, payload, g = _hard_case(T, B, T, S)
    tq, tk, tv, tp = (_g(a).requires_grad_(True) for a in (q, k, v, payload))
    y = HardRosaGPU.apply(tq, tk, tv, tp)
    y.backward(_g(g))
    ey, _ = orr.hard_rosa_forward(q, k, v, payload)
    assert torch.equal(y.detach().cpu(), torch.from_numpy(ey))
    egq, egk, egv, egp = orr.hard_rosa_backward(q, k, v, payload, g)
    for got, exp in ((tq.grad, egq), (tk.grad, egk), (tv.grad, egv), (tp.grad, egp)):
        got = got.cpu().numpy()
        scale = np.abs(exp).max() + 1e-30
        np.testing.assert_allclose(got, exp, rtol=1e-5, atol=1e-5 * scale)
        assert np.array_equal(got == 0, exp == 0)  # the same flips change the sign


def test_credits_t2048_sampled_flips():
    """At T = 2048 the oracle checks sampled flips by re-matching each flipped stream."""
    rng = np.random.default_rng(77)
    B, T, S = 1, 2048, 3
    q, k, v, payload, g = _hard_case(77, B, T, S)
    tq, tk, tv = (_g(a).requires_grad_(True) for a in (q, k, v))
    y = HardRosaGPU.apply(tq, tk, tv, _g(payload))
    y.backward(_g(g))
    bits = [orr.bits_of(a[0].T) for a in (q, k, v)]  # (S, T)
    base, _, _ = orr.match(*bits)
    gsign = (g[0].T * payload[:, None]).astype(np.float64)
    for which, grad in ((0, tq.grad), (1, tk.grad), (2, tv.grad)):
        pre = (q, k, v)[which][0].T
        sig = orr.sigmoid32(pre)
        bern = (sig * (np.float32(1) - sig)).astype(np.float32)
        gg = grad[0].T.cpu().numpy()  # (S, T)
        for s in range(S):
            for p in rng.choice(T, 12, replace=False):
                fl = [b[s:s + 1].copy() for b in bits]
                fl[which][0, p] ^= 1
                sp, _, _ = orr.match(*fl)
                cred = float(((sp[0] - base[s]) * gsign[s]).sum())
                exp = np.float32(cred * (1.0 - 2.0 * bits[which][s, p])) * bern[s, p]
                assert abs(gg[s, p] - exp) <= 1e-5 * max(1.0, abs(exp)), (which, s, p, gg[s, p], exp)


def test_rosa_mixer_eval_and_training():
    torch.manual_seed(0)
    m = RosaMixer(64, 16).to(DEV)
    with torch.no_grad():
        m.out_proj.weight.normal_(0, 0.05)
    x = torch.randn(2, 24, 64, device=DEV)
    m.eval()
    y = m(x)
    q_in, k_in, v_in = m._shifted(x)
    with torch.no_grad():
        bits = [orr.bits_of(p(i).cpu().numpy()).transpose(0, 2, 1).reshape(-1, 24)
                for p, i in ((m.q_proj, q_in), (m.k_proj, k_in), (m.v_proj, v_in))]
    sign, _, _ = orr.match(*bits)
    hard = (m.payload.detach().cpu().numpy()[None, :, None] * sign.reshape(2, 16, 24)).transpose(0, 2, 1)
    exp = m.out_proj(torch.from_numpy(np.ascontiguousarray(hard)).to(DEV))
    torch.testing.assert_close(y, exp, rtol=1e-5, atol=1e-6)
    y.square().mean().backward()
    assert m.payload.grad is not None and m.q_proj.weight.grad is None
    m.zero_grad()
    m.train()
    m(x).square().mean().backward()
    for name in ("payload", "q_proj.weight", "k_proj.weight", "v_proj.weight", "time_mix_q"):
        p = dict(m.named_parameters())[name]
        assert p.grad is not None and torch.isfinite(p.grad).all(), name


def _credits_direct(q, k, v, gsign, lmax=None):
    """ksd_rosa_credits on (n, T) bit streams, grad_sign (n, T): credits (n, 3, T)."""
    from ksdraft_amd import _lib
    n, T = q.shape
    rng = np.random.default_rng(T)
    proj = [_bits_to_proj(b, rng).T[None] for b in (q, k, v)]  # (1, T, n)
    packed = [R.pack_bits(_g(p)).reshape(n, -1).contiguous() for p in proj]
    lmax = orr.default_max_match_len(T, lmax)
    _, mj = R.match_packed(*packed, T, max_match_len=lmax, want_j=True)
    grad = _g(np.ascontiguousarray(gsign.T[None]))  # (1, T, n), payload 1
    pay = torch.ones(n, device=DEV)
    cred = torch.full((n, 3, T), float("nan"), device=DEV)  # every entry is written
    part = torch.empty((n,), device=DEV)
    sums = torch.empty((n, 3, T), dtype=torch.int64, device=DEV)
    _lib.call("ksd_rosa_credits", packed[0].data_ptr(), packed[1].data_ptr(), packed[2].data_ptr(),
              mj.contiguous().data_ptr(), grad.data_ptr(), pay.data_ptr(), 1, T, n, lmax,
              cred.data_ptr(), part.data_ptr(), _lib.ptr(sums), _lib.stream_ptr(torch.device(DEV)))
    return cred.cpu().numpy()


# The balanced credits kernel has two paths per position (bit-parallel, per-candidate),
# chosen from each stream's statistics and the position; KSD_ROSA_CREDITS_PATH forces one.
PATHS = ["bits", "scan", "auto"]


def _set_path(monkeypatch, path):
    if path == "auto":
        monkeypatch.delenv("KSD_ROSA_CREDITS_PATH", raising=False)
    else:
        monkeypatch.setenv("KSD_ROSA_CREDITS_PATH", path)


@pytest.mark.parametrize("path", PATHS)
@pytest.mark.parametrize("T", [256, 300])
def test_credits_structured_streams_bruteforce(T, path, monkeypatch):
    """Constant, periodic and varied-density streams (deep chains, buckets resolved by every
    checkpoint and by their own chain) against the definition, every flip, on each path."""
    _set_path(monkeypatch, path)
    rng = np.random.default_rng(1000 + T)
    n = 16
    q = _streams(rng, n, T)
    k = np.concatenate([q[:5], _streams(rng, n - 5, T)])
    k[5] = np.roll(q[5], 3)
    v = _streams(rng, n, T)[::-1].copy()
    gsign = rng.standard_normal((n, T)).astype(np.float32)
    gsign[:, ::7] = 0.0  # positions whose gradient is zero contribute nothing
    got = _credits_direct(q, k, v, gsign)
    exp = orr.credits(q, k, v, gsign)
    scale = np.abs(exp).max() + 1e-30
    np.testing.assert_allclose(got, exp, rtol=1e-5, atol=1e-5 * scale)
    assert np.array_equal(got == 0, exp == 0)


@pytest.mark.parametrize("path", ["bits", "scan"])
@pytest.mark.parametrize("lmax", [2, 3, 5, 7])
def test_credits_explicit_max_match_len_bruteforce(lmax, path, monkeypatch):
    """Short caps: every flip's re-match under the same cap (the definition) at T = 200."""
    _set_path(monkeypatch, path)
    T, n = 200, 12
    rng = np.random.default_rng(500 + lmax)
    q = _streams(rng, n, T)
    k = np.concatenate([q[:4], _streams(rng, n - 4, T)])
    v = _streams(rng, n, T)
    gsign = rng.standard_normal((n, T)).astype(np.float32)
    got = _credits_direct(q, k, v, gsign, lmax)
    exp = orr.credits(q, k, v, gsign, max_match_len=lmax)
    scale = np.abs(exp).max() + 1e-30
    np.testing.assert_allclose(got, exp, rtol=1e-5, atol=1e-5 * scale)
    assert np.array_equal(got == 0, exp == 0)


def test_credits_paths_agree_bitwise(monkeypatch):
    """T = 2048 streams of every kind (random, long runs, constant, periodic, copies of q): the
    bit-parallel path alone, the per-candidate path alone and the automatic choice (which
    takes each path on some streams and positions here) give the same bits, exact sums of
    the same contributions; sampled flips match the definition."""
    rng = np.random.default_rng(2048)
    n, T = 24, 2048
    q = _streams(rng, n, T)
    runs = [np.cumsum(rng.uniform(size=T) < pr) % 2 for pr in (0.02, 0.05, 0.1, 0.2)]
    q[12:16] = np.stack(runs).astype(np.uint8)
    k = np.concatenate([q[:6], _streams(rng, n - 6, T)])
    k[12:16] = np.stack([np.cumsum(rng.uniform(size=T) < pr) % 2 for pr in (0.02, 0.05, 0.1, 0.2)])
    k[8] = np.roll(q[8], 5)
    v = _streams(rng, n, T)
    gsign = rng.standard_normal((n, T)).astype(np.float32)
    out = {}
    for path in PATHS:
        _set_path(monkeypatch, path)
        out[path] = _credits_direct(q, k, v, gsign)
    assert np.array_equal(out["bits"].view(np.uint32), out["scan"].view(np.uint32))
    assert np.array_equal(out["bits"].view(np.uint32), out["auto"].view(np.uint32))
    base, _, _ = orr.match(q, k, v)
    g64 = gsign.astype(np.float64)
    for s in (0, 3, 8, 12, 14, 20):
        for which in range(3):
            for p in rng.choice(T, 6, replace=False):
                fl = [b[s:s + 1].copy() for b in (q, k, v)]
                fl[which][0, p] ^= 1
                sp, _, _ = orr.match(*fl)
                exp = float(((sp[0] - base[s]) * g64[s]).sum())
                got = float(out["auto"][s, which, p])
                assert abs(got - exp) <= 1e-5 * max(1.0, abs(exp)), (s, which, p, got, exp)


def test_credits_are_deterministic():
    """Every credit is an exact fixed-point sum, formed by waves that take (stream, chunk)
    items in whatever order they finish: two runs give the same bits (structured streams
    with deep chains, many contributions per entry), and the values match the definition on
    sampled flips."""
    rng = np.random.default_rng(4242)
    n, T = 24, 2048
    q = _streams(rng, n, T)
    k = np.concatenate([q[:8], _streams(rng, n - 8, T)])
    k[8] = np.roll(q[8], 5)
    v = _streams(rng, n, T)
    gsign = (rng.standard_normal((n, T)) * np.exp(rng.uniform(-8, 8, (n, T)))).astype(np.float32)
    a = _credits_direct(q, k, v, gsign)
    b = _credits_direct(q, k, v, gsign)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    base, _, _ = orr.match(q, k, v)
    for s in range(0, n, 5):
        for which in range(3):
            for p in rng.choice(T, 3, replace=False):
                fl = [x[s:s + 1].copy() for x in (q, k, v)]
                fl[which][0, p] ^= 1
                sp, _, _ = orr.match(*fl)
                exp = float(((sp[0] - base[s]) * gsign[s].astype(np.float64)).sum())
                assert abs(a[s, which, p] - exp) <= 1e-5 * max(abs(exp), np.abs(gsign[s]).max()), (s, which, p)


def _dense_entry(q, k, v, g, s, which, p, base):
    """Credit (which, p) of stream s by definition: the re-match after the flip, then the
    dense float64 sum of delta * g over every t (IEEE: 0 * inf and NaN give NaN)."""
    fl = [x[s:s + 1].copy() for x in (q, k, v)]
    fl[which][0, p] ^= 1
    sp, _, _ = orr.match(*fl)
    with np.errstate(invalid="ignore"):
        return float(((sp[0] - base[s]).astype(np.float64) * g[s].astype(np.float64)).sum())


@pytest.mark.parametrize("T,path", [(300, "bits"), (300, "scan"), (2100, "auto")])
def test_credits_nonfinite_gradient_follows_the_dense_sum(T, path, monkeypatch):
    """Streams whose gradient holds inf or NaN: the reference sums delta * g over every t
    (rosa_credit_gpu.py:48), so 0 * inf and NaN make an entry NaN unless every infinite
    position flips it, which then holds +-inf (NaN if the infinite terms have both signs).
    T = 300 against the definition on every entry (on both paths of the balanced kernel),
    T = 2100 (the candidate-per-lane kernel) on sampled entries and on every entry the
    infinite positions flip. The finite streams of the call stay exact."""
    _set_path(monkeypatch, path)
    rng = np.random.default_rng(77 + T)
    n = 7
    q = _streams(rng, n, T)
    k = np.concatenate([q[:3], _streams(rng, n - 3, T)])
    v = _streams(rng, n, T)
    gsign = rng.standard_normal((n, T)).astype(np.float32)
    gsign[1, 17] = np.inf                          # one +inf
    gsign[2, 40] = np.nan                          # NaN: every entry NaN
    gsign[3, [50, 90]] = [np.inf, -np.inf]         # both signs
    gsign[4, 0] = -np.inf                          # at t = 0 (no candidate: every entry NaN)
    gsign[5, [60, 61]] = np.inf
    got = _credits_direct(q, k, v, gsign)
    assert np.isnan(got[2]).all() and np.isnan(got[4]).all()
    if T <= 300:
        with np.errstate(invalid="ignore"):
            exp = orr.credits(q, k, v, gsign)
        assert np.array_equal(np.isnan(got), np.isnan(exp))
        assert np.array_equal(np.isposinf(got), np.isposinf(exp))
        assert np.array_equal(np.isneginf(got), np.isneginf(exp))
        np.testing.assert_allclose(got[[0, 6]], exp[[0, 6]], rtol=1e-5, atol=1e-5 * np.abs(exp[[0, 6]]).max())
        assert np.isinf(got[1]).any()
        return
    base, _, _ = orr.match(q, k, v)
    for s in (1, 3, 5):
        inf_entries = np.argwhere(np.isinf(got[s]))
        picks = [tuple(e) for e in inf_entries[:6]]
        picks += [(int(w), int(p)) for w, p in zip(rng.integers(0, 3, 6), rng.integers(0, T, 6))]
        for which, p in picks:
            exp = _dense_entry(q, k, v, gsign, s, which, p, base)
            a = got[s, which, p]
            assert (np.isnan(a) and np.isnan(exp)) or a == exp, (s, which, p, a, exp)
    for which, p in zip(rng.integers(0, 3, 6), rng.integers(0, T, 6)):
        exp = _dense_entry(q, k, v, gsign, 0, which, p, base)
        assert abs(got[0, which, p] - exp) <= 1e-5 * max(abs(exp), np.abs(gsign[0]).max())


def test_credits_repeated_calls_zero_gradient():
    """Many calls on freshly allocated output buffers filled with NaN beforehand, zero
    gradient: every credit is exactly zero on every call (the conversion kernel reads each
    stream's mode words, held in the output buffer, before overwriting them)."""
    from ksdraft_amd import _lib
    rng = np.random.default_rng(9)
    n, T = 256, 2048
    q, k, v = (_streams(rng, n, T) for _ in range(3))
    proj = [_bits_to_proj(b, rng).T[None] for b in (q, k, v)]
    packed = [R.pack_bits(_g(p)).reshape(n, -1).contiguous() for p in proj]
    _, mj = R.match_packed(*packed, T, want_j=True)
    grad = torch.zeros((1, T, n), device=DEV)
    pay = torch.ones(n, device=DEV)
    bad = []
    for i in range(100):
        cred = torch.full((n, 3, T), float("nan"), device=DEV)
        part = torch.full((n,), float("nan"), device=DEV)
        sums = torch.full((n, 3, T), -1, dtype=torch.int64, device=DEV)
        _lib.call("ksd_rosa_credits", packed[0].data_ptr(), packed[1].data_ptr(), packed[2].data_ptr(),
                  mj.contiguous().data_ptr(), grad.data_ptr(), pay.data_ptr(), 1, T, n, 62,
                  cred.data_ptr(), part.data_ptr(), sums.data_ptr(), _lib.stream_ptr(torch.device(DEV)))
        bad.append(torch.stack([(cred != 0).sum(), (part != 0).sum()]))
    bad = torch.stack(bad).cpu().numpy()
    assert not bad.any(), np.nonzero(bad.any(1))[0][:5]


def test_credits_t2100_sampled_flips():
    """T above 2048 takes the candidate-per-lane kernel: sampled flips by definition."""
    rng = np.random.default_rng(2100)
    n, T = 2, 2100
    q = _streams(rng, n, T)
    k = np.concatenate([q[:1], _streams(rng, n - 1, T)])
    v = _streams(rng, n, T)
    gsign = rng.standard_normal((n, T)).astype(np.float32)
    got = _credits_direct(q, k, v, gsign)
    base, _, _ = orr.match(q, k, v)
    for s in range(n):
        for which in range(3):
            for p in rng.choice(T, 5, replace=False):
                fl = [b[s:s + 1].copy() for b in (q, k, v)]
                fl[which][0, p] ^= 1
                sp, _, _ = orr.match(*fl)
                exp = float(((sp[0] - base[s]) * gsign[s].astype(np.float64)).sum())
                assert abs(got[s, which, p] - exp) <= 1e-5 * max(1.0, abs(exp)), (s, which, p)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_rosa_mixer_int8_projections_eval_fused_branch(dtype):
    """RosaMixer in eval with Int8Linear q/k/v/out (the to_int8 surfaces): the time shift
    and the three input quantizations run as one kernel, then the W8A8 GEMMs (+ bias) and
    the match. Checked stage by stage against the oracle: the shifted inputs' codes, the
    projections (ordered-group contract + bias, in x's dtype), the match signs, and the
    output projection of payload * sign."""
    from ksdraft_amd.kernels.linear import Int8Linear
    from oracle import gemm as og
    torch.manual_seed(5)
    d, S, B, T = 256, 32, 2, 40
    m = RosaMixer(d, S).to(DEV)
    with torch.no_grad():
        for lin in (m.q_proj, m.k_proj, m.v_proj, m.out_proj):
            lin.weight.normal_(0, 0.05)
            lin.bias.normal_(0, 0.05)
        for mix in (m.time_mix_q, m.time_mix_k, m.time_mix_v):
            mix.normal_(0, 1.0)
    for name in ("q_proj", "k_proj", "v_proj", "out_proj"):
        setattr(m, name, Int8Linear.from_float(getattr(m, name)))
    m.eval()
    x = (torch.randn(B, T, d) * 1.5).to(dtype).to(DEV)
    with torch.no_grad():
        y = m(x)
    xv = x.float().cpu().numpy()
    bits = []
    for proj, mix in ((m.q_proj, m.time_mix_q), (m.k_proj, m.time_mix_k), (m.v_proj, m.time_mix_v)):
        sig = torch.sigmoid(mix.detach().float()).cpu().numpy()
        lerp = orr.shifted(xv, sig, str(dtype).split(".")[-1]).reshape(B * T, d)
        xq, xs = oq.quantize_last_dim(lerp)
        wq, ws = oq.quantize_last_dim(proj.weight.detach().cpu().numpy())
        pre = og.gemm_ordered(xq, xs, wq, ws, bias=proj.bias.detach().cpu().numpy())
        pre = torch.from_numpy(pre).to(dtype).float().numpy()   # the projection's output dtype
        bits.append(orr.bits_of(pre.reshape(B, T, S)).transpose(0, 2, 1).reshape(B * S, T))
    sign, _, _ = orr.match(*bits)
    hard = (m.payload.detach().cpu().numpy()[None, :, None] * sign.reshape(B, S, T)).transpose(0, 2, 1)
    hin = torch.from_numpy(np.ascontiguousarray(hard)).to(dtype).float().numpy().reshape(B * T, S)
    hq, hs = oq.quantize_last_dim(hin)
    oq_, os_ = oq.quantize_last_dim(m.out_proj.weight.detach().cpu().numpy())
    exp = og.gemm_ordered(hq, hs, oq_, os_, bias=m.out_proj.bias.detach().cpu().numpy())
    exp = torch.from_numpy(exp).to(dtype).reshape(B, T, d)
    assert torch.equal(y.cpu(), exp)


def _x_of(dtype, shape, gen, scale=1.5):
    t = torch.randn(*shape, generator=gen) * scale
    return t.to(getattr(torch, dtype)).to(DEV)


@pytest.mark.parametrize("dtype", ["float32", "bfloat16", "float16"])
@pytest.mark.parametrize("B,T,d", [(2, 33, 320), (1, 130, 256), (3, 64, 1536), (2, 100, 136)])
def test_shift_quantize_dual(dtype, B, T, d):
    """Training form of the fused shift: each input's row codes and its transposed,
    requantized operand bit-exact against quantize_last_dim and requant_transpose of the
    oracle's shift (the Int8Linear training recipe applied to _shifted's outputs)."""
    gen = torch.Generator().manual_seed(B * 1000 + T + d)
    x = _x_of(dtype, (B, T, d), gen)
    sig = [torch.sigmoid(torch.randn(d, generator=gen) * 2).to(DEV) for _ in range(3)]
    got = R.shift_quantize_dual(x, *sig)
    xv = x.float().cpu().numpy()
    for m in range(3):
        lerp = orr.shifted(xv, sig[m].cpu().numpy(), dtype).reshape(B * T, d)
        xq, xs = oq.quantize_last_dim(lerp)
        xtq, xts = oq.requant_transpose(xq, xs)
        codes, scales, codes_t, scales_t = (t.cpu().numpy() for t in got[m])
        assert np.array_equal(codes, xq), m
        assert np.array_equal(scales.view(np.uint16), xs.view(np.uint16)), m
        assert np.array_equal(codes_t, xtq), m
        assert np.array_equal(scales_t.view(np.uint16), xts.view(np.uint16)), m


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
@pytest.mark.parametrize("B,T,d", [(2, 33, 320), (1, 130, 260), (3, 70, 1536), (2, 17, 258)])
def test_shift_backward(dtype, B, T, d):
    """The shift's backward against the oracle's float64 gradient: dx within fp32 rounding
    of six terms (one bf16 rounding for bf16 x), dsig within fp32 accumulation over the
    tokens (bounded by the sum of |g * (x - prev)|)."""
    gen = torch.Generator().manual_seed(B * 7 + T + d)
    x = _x_of(dtype, (B, T, d), gen)
    sig = torch.sigmoid(torch.randn(3, d, generator=gen) * 2).to(DEV)
    gs = [torch.randn(B, T, d, generator=gen).to(DEV) for _ in range(3)]
    dx, dsig = R.shift_backward(x, *gs, sig[0], sig[1], sig[2])
    assert dx.dtype == x.dtype and dx.shape == x.shape
    edx, edsig = orr.shifted_backward(x.float().cpu().numpy(), sig.cpu().numpy(),
                                      [g.cpu().numpy() for g in gs], dtype)
    got = dx.float().cpu().numpy()
    if dtype == "float32":
        np.testing.assert_allclose(got, edx, rtol=1e-5, atol=1e-6 * np.abs(edx).max())
    else:
        np.testing.assert_allclose(got, edx, rtol=2.0 ** -8, atol=1e-6 * np.abs(edx).max())
    xv = x.float().cpu().numpy()
    prev = np.concatenate([np.zeros_like(xv[:, :1]), xv[:, :-1]], 1)
    bound = sum(np.abs(g.cpu().numpy() * (xv - prev)).sum(axis=(0, 1)) for g in gs)
    assert np.all(np.abs(dsig.cpu().numpy() - edsig) <= 1e-5 * bound + 1e-30)


def _int8_mixer(d, S, seed):
    from ksdraft_amd.kernels.linear import Int8Linear
    torch.manual_seed(seed)
    m = RosaMixer(d, S)
    with torch.no_grad():
        for p in (m.time_mix_q, m.time_mix_k, m.time_mix_v):
            p.normal_(0, 1)
        m.out_proj.weight.normal_(0, 0.05)
        for p in (m.q_proj, m.k_proj, m.v_proj):
            p.bias.normal_(0, 0.1)
    m = m.to(DEV)
    for name in ("q_proj", "k_proj", "v_proj", "out_proj"):
        setattr(m, name, Int8Linear.from_float(getattr(m, name)))
    return m


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_shifted_int8_projections_training_match_composed(dtype):
    """Training with Int8Linear q/k/v: the fused shift + dual quantization path
    (ShiftedInt8Projections) against torch's _shifted followed by the three Int8Linear
    layers on the same inputs. q/k/v outputs, dW and db bit-exact (the same int8 operands
    and GEMMs); dx and the time-mix gradients within fp32 summation order."""
    import copy
    m1 = _int8_mixer(256, 64, 3)
    m2 = copy.deepcopy(m1)
    m2.fused_shift = False
    m1.train(), m2.train()
    x0 = torch.randn(2, 40, 256, generator=torch.Generator().manual_seed(4)).to(dtype).to(DEV)
    x1 = x0.clone().requires_grad_(True)
    x2 = x0.clone().requires_grad_(True)
    outs1 = m1._fused_training_projections(x1)
    assert outs1 is not None
    q_in, k_in, v_in = m2._shifted(x2)
    outs2 = (m2.q_proj(q_in), m2.k_proj(k_in), m2.v_proj(v_in))
    gen = torch.Generator().manual_seed(5)
    gs = [torch.randn(o.shape, generator=gen).to(DEV) * 1e-2 for o in outs2]
    for a, b in zip(outs1, outs2):
        assert a.dtype == b.dtype == torch.float32
        assert torch.equal(a, b)
    torch.autograd.backward(outs1, gs)
    torch.autograd.backward(outs2, gs)
    for name in ("q_proj", "k_proj", "v_proj"):
        p1, p2 = getattr(m1, name), getattr(m2, name)
        assert torch.equal(p1.weight.grad, p2.weight.grad), name
        assert torch.equal(p1.bias.grad, p2.bias.grad), name
    assert x1.grad.dtype == x2.grad.dtype == dtype
    rt = 1e-5 if dtype == torch.float32 else 2.0 ** -7
    torch.testing.assert_close(x1.grad.float(), x2.grad.float(), rtol=rt,
                               atol=rt * x2.grad.float().abs().max().item())
    for name in ("time_mix_q", "time_mix_k", "time_mix_v"):
        g1, g2 = getattr(m1, name).grad, getattr(m2, name).grad
        torch.testing.assert_close(g1, g2, rtol=1e-4, atol=1e-4 * g2.abs().max().item())
    # and the whole training forward of the mixer agrees
    y1 = m1(x0)
    y2 = m2(x0)
    assert torch.equal(y1, y2)
