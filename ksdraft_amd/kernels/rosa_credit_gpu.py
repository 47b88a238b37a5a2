"""GPU-native Rosa counterfactual credits (mirror of reference
ksdraft/kernels/rosa_credit_gpu.py).

``HardRosaGPU.apply(q, k, v, payload)`` keeps the reference's forward (the longest-suffix
match, rosa_credit_gpu.py:62-75) and backward (exact first-order single-bit credits with
the Bernoulli logit map, :78-112). The reference re-matches a (C, 3T, T) perturbation tensor
and therefore refuses T > 63; here the credits come from ksd_rosa_credits, which derives
every flip's new match from one scan per position, so the window guard is lifted. The
credits' summation order is not the reference's (fp32 atomics): flip decisions are exact,
credit values agree to rounding.
"""

from __future__ import annotations

import torch

from .. import _lib
from . import rosa as R

MAX_WINDOW = 65535  # supported T (the reference's exact int64 path stops at 63)


class HardRosaGPU(torch.autograd.Function):
    """q/k/v: (B, T, S) pre-bit projections; payload: (S,) -> hard (B, T, S) fp32."""

    @staticmethod
    def forward(ctx, q, k, v, payload):
        if q.shape[1] > MAX_WINDOW:
            raise ValueError(f"GPU exact credits support T <= {MAX_WINDOW}; got T={q.shape[1]}")
        B, T, S = q.shape
        bits = R.pack_bits3(q.detach(), k.detach(), v.detach())
        sign, mj = R.match_packed(*(b.reshape(B * S, -1) for b in bits), T, want_j=True)
        sign = sign.reshape(B, S, T)
        ctx.save_for_backward(q, k, v, payload, sign, mj, *bits)
        return R.hard_out(sign, payload.detach(), torch.float32)

    @staticmethod
    def backward(ctx, grad_out):
        q, k, v, payload, sign, mj, qb, kb, vb = ctx.saved_tensors
        B, T, S = q.shape
        dev = q.device
        grad = grad_out.float().contiguous()
        p32 = payload.detach().float().contiguous()
        lmax = R.resolve_max_match_len(T)
        cred = torch.empty((B * S, 3, T), dtype=torch.float32, device=dev)
        part = torch.empty((B * S,), dtype=torch.float32, device=dev)
        # int64 fixed-point sums: the credits come out the same on every run
        sums = torch.empty((B * S, 3, T), dtype=torch.int64, device=dev)
        st = _lib.stream_ptr(dev)
        _lib.call("ksd_rosa_credits", qb.data_ptr(), kb.data_ptr(), vb.data_ptr(), mj.data_ptr(),
                  grad.data_ptr(), p32.data_ptr(), B, T, S, lmax, cred.data_ptr(),
                  part.data_ptr(), sums.data_ptr(), st)
        dt = q.dtype if q.dtype in (torch.float32, torch.bfloat16, torch.float16) else torch.float32
        qc, kc, vc = (t.detach().to(dt).contiguous() for t in (q, k, v))
        gq, gk, gv = (torch.empty((B, T, S), dtype=dt, device=dev) for _ in range(3))
        gp = torch.empty((S,), dtype=torch.float32, device=dev)
        _lib.call("ksd_rosa_credit_grads", cred.data_ptr(), qc.data_ptr(), kc.data_ptr(),
                  vc.data_ptr(), _lib.dtype_code(dt), part.data_ptr(), B, T, S,
                  gq.data_ptr(), gk.data_ptr(), gv.data_ptr(), gp.data_ptr(), st)
        return gq.to(q.dtype), gk.to(k.dtype), gv.to(v.dtype), gp.to(payload.dtype)
