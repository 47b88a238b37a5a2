#!/usr/bin/env python3
"""Benchmark: KSDraft INT8 tier on one MI355X.

Workload: one W8A8 GS128 linear layer at training shape,
forward + both backward GEMMs, M = 8192 tokens (batch 4 x seq 2048), K = N = 1536.
X ~ N(0,1), W ~ N(0,0.02) fp32 master, dY ~ N(0,1e-2), all fp32, seeded (torch CPU
generator, seed 0) and resident in HBM before timing.

One step = exactly what the training path (Int8Linear / W8A8LinearFunction) runs for
this layer when it quantizes its own master:
    quantize W, and W^T requantized along N, in one pass (quantize_dual)
    -> quantize X, and X^T requantized along M, in one pass (quantize_dual)
      -> GEMM Y = X W^T (fp32 out)
    quantize dY along N and along M in one pass (quantize_dual)
      -> GEMM dX = dY W -> GEMM dW = dY^T X   (fp32)
value = algorithmic int8 ops of the three GEMMs (3 * 2*M*N*K) / step time, in TOPS.
The steps run as a captured HIP graph of G consecutive steps (G the largest divisor of K
up to 16), replayed K / G times: no host launch overhead, and the ~15 us that each graph
replay costs beyond its kernels is paid once per G steps. Replays are checked bit-equal to
the eager step; the one-step graph and the eager step times are reported beside it.

Also reported: the step's four launches timed inside the step (HIP events between them
on the launch stream, eager steps); per-kernel average launch times of back-to-back
launches (HIP events around graphs of them); the GEMM roofline against the 5.0 POPS
dense int8 peak, from the in-step GEMM durations; and the CPU oracle (the reference's CPU
path: dequantize + fp32 matmul) timed on a bounded sample on this host.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from ksdraft_amd.kernels.linear import (w8a8_linear_backward,  # noqa: E402
                                        w8a8_linear_forward_train)
from ksdraft_amd.kernels.quant import (quantize_dual, quantize_dual2, quantize_last_dim,  # noqa: E402
                                       quantize_transpose, requant_transpose)
from ksdraft_amd.kernels.gemm import w8a8_gemm_out, w8a8_gemm_pair  # noqa: E402
from ksdraft_amd.train import adamw_requant_, cross_entropy_grad_int8, cross_entropy_stats  # noqa: E402

METRIC = ("W8A8 GS128 GEMM TOPS fwd+bwd @d=1536 (% int8 peak); draft train-step tok/s")
PEAK_INT8 = 5.0e15   # MI355X dense int8 MFMA, ops/s
PEAK_HBM = 8.0e12    # MI355X HBM3E, bytes/s
M, K, N = 8192, 1536, 1536
GEMM_OPS = 2 * M * N * K


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--kernel-reps", type=int, default=20)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=15.0)
    p.add_argument("--no-ks3", action="store_true", help="skip the KS3 kernel report")
    p.add_argument("--no-rosa", action="store_true", help="skip the Rosa kernel report")
    p.add_argument("--no-c3", action="store_true", help="skip the config-3 LM-head report")
    p.add_argument("--no-ln", action="store_true", help="skip the fused LayerNorm + quantize report")
    p.add_argument("--no-c5", action="store_true", help="skip the config-5 draft train step")
    p.add_argument("--c5-steps", type=int, default=3)
    p.add_argument("--c5-loss-scale", type=float, default=C5_LOSS_SCALE,
                   help="power-of-two loss scale of the config-5 step (1 = unscaled)")
    p.add_argument("--only-c5", action="store_true", help="run only the config-5 step (profiling)")
    p.add_argument("--pmc-probe", action="store_true",
                   help="for rocprofv3 --pmc runs: a 256 MiB device copy (counter "
                        "calibration), then 3 launches of each GEMM of the step; no timing")
    return p.parse_args()


def pmc_probe(x, w, dy):
    """Workload for the HBM-traffic counters: torch's device copy of a known size
    (256 MiB read + 256 MiB written) to calibrate FETCH_SIZE/WRITE_SIZE, then the three
    GEMMs on their real operands, 3 launches each, then 3 paired dX + dW launches (the
    step's backward)."""
    src = torch.empty(64 * 1024 * 1024, dtype=torch.float32, device=x.device).fill_(1.0)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
    wq, ws = quantize_last_dim(w)
    xq, xs = quantize_last_dim(x)
    gq, gs = quantize_last_dim(dy)
    wtq, wts = requant_transpose(wq, ws)
    gtq, gts = quantize_transpose(dy)
    xtq, xts = requant_transpose(xq, xs)
    torch.cuda.synchronize()
    for _ in range(3):
        w8a8_gemm_out(xq, xs, wq, ws)
        w8a8_gemm_out(gq, gs, wtq, wts)
        w8a8_gemm_out(gtq, gts, xtq, xts)
    for _ in range(3):  # the step's backward: dX and dW as one launch
        w8a8_gemm_pair((gq, gs, wtq, wts, torch.float32), (gtq, gts, xtq, xts, torch.float32))
    torch.cuda.synchronize()
    print("pmc probe done", flush=True)


def make_inputs(dev):
    g = torch.Generator().manual_seed(0)
    x = torch.randn(M, K, generator=g)
    w = torch.randn(N, K, generator=g) * 0.02
    dy = torch.randn(M, N, generator=g) * 1e-2
    return x, w, dy, x.to(dev), w.to(dev), dy.to(dev)


def step(x, w, dy):
    # W's row codes and the requantized W^T that dX needs, and X's codes and requantized
    # X^T that dW needs, from one pass over each, in one launch (Int8Linear's training
    # forward does the same when its codes are stale)
    (wq, ws, wtq, wts), xpre = quantize_dual2(w, x)
    y, xtq, xts = w8a8_linear_forward_train(x, wq, ws, None, out_dtype=torch.float32, xpre=xpre)
    # dX and dW in one launch (w8a8_linear_backward pairs them)
    dx, dw = w8a8_linear_backward(dy, None, None, wq, ws, dx_dtype=torch.float32, xt=(xtq, xts),
                                  wt=(wtq, wts))
    return y, dx, dw


def step_kernel_times(x, w, dy, steps, warmup):
    """Average duration (us) of each of the step's four launches, measured inside the step:
    HIP events recorded between the launches on the launch stream over `steps` eager steps
    (the launches of step() with the backward split into its dual quantization and its
    paired GEMM launch, checked bit-equal to step()). An interval also holds the dispatch
    gap before its launch, so it bounds the kernel's own time from above."""
    f32 = torch.float32

    def run(evs=None):
        def rec(i):
            if evs is not None:
                evs[i].record()
        rec(0)
        (wq, ws, wtq, wts), xpre = quantize_dual2(w, x)
        rec(1)
        y, xtq, xts = w8a8_linear_forward_train(x, wq, ws, None, out_dtype=f32, xpre=xpre)
        rec(2)
        gq, gs, gtq, gts = quantize_dual(dy)
        rec(3)
        dx, dw = w8a8_gemm_pair((gq, gs, wtq, wts, f32), (gtq, gts, xtq, xts, f32))
        rec(4)
        return y, dx, dw

    for a, b in zip(run(), step(x, w, dy)):
        if not torch.equal(a, b):
            raise SystemExit("the instrumented step differs from step()")
    for _ in range(warmup):
        run()
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(5)] for _ in range(steps)]
    torch.cuda.synchronize()
    for e in evs:
        run(e)
    torch.cuda.synchronize()
    names = ["quantize_W_X_dual2", "gemm_fwd", "quantize_dY_dual", "gemm_dX_dW_pair"]
    return {n: round(1e3 * sum(e[i].elapsed_time(e[i + 1]) for e in evs) / steps, 3)
            for i, n in enumerate(names)}


def time_graph(fn, reps, warm=3):
    """Capture fn() once, replay; returns (graph, outputs, avg ms per replay)."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(warm):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = fn()
    for _ in range(warm):
        graph.replay()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for _ in range(reps):
        graph.replay()
    e1.record(st)
    torch.cuda.synchronize()
    return graph, out, e0.elapsed_time(e1) / reps


def kernel_times(x, w, dy, reps):
    """Average launch time (us) of every kernel of the step, each timed as a graph of
    `reps` back-to-back launches bracketed by HIP events on the capture stream."""
    wq, ws = quantize_last_dim(w)
    xq, xs = quantize_last_dim(x)
    gq, gs = quantize_last_dim(dy)
    wtq, wts = requant_transpose(wq, ws)
    gtq, gts = quantize_transpose(dy)
    xtq, xts = requant_transpose(xq, xs)
    stages = {
        "quantize_W_dual": (lambda: quantize_dual(w, t_from_codes=True), 4 * N * K + 2 * (N * K + 2 * N * K // 128)),
        "quantize_X_dual": (lambda: quantize_dual(x, t_from_codes=True), 4 * M * K + 2 * (M * K + 2 * M * K // 128)),
        "gemm_fwd": (lambda: w8a8_gemm_out(xq, xs, wq, ws), None),
        # W's and X's dual quantization as one launch (the step's first kernel)
        "quantize_W_X_dual2": (lambda: quantize_dual2(w, x), 4 * (M + N) * K + 2 * ((M + N) * K + 2 * (M + N) * K // 128)),
        "quantize_dY_dual": (lambda: quantize_dual(dy), 4 * M * N + 2 * (M * N + 2 * M * N // 128)),
        "gemm_dX": (lambda: w8a8_gemm_out(gq, gs, wtq, wts), None),
        "gemm_dW": (lambda: w8a8_gemm_out(gtq, gts, xtq, xts), None),
        # dX and dW as one launch (the step's backward): ops of two GEMMs
        "gemm_dX_dW_pair": (lambda: w8a8_gemm_pair((gq, gs, wtq, wts, torch.float32),
                                                   (gtq, gts, xtq, xts, torch.float32)), None),
        # the single-layout kernels the dual ones replace in the step (for comparison)
        "quantize_W": (lambda: quantize_last_dim(w), 4 * N * K + N * K + 2 * N * K // 128),
        "requant_WT": (lambda: requant_transpose(wq, ws), 2 * (N * K + 2 * N * K // 128)),
        "quantize_X": (lambda: quantize_last_dim(x), 4 * M * K + M * K + 2 * M * K // 128),
        "requant_XT": (lambda: requant_transpose(xq, xs), 2 * (M * K + 2 * M * K // 128)),
        "quantize_dY": (lambda: quantize_last_dim(dy), 4 * M * N + M * N + 2 * M * N // 128),
        "quantize_T_dY": (lambda: quantize_transpose(dy), 4 * M * N + M * N + 2 * M * N // 128),
    }
    res = {}
    for name, (fn, nbytes) in stages.items():
        def rep(fn=fn):
            for _ in range(reps):
                fn()
        _, _, ms = time_graph(rep, 3, warm=1)
        us = ms * 1e3 / reps
        ent = {"us": round(us, 3)}
        if nbytes is None:
            nops = GEMM_OPS * (2 if name.endswith("_pair") else 1)
            ent["tops"] = round(nops / (us * 1e-6) / 1e12, 1)
        else:
            ent["GBps"] = round(nbytes / (us * 1e-6) / 1e9, 1)
            ent["hbm_frac"] = round(nbytes / (us * 1e-6) / PEAK_HBM, 3)
        res[name] = ent
    return res


def ks3_kernel_times(dev, reps):
    """The KS3 cell's kernels at BASELINE config 4's shape (M = 8192 tokens, d = 1536,
    F = 5888 charts): average launch time and HBM rate against the algorithmic bytes.
    Synthetic inputs: coordinates ~N(0, 0.8) (x ~N(0,1) through down ~N(0,0.02)),
    value ~N(0, 1e-2), reference inits for the cell (coefficients ~N(0,0.05), raw_scale
    0.75, raw_shift 0; model/ks3.py:85-88). GEMM entries (the down GEMM, and project_fused
    with the spine in one launch or two) report TOPS against the down GEMM's 2·M·F·d."""
    from ksdraft_amd.kernels import ks3_int8 as K
    from ksdraft_amd.kernels.ks3_triton import project_fused
    Mk, d, Fc, G = 8192, 1536, 5888, 128
    g = torch.Generator().manual_seed(0)
    coeffs = (torch.randn(Fc, 6, generator=g) * 0.05).to(dev)
    raw_scale = torch.full((Fc,), 0.75, device=dev)
    raw_shift = torch.zeros(Fc, device=dev)
    coords16 = (torch.randn(Mk, Fc, generator=g) * 0.8).to(dev).half()
    acc32 = coords16.float()
    value16 = (torch.randn(Mk, Fc, generator=g) * 1e-2).to(dev).half()
    x = torch.randn(Mk, d, generator=g).to(dev)
    down = (torch.randn(Fc, d, generator=g) * 0.02).to(dev)
    sq, ss = K.pack_spine(coeffs, G)
    sc16 = (torch.nn.functional.softplus(raw_scale) + 1e-4).half()
    sh16 = (0.5 * torch.tanh(raw_shift)).half()
    lut = K.make_tanh_lut(dev)
    xq, xs = quantize_last_dim(x)
    dq, ds = quantize_last_dim(down)
    MF = Mk * Fc
    stages = {
        "gemm_down_f16sat": (lambda: w8a8_gemm_out(xq, xs, dq, ds, fp16_saturate=True), None),
        "ks3_spine_fwd": (lambda: K.spine_int8(coords16, sq, ss, sc16, sh16, lut, G),
                          2 * MF + MF + 2 * MF // G),
        "ks3_spine_fused": (lambda: K.spine_fused_int8(acc32, sq, ss, sc16, sh16, lut, G),
                            4 * MF + MF + 2 * MF // G),
        "ks3_vjp": (lambda: K.ks3_vjp(value16, coords16, sq, ss, sc16, sh16, raw_scale,
                                      raw_shift, G),
                    2 * MF + 2 * MF + MF + MF + 2 * 2 * MF // G + 2 * 8 * Fc * 4 * (Mk // 512)),
        # project_fused 'int8': the down GEMM with the spine and requantization in its
        # epilogue (one launch after the table), and the default two-launch form
        "ks3_project_fused_one_launch": (lambda: project_fused(xq, xs, dq, ds, sq, ss, sc16, sh16, lut,
                                                               G, "int8", one_launch=True), None),
        "ks3_project_fused_two_launches": (lambda: project_fused(xq, xs, dq, ds, sq, ss, sc16, sh16,
                                                                 lut, G, "int8", one_launch=False), None),
    }
    res = {}
    for name, (fn, nbytes) in stages.items():
        def rep(fn=fn):
            for _ in range(reps):
                fn()
        _, _, ms = time_graph(rep, 3, warm=1)
        us = ms * 1e3 / reps
        ent = {"us": round(us, 3)}
        if nbytes is None:
            ent["tops"] = round(2 * Mk * Fc * d / (us * 1e-6) / 1e12, 1)
        else:
            ent["bytes"] = nbytes
            ent["GBps"] = round(nbytes / (us * 1e-6) / 1e9, 1)
            ent["hbm_frac"] = round(nbytes / (us * 1e-6) / PEAK_HBM, 3)
        res[name] = ent
    return res


def lmhead_c3_times(dev, reps):
    """the LM-head / vocab projection as one W8A8 GS128 linear layer,
    forward + dX + dW, M = 4096 tokens, K = 1536, N = 150144 (int8 W 230.6 MB, fp32 Y
    2.46 GB). X ~N(0,1), W ~N(0,0.02) drawn by a seeded generator on the device (1 GB of
    fp32 master weights), targets t uniform in [0, N). The step is the head's training step:
    the fused AdamW + int8 repack of W, the forward GEMM, the fused cross entropy (row
    statistics, then dY quantized in both layouts), and the dX and dW GEMMs. Each kernel is
    timed as a graph of back-to-back launches; GEMMs are reported in TOPS against
    2*M*N*K = 1.889e12 ops per GEMM (the backward's dX and dW run as one launch), the rest in GB/s against their algorithmic bytes. Entries named
    cmp_* are unfused alternatives, timed for comparison and not summed."""
    M3, K3, N3 = 4096, 1536, 150144
    g = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn(M3, K3, device=dev, generator=g)
    w = torch.randn(N3, K3, device=dev, generator=g) * 0.02
    wq, ws = quantize_last_dim(w)
    xq, xs = quantize_last_dim(x)
    y = w8a8_gemm_out(xq, xs, wq, ws)
    t = torch.randint(0, N3, (M3,), device=dev, generator=g)
    dy = torch.softmax(y, dim=1)
    dy[torch.arange(M3, device=dev), t] -= 1.0
    gq, gs = quantize_last_dim(dy)
    wtq, wts = requant_transpose(wq, ws)
    gtq, gts = quantize_transpose(dy)
    xtq, xts = requant_transpose(xq, xs)
    ops = 2 * M3 * N3 * K3
    # the loss side: fused cross entropy on the logits (row statistics, then dY formed and
    # quantized in both layouts without an fp32 dY)
    _, rmax, rinv, n_rows = cross_entropy_stats(y, t, check_targets=False)
    gsc = (torch.ones((), device=dev) / n_rows).reshape(1)
    # the optimizer side: AdamW on the fp32 master fused with its int8 repack (this replaces
    # the forward's per-call weight quantization), and torch's AdamW + quantize to compare
    wm = torch.zeros_like(w)
    wv = torch.zeros_like(w)
    wg = torch.randn(N3, K3, device=dev, generator=g) * 1e-3
    tw = w.clone().requires_grad_(True)
    tw.grad = wg.clone()
    topt = torch.optim.AdamW([tw], lr=1e-3, weight_decay=0.01, capturable=True)

    def torch_adamw_quantize():
        topt.step()
        return quantize_last_dim(tw.detach())

    stages = {
        "adamw_requant_W": (lambda: adamw_requant_(w, wg, wm, wv, 2, 1e-3, weight_decay=0.01),
                            29 * N3 * K3 + 2 * N3 * K3 // 128),
        "quantize_X_dual": (lambda: quantize_dual(x, t_from_codes=True), 4 * M3 * K3 + 2 * (M3 * K3 + 2 * M3 * K3 // 128)),
        "gemm_fwd": (lambda: w8a8_gemm_out(xq, xs, wq, ws), None),
        "ce_row_stats": (lambda: cross_entropy_stats(y, t, check_targets=False), 4 * M3 * N3),
        "ce_grad_int8_dual": (lambda: cross_entropy_grad_int8(y, t, rmax, rinv, gsc),
                              4 * M3 * N3 + 2 * (M3 * N3 + 2 * M3 * N3 // 128)),
        "requant_WT": (lambda: requant_transpose(wq, ws), 2 * (N3 * K3 + 2 * N3 * K3 // 128)),
        # dX and dW as one launch (the step's backward): ops of two GEMMs
        "gemm_dX_dW_pair": (lambda: w8a8_gemm_pair((gq, gs, wtq, wts, torch.float32),
                                                   (gtq, gts, xtq, xts, torch.float32)), None),
        # not part of the step: dX and dW as two launches, the unfused dual quantization
        # of a dY computed beforehand,
        # the forward's weight quantization the fused optimizer makes unnecessary, and
        # torch's AdamW step followed by that quantization
        "cmp_gemm_dX": (lambda: w8a8_gemm_out(gq, gs, wtq, wts), None),
        "cmp_gemm_dW": (lambda: w8a8_gemm_out(gtq, gts, xtq, xts), None),
        "cmp_quantize_dY_dual": (lambda: quantize_dual(dy), 4 * M3 * N3 + 2 * (M3 * N3 + 2 * M3 * N3 // 128)),
        "cmp_quantize_W": (lambda: quantize_last_dim(w), 4 * N3 * K3 + N3 * K3 + 2 * N3 * K3 // 128),
        "cmp_torch_adamw_then_quantize_W": (torch_adamw_quantize, 29 * N3 * K3 + 2 * N3 * K3 // 128),
    }
    res = {}
    for name, (fn, nbytes) in stages.items():
        def rep(fn=fn):
            for _ in range(reps):
                fn()
        _, _, ms = time_graph(rep, 1, warm=1)
        us = ms * 1e3 / reps
        ent = {"us": round(us, 2)}
        if nbytes is None:
            ent["tops"] = round(ops * (2 if name.endswith("_pair") else 1) / (us * 1e-6) / 1e12, 1)
        else:
            ent["GBps"] = round(nbytes / (us * 1e-6) / 1e9, 1)
            ent["hbm_frac"] = round(nbytes / (us * 1e-6) / PEAK_HBM, 3)
        res[name] = ent
        torch.cuda.empty_cache()
    gemm_us = res["gemm_fwd"]["us"] + res["gemm_dX_dW_pair"]["us"]
    step_us = sum(v["us"] for k, v in res.items() if not k.startswith("cmp_"))
    res["three_gemms_ms"] = round(gemm_us / 1e3, 3)
    res["three_gemms_tops"] = round(3 * ops / (gemm_us * 1e-6) / 1e12, 1)
    res["step_ms_sum_of_kernels"] = round(step_us / 1e3, 3)
    res["step_tops_incl_quantize"] = round(3 * ops / (step_us * 1e-6) / 1e12, 1)
    return res


def rosa_kernel_times(dev, reps):
    """The Rosa mixer step's kernels at BASELINE config 4's shape (B = 4, T = 2048,
    d = 1536, S = 512 streams). x ~N(0,1) bf16; projections ~N(0,1) (their signs are the
    symbol bits); time mixes 0 and payload 1 (model/rosa.py:117-123 inits); upstream
    gradient ~N(0,1). The match and the credits are integer-VALU work over the
    B*S*T*(T-1)/2 = 4.29e9 (t, j) pairs, reported as pairs/s."""
    from ksdraft_amd.kernels import rosa as R
    from ksdraft_amd.kernels.rosa_credit_gpu import HardRosaGPU
    Bq, T, d, S = 4, 2048, 1536, 512
    g = torch.Generator().manual_seed(0)
    x = torch.randn(Bq, T, d, generator=g).to(dev).to(torch.bfloat16)
    sig = torch.full((d,), 0.5, device=dev)
    q, k, v = (torch.randn(Bq, T, S, generator=g).to(dev) for _ in range(3))
    payload = torch.ones(S, device=dev)
    gout = torch.randn(Bq, T, S, generator=g).to(dev)
    bits = [R.pack_bits(t) for t in (q, k, v)]
    flat = [b.reshape(Bq * S, -1) for b in bits]
    sign, mj = R.match_packed(*flat, T, want_j=True)
    pairs = Bq * S * T * (T - 1) // 2
    from ksdraft_amd import _lib
    cred = torch.empty(Bq * S, 3, T, device=dev)
    part = torch.empty(Bq * S, device=dev)
    sums = torch.empty(Bq * S, 3, T, dtype=torch.int64, device=dev)

    def credits():
        _lib.call("ksd_rosa_credits", flat[0].data_ptr(), flat[1].data_ptr(), flat[2].data_ptr(),
                  mj.data_ptr(), gout.data_ptr(), payload.data_ptr(), Bq, T, S, 62,
                  cred.data_ptr(), part.data_ptr(), sums.data_ptr(), _lib.stream_ptr(dev))

    BTd, BTS = Bq * T * d, Bq * T * S
    # the training form on fp32 x (config 5's stream dtype): both layouts of q/k/v_in, and
    # the shift's backward from three fp32 input gradients
    x32 = x.float()
    gin = [torch.randn(Bq, T, d, generator=g).to(dev) for _ in range(3)]
    stages = {
        "rosa_shift_quant": (lambda: R.shift_quantize(x, sig, sig, sig), 2 * BTd + 3 * (BTd + 2 * BTd // 128), None),
        "rosa_shift_quant_dual_f32": (lambda: R.shift_quantize_dual(x32, sig, sig, sig),
                                      4 * BTd + 6 * (BTd + 2 * BTd // 128), None),
        "rosa_shift_backward_f32": (lambda: R.shift_backward(x32, *gin, sig, sig, sig), 20 * BTd, None),
        "rosa_pack_bits_x3": (lambda: R.pack_bits3(q, k, v), 3 * (4 * BTS + BTS // 8), None),
        "rosa_match": (lambda: R.match_packed(*flat, T, want_j=True), None, pairs),
        "rosa_hard_out": (lambda: R.hard_out(sign.reshape(Bq, S, T), payload), BTS + 4 * BTS, None),
        "rosa_credits": (credits, None, pairs),
    }
    res = {}
    for name, (fn, nbytes, npairs) in stages.items():
        r = reps if npairs is None else max(1, reps // 4)

        def rep(fn=fn, r=r):
            for _ in range(r):
                fn()
        _, _, ms = time_graph(rep, 3, warm=1)
        us = ms * 1e3 / r
        ent = {"us": round(us, 3)}
        if nbytes is not None:
            ent["bytes"] = nbytes
            ent["GBps"] = round(nbytes / (us * 1e-6) / 1e9, 1)
            ent["hbm_frac"] = round(nbytes / (us * 1e-6) / PEAK_HBM, 3)
        else:
            ent["pairs"] = npairs
            ent["Gpairs_per_s"] = round(npairs / (us * 1e-6) / 1e9, 1)
        res[name] = ent
    # the autograd path end to end (forward + exact-credit backward)
    qg, kg, vg = (t.clone().requires_grad_(True) for t in (q, k, v))
    for _ in range(2):  # allocator warm-up
        HardRosaGPU.apply(qg, kg, vg, payload).backward(gout)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(3):
        HardRosaGPU.apply(qg, kg, vg, payload).backward(gout)
    torch.cuda.synchronize()
    res["hard_rosa_fwd_bwd_ms"] = round((time.perf_counter() - t0) * 1e3 / 3, 3)
    return res


def ln_quant_times(dev, reps):
    """The fused pre-norm + A-operand quantization at BASELINE config 4's activation shape
    (M = B*T = 8192 rows, d = 1536): nn.LayerNorm (model/block.py:27-41) then
    quantize_last_dim (kernels/linear.py:69) in one pass, against torch's LayerNorm
    followed by the library quantizer. x ~N(0,1), weight ~1, bias ~0. Bytes: read x, write
    the int8 codes and fp16 scales."""
    from ksdraft_amd.kernels import quant as kq
    import torch.nn.functional as F
    M, d = 8192, 1536
    g = torch.Generator().manual_seed(0)
    x32 = torch.randn(M, d, generator=g).to(dev)
    w = (1.0 + 0.1 * torch.randn(d, generator=g)).to(dev)
    b = (0.1 * torch.randn(d, generator=g)).to(dev)
    res = {}
    for tag, x in (("f32", x32), ("bf16", x32.to(torch.bfloat16))):
        nbytes = M * d * x.element_size() + M * d + 2 * M * (d // 128)
        stages = {
            f"ln_quantize_{tag}": lambda x=x: kq.layer_norm_quantize(x, w, b),
            f"cmp_torch_layer_norm_then_quantize_{tag}":
                lambda x=x: kq.quantize_last_dim(F.layer_norm(x, (d,), w.to(x.dtype), b.to(x.dtype))),
        }
        for name, fn in stages.items():
            def rep(fn=fn):
                for _ in range(reps):
                    fn()
            _, _, ms = time_graph(rep, 3, warm=1)
            us = ms * 1e3 / reps
            res[name] = {"us": round(us, 3), "bytes": nbytes,
                         "GBps": round(nbytes / (us * 1e-6) / 1e9, 1),
                         "hbm_frac": round(nbytes / (us * 1e-6) / PEAK_HBM, 3)}
    return res


# The config-5 step's loss scale. 2^12 gives every GS128 gradient group of the 24 layers
# a normal or subnormal fp16 scale (the unscaled step leaves every layer's weight gradient
# exactly zero: the groups' scales clamp to 2^-24 and their codes round to 0). Larger
# scales overflow the KS3 backward's fp16 column sums of dcoeff (reference
# ks3_int8.py:379-388 sums in fp16) within two optimizer steps (2^16: inf at step 3).
C5_LOSS_SCALE = 2.0 ** 12


def _zero_tile_fraction(tr, tokens, teacher):
    """One untimed training step with the backward GEMM launches wrapped: the fraction of
    the 128 x 128 tiles of their A operands (the int8 codes of the upstream gradients,
    dY and dY^T, and of the KS3 cell's dc) that hold only zero codes."""
    import ksdraft_amd.kernels.ks3_int8 as kk
    import ksdraft_amd.kernels.linear as kl
    import ksdraft_amd.train as ktr
    stats = [0, 0]
    orig = kl.w8a8_gemm_pair

    def counting(first, second, group=128):
        for prob in (first, second):
            a = prob[0]
            M, K = a.shape
            Mp, Kp = -(-M // 128) * 128, -(-K // 128) * 128
            nz = torch.nn.functional.pad(a != 0, (0, Kp - K, 0, Mp - M))
            nz = nz.view(Mp // 128, 128, Kp // 128, 128).any(3).any(1)
            stats[0] += int((~nz).sum())
            stats[1] += nz.numel()
        return orig(first, second, group)
    mods = (kl, kk, ktr)
    saved = [m.w8a8_gemm_pair for m in mods]
    for m in mods:
        m.w8a8_gemm_pair = counting
    try:
        tr.step(tokens, teacher)
    finally:
        for m, f in zip(mods, saved):
            m.w8a8_gemm_pair = f
    torch.cuda.synchronize()
    return round(stats[0] / max(1, stats[1]), 4)


def draft_c5(dev, steps, warmup, loss_scale=C5_LOSS_SCALE, int8_injection=True):
    """the full KSDraft draft training step, INT8 forward + backward
    through every linear. 24 DraftBlocks (Rosa 512 streams, DSpine injection, KS3 5888
    charts) at d = 1536, vocabulary 150144 with the tied int8 head and the fused
    cross-entropy, a synthetic bf16 teacher state ~N(0,1) (d 1536) on the teacher_proj
    seam, B 4 x T 2048 uniform token ids (T + 1 drawn for the shift), AdamW (lr 3e-4, wd
    0.01) fused with the int8 repack, grad-norm clip 1.0. Random init: the reference's
    inits with the zero-init surfaces woken to N(0, 0.02). int8_injection: the DSpine
    low-rank maps are Int8Linear surfaces too (every linear of the step is INT8).
    loss_scale: backward runs on loss_scale * loss (a power of two, divided out again in
    the clip factor); at random init the unscaled mean loss over 8192 tokens leaves most
    GS128 gradient groups below the fp16 scale floor, so their codes are all zero.
    tok/s = 8192 / step time (HIP events over `steps` steps after `warmup`); the forward,
    backward and optimizer parts of the step are timed with events too. The fraction of
    all-zero 128 x 128 gradient tiles among the backward GEMMs' A operands comes from one
    extra untimed step."""
    from ksdraft_amd.config import baseline_config
    from ksdraft_amd.model import KSDraftModel, to_int8
    from ksdraft_amd.train.int8_step import Int8DraftTrainer
    cfg = baseline_config()
    torch.manual_seed(0)
    fm = KSDraftModel(cfg, teacher_dim=cfg.d_model, device=dev)
    with torch.no_grad():
        for name, p in fm.named_parameters():
            if name.endswith(("up.weight", "out_proj.weight", "teacher_proj.weight")):
                p.normal_(0, 0.02)
    model = to_int8(fm, trainable=True, int8_injection=int8_injection)
    del fm
    torch.cuda.empty_cache()
    tr = Int8DraftTrainer(model, lr=3e-4, weight_decay=0.01, grad_clip=1.0,
                          loss_scale=loss_scale)
    g = torch.Generator(device=dev).manual_seed(0)
    B, T = 4, 2048
    tokens = torch.randint(0, cfg.vocab_size, (B, T + 1), device=dev, generator=g)
    teacher = torch.randn(B, T, cfg.d_model, device=dev, generator=g).to(torch.bfloat16)
    for _ in range(warmup):
        tr.step(tokens, teacher)
    torch.cuda.synchronize()
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(steps)]
    losses = []
    t0 = time.perf_counter()
    for i in range(steps):
        e = ev[i]
        e[0].record()
        tr.model.train()
        loss, ce, ts = tr.loss(tokens, teacher)
        e[1].record()
        tr.backward(loss)
        e[2].record()
        tr.optimizer_step()
        e[3].record()
        losses.append(loss.detach())
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / steps
    fwd = float(np.mean([e[0].elapsed_time(e[1]) for e in ev]))
    bwd = float(np.mean([e[1].elapsed_time(e[2]) for e in ev]))
    opt = float(np.mean([e[2].elapsed_time(e[3]) for e in ev]))
    step_ms = float(np.mean([e[0].elapsed_time(e[3]) for e in ev]))
    res = {
        "tok_per_s": round(B * T / (step_ms * 1e-3), 1),
        "ms_per_step": round(step_ms, 3),
        "wall_ms_per_step": round(wall * 1e3, 3),
        "forward_ms": round(fwd, 3), "backward_ms": round(bwd, 3), "optimizer_ms": round(opt, 3),
        "steps": steps, "warmup": warmup,
        "loss_first_last": [round(float(losses[0]), 4), round(float(losses[-1]), 4)],
        "params": sum(p.numel() for p in model.parameters()),
        "int8_gemm_ops_per_step": _c5_gemm_ops(cfg, B * T),
        "peak_mem_gb": round(torch.cuda.max_memory_allocated(dev) / 2**30, 2),
        "workload": "BASELINE config 5: 24 layers, d 1536, 512 streams, 5888 charts, vocab "
                    "150144, B 4 x T 2048, teacher state bf16 (d 1536)",
        "int8_injection": bool(int8_injection),
        "loss_scale": loss_scale,
        "zero_grad_tile_frac": _zero_tile_fraction(tr, tokens, teacher),
    }
    res["int8_gemm_tops"] = round(res["int8_gemm_ops_per_step"] / (step_ms * 1e-3) / 1e12, 1)
    # the staged int8 embedding lookup (codes of the tied head) against the float lookup
    from ksdraft_amd.kernels.embedding import embedding_gather_int8
    head = model.head
    if not head._codes_current():
        head._quantize_weight()
    ids = tokens[:, :-1]
    emb_w = model.embedding.weight.detach()
    n_ids, dm = ids.numel(), cfg.d_model
    for name, nbytes, fn in (
            ("int8_embedding_gather", n_ids * (dm + 2 * dm // 128 + 4 * dm + 8),
             lambda: embedding_gather_int8(head.weight_codes, head.weight_scales, ids,
                                           check_ids=False)),
            ("cmp_float_embedding", n_ids * (8 * dm + 8),
             lambda: torch.nn.functional.embedding(ids, emb_w))):
        def rep(fn=fn):
            for _ in range(20):
                fn()
        _, _, ms = time_graph(rep, 3, warm=1)
        us = ms * 1e3 / 20
        res[name] = {"us": round(us, 2), "GBps": round(nbytes / (us * 1e-6) / 1e9, 1)}
    del tr, model
    torch.cuda.empty_cache()
    return res


def _c5_gemm_ops(cfg, tokens):
    """int8 GEMM ops of one config-5 step: per layer the KS3 down/up (fwd, dX, dW each) and
    the Rosa q/k/v/out, plus the head and teacher_proj (no dX: its input needs no grad)."""
    d, F_, S, V = cfg.d_model, cfg.charts, cfg.rosa_streams, cfg.vocab_size
    per_layer = 3 * 2 * tokens * d * F_ * 2 + 3 * 2 * tokens * d * S * 4
    return cfg.layers * per_layer + 3 * 2 * tokens * d * V + 2 * 2 * tokens * d * d


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(x, w, dy, budget_s):
    """The reference's CPU path for the config-2 step, timed on this host's cores: the
    operand quantizations of the oracle (numpy restatement of quant.py:30-67) and each GEMM
    as the reference's CPU branch computes it (gemm.py:76-82): dequantize both operands,
    then torch's fp32 matmul. torch uses every core of the process affinity; 2 warm-up
    steps, then the median of at least 5 timed steps (more while the budget lasts)."""
    from concurrent.futures import ThreadPoolExecutor
    from oracle import quant as oq
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    X, W, DY = x.numpy(), w.numpy(), dy.numpy()
    pool = ThreadPoolExecutor(cores)

    def rows(fn, *arrs):
        """fn over row blocks of the arrays on every core (the oracle's numpy ops release
        the GIL; rows are independent, so the result equals one call)."""
        n = arrs[0].shape[0]
        cuts = [n * i // cores for i in range(cores + 1)]
        parts = list(pool.map(lambda i: fn(*(a[cuts[i]:cuts[i + 1]] for a in arrs)),
                              [i for i in range(cores) if cuts[i] < cuts[i + 1]]))
        if isinstance(parts[0], tuple):
            return tuple(np.concatenate(p) for p in zip(*parts))
        return np.concatenate(parts)

    def quant(a):  # quant.py:30-52
        return rows(oq.quantize_last_dim, a)

    def dequant(c, s):  # quant.py:55-67
        return rows(oq.dequantize_last_dim, c, s)

    def mm(aq, as_, wq, ws):  # gemm.py:77-82
        return torch.from_numpy(dequant(aq, as_)) @ torch.from_numpy(dequant(wq, ws)).T

    def cstep():
        wq, ws = quant(W)
        xq, xs = quant(X)
        mm(xq, xs, wq, ws)
        gq, gs = quant(DY)
        wtq, wts = quant(np.ascontiguousarray(dequant(wq, ws).T))   # requant W^T
        mm(gq, gs, wtq, wts)
        gtq, gts = quant(np.ascontiguousarray(DY.T))                 # quantize dY^T
        xtq, xts = quant(np.ascontiguousarray(dequant(xq, xs).T))   # requant X^T
        mm(gtq, gts, xtq, xts)

    # the threaded restatement is the oracle's, block by block
    chk = quant(X[:512])
    ref = oq.quantize_last_dim(X[:512])
    assert np.array_equal(chk[0], ref[0]) and np.array_equal(chk[1].view(np.uint16), ref[1].view(np.uint16))

    for _ in range(2):
        cstep()
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 5 or (time.perf_counter() < t_end and len(times) < 15):
        t0 = time.perf_counter()
        cstep()
        times.append(time.perf_counter() - t0)
    pool.shutdown()
    t = float(np.median(times))
    cfg = torch.__config__.show()
    blas = "MKL" if "MKL" in cfg else ("OpenBLAS" if "OpenBLAS" in cfg else "torch BLAS")
    return {
        "value": round(3 * GEMM_OPS / t / 1e12, 4), "unit": "TOPS", "cores": cores,
        "kind": "port",
        "sample": (f"full config-2 step (M={M}, K=N={K}: quantize W, X, dY; requant W^T, X^T; "
                   f"three dequantize + fp32 matmul GEMMs), median of {len(times)} after 2 "
                   f"warm-ups, {t:.3f} s/step; host {_cpu_model()}, torch "
                   f"{torch.__version__} with {torch.get_num_threads()} threads ({blas}); "
                   f"quantizers: the oracle's numpy restatement over {cores} threads of row blocks"),
    }


def traffic_from_profiles():
    path = os.path.join(ROOT, "profiles", "gemm_g128_c2_pmc.json")
    if not os.path.exists(path):
        return None, None
    with open(path) as f:
        d = json.load(f)
    return d.get("traffic_bytes_per_launch"), "profiles/gemm_g128_c2_pmc.json"


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(one MI355X per box); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    xc, wc, dyc, x, w, dy = make_inputs(dev)
    if args.pmc_probe:
        pmc_probe(x, w, dy)
        return
    if args.only_c5:
        print(json.dumps({"draft_c5": draft_c5(dev, args.c5_steps, 1, args.c5_loss_scale)}),
              flush=True)
        return

    # eager: warm-up then K timed steps
    for _ in range(args.warmup):
        ref = step(x, w, dy)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(args.steps):
        step(x, w, dy)
    e1.record()
    torch.cuda.synchronize()
    eager_ms = e0.elapsed_time(e1) / args.steps
    eager_wall_ms = (time.perf_counter() - t0) * 1e3 / args.steps

    # graphs: one of a single step, and one of G consecutive steps (G the largest divisor
    # of K up to 16); each replay is checked against the eager result, then K steps are
    # timed as K replays of the first and K / G replays of the second. A replay costs
    # ~15 us beyond its kernels (their launches run back to back inside it), so the
    # G-step graph is the headline.
    ref = [t.clone() for t in step(x, w, dy)]
    G = max(d for d in range(1, 17) if args.steps % d == 0)

    def g_steps():
        for _ in range(G):
            out = step(x, w, dy)
        return out

    def timed_graph(fn, nsteps):
        graph, outs, _ = time_graph(fn, 1)
        for _ in range(3):
            graph.replay()
            step(x, w, dy)           # eager work between replays
            torch.cuda.synchronize()
            for a, b in zip(outs, ref):
                if not torch.equal(a, b):
                    raise SystemExit("graph replay differs from the eager step")
        for _ in range(max(1, args.warmup // nsteps)):
            graph.replay()
        torch.cuda.synchronize()
        g0, g1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        g0.record()
        for _ in range(args.steps // nsteps):
            graph.replay()
        g1.record()
        torch.cuda.synchronize()
        return g0.elapsed_time(g1) / args.steps

    ms1 = timed_graph(lambda: step(x, w, dy), 1)
    ms = timed_graph(g_steps, G)

    in_step = step_kernel_times(x, w, dy, args.steps, args.warmup)
    kern = kernel_times(x, w, dy, args.kernel_reps)
    gemm_us = [kern[k]["us"] for k in ("gemm_fwd", "gemm_dX", "gemm_dW")]
    # the step's GEMM launches, timed inside the step: the forward, and dX + dW paired in
    # one launch
    step_gemm_us = in_step["gemm_fwd"] + in_step["gemm_dX_dW_pair"]
    achieved = 3 * GEMM_OPS / (step_gemm_us * 1e-6)
    traffic, tsrc = traffic_from_profiles()

    value = 3 * GEMM_OPS / (ms * 1e-3) / 1e12
    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic: seeded X~N(0,1), W~N(0,0.02), dY~N(0,1e-2), fp32, resident in HBM",
        "config": {"workload": "BASELINE config 2: W8A8 GS128 linear fwd + dX + dW, "
                               "M=8192 (4x2048), K=N=1536, fp32 in/out, steps replayed as a HIP graph",
                   "M": M, "K": K, "N": N, "group": 128},
        "pct_int8_peak": round(100 * value * 1e12 / PEAK_INT8, 2),
        "tok_per_s": round(M / (ms * 1e-3), 1),
        "gemm_only_tops": round(achieved / 1e12, 1),
        "gemm_separate_launches_tops": round(3 * GEMM_OPS / (sum(gemm_us) * 1e-6) / 1e12, 1),
        "graph_steps_per_replay": G,
        "graph1_ms_per_step": round(ms1, 5),
        "eager_ms_per_step": round(eager_ms, 4),
        "eager_wall_ms_per_step": round(eager_wall_ms, 4),
        "draft_train_step_tok_s": None,
        "draft_c5": None,
        "step_kernels_us": in_step,
        "kernels": kern,
        "ks3_c4_kernels": None if args.no_ks3 else ks3_kernel_times(dev, args.kernel_reps),
        "rosa_c4_kernels": None if args.no_rosa else rosa_kernel_times(dev, args.kernel_reps),
        "lmhead_c3": None if args.no_c3 else lmhead_c3_times(dev, 3),
        "ln_quant_c4": None if args.no_ln else ln_quant_times(dev, args.kernel_reps),
        "roofline": {
            "kernel": "ksd::g128::gemm_g128_kernel<f32> (the step's GEMM launches: the forward, "
                      "and dX + dW paired; ops over their summed durations inside the step, "
                      "HIP events between the step's launches)",
            "bound": "mfma",
            "achieved": round(achieved / 1e12, 1),
            "peak": PEAK_INT8 / 1e12,
            "unit": "TOPS",
            "frac": round(achieved / PEAK_INT8, 4),
            "traffic": traffic,
            "traffic_source": tsrc,
            "avg_launch_us": round(step_gemm_us / 2, 3),
            "ops_per_launch": round(1.5 * GEMM_OPS),
        },
    }
    if not args.no_c5:
        torch.cuda.empty_cache()
        # the headline step: every linear INT8, live gradients (loss scale 2^12)
        out["draft_c5"] = draft_c5(dev, args.c5_steps, 1, args.c5_loss_scale)
        out["draft_train_step_tok_s"] = out["draft_c5"]["tok_per_s"]
        torch.cuda.empty_cache()
        # beside it: the unscaled loss, whose gradients mostly quantize to zero codes
        out["draft_c5_unscaled"] = draft_c5(dev, args.c5_steps, 1, 1.0)
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(xc, wc, dyc, args.cpu_seconds)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
