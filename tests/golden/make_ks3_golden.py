"""Write golden vectors for the KS3 int8 cell from the reference implementation.

Run in the build container only (the reference is not present on GPU boxes):

    python tests/golden/make_ks3_golden.py /root/reference

It pins the two functions nothing else fixes at the bit level: the int8-mode spine
features (reference ksdraft/kernels/ks3_int8.py:205-234, whose fp16 rounding follows
torch's per-op opmath conventions) and the fp16 geometry VJP of
_KS3Int8Train.backward (ks3_int8.py:341-401). The reference's own CPU path is run on a
small seeded cell; its intermediates are captured by wrapping its quantize / GEMM
functions and recorded as plain arrays (npz, no pickles). Only data is committed.
"""

from __future__ import annotations

import os
import sys

import numpy as np
import torch

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "ks3_int8_golden.npz")


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    import ksdraft.kernels.ks3_int8 as K
    from ksdraft.model.ks3 import KS3

    torch.manual_seed(1234)
    d, F, M = 128, 256, 64
    cell = KS3(d, F)
    with torch.no_grad():
        cell.up.weight.normal_(0, 0.05)
        cell.coefficients.normal_(0, 0.3)
        cell.raw_scale.add_(torch.randn(F) * 0.3)
        cell.raw_shift.normal_(0, 0.5)
    q = K.KS3Int8Cell(cell, group=128, nonlinear="int8", trainable=True)

    rec = {"quant_in": [], "gemm_out": [], "spine": []}
    orig_q, orig_g = K.quantize_last_dim, K.w8a8_gemm

    def q_rec(x, group=128):
        rec["quant_in"].append(x.detach().clone())
        return orig_q(x, group)

    def g_rec(*a, **k):
        y = orig_g(*a, **k)
        rec["gemm_out"].append(y.detach().clone())
        return y

    orig_spine = q._spine_features

    def spine_rec(*args):
        out = orig_spine(*args)
        rec["spine"].append((args[0].detach().clone(), out.detach().clone()))
        return out

    K.quantize_last_dim, K.w8a8_gemm = q_rec, g_rec
    q._spine_features = spine_rec
    try:
        cases = {}
        for name, xscale in (("std1", 1.0), ("std8", 8.0)):
            for k in rec:
                rec[k].clear()
            g = torch.Generator().manual_seed(7 if name == "std1" else 8)
            x = (torch.randn(M, d, generator=g) * xscale).requires_grad_(True)
            grad_out = torch.randn(M, d, generator=g) * 0.1
            for p in q.parameters():
                p.grad = None
            y = q(x)
            n_fwd_q = len(rec["quant_in"])
            y.backward(grad_out)
            coords, h = rec["spine"][0]
            bq = rec["quant_in"][n_fwd_q:]
            cases[name] = {
                "x": x.detach().numpy(),
                "coords": coords.reshape(M, F).numpy(),   # fp32 holding fp16 values
                "h": h.reshape(M, F).numpy(),              # spine output (fp32)
                "y": y.detach().numpy(),
                "grad_out": grad_out.numpy(),
                "value": rec["gemm_out"][2].to(torch.float16).numpy(),  # backward GEMM 1 -> fp16
                "dc": bq[2].numpy(),                        # 3rd backward quantize input
                "dx": x.grad.numpy(),
                "ddown": q.master_down.grad.half().numpy(),   # fp16 view (inf where the
                                                              # reference handed off fp32)
                "dup": q.master_up.grad.half().numpy(),
                "dcoeff": q.master_coefficients.grad.float().numpy(),
                "dscale": q.master_raw_scale.grad.float().numpy(),
                "dshift": q.master_raw_shift.grad.float().numpy(),
            }
    finally:
        K.quantize_last_dim, K.w8a8_gemm = orig_q, orig_g

    arrays = {
        "master_down": q.master_down.detach().numpy(),
        "master_up": q.master_up.detach().numpy(),
        "master_coefficients": q.master_coefficients.detach().numpy(),
        "master_raw_scale": q.master_raw_scale.detach().numpy(),
        "master_raw_shift": q.master_raw_shift.detach().numpy(),
        "spine_codes": q.spine_codes.numpy(), "spine_scale": q.spine_scale.numpy(),
        "warp_scale_codes": q.warp_scale_codes.numpy(),
        "warp_scale_scales": q.warp_scale_scales.numpy(),
        "warp_shift_codes": q.warp_shift_codes.numpy(),
        "warp_shift_scales": q.warp_shift_scales.numpy(),
        "tanh_lut": q.tanh_lut.numpy(),
    }
    for name, c in cases.items():
        for k, v in c.items():
            arrays[f"{name}/{k}"] = v
    np.savez_compressed(OUT, **arrays)
    print("wrote", OUT, {k: v.shape for k, v in arrays.items() if k.startswith("std1/")})


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
