"""Write golden vectors for the KS3 int8 cell's 'fp16' and 'fp32' nonlinear modes.

Run in the build container only (the reference is not present on GPU boxes):

    python tests/golden/make_ks3_modes_golden.py /root/reference

It pins what no other check fixes: the composed spine features of the two float modes
(reference ksdraft/kernels/ks3_int8.py:172-203) on the coordinates the reference itself
materialises, and the composed cell output (_forward_composed, :279-288). The reference's
own CPU path runs on a small seeded cell (rank 1, group 128) at two input scales; the
spine's inputs and outputs are captured by wrapping its _spine_features, and stored as
plain arrays (npz, no pickles). Only data is committed.
"""

from __future__ import annotations

import os
import sys

import numpy as np
import torch

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "ks3_modes_golden.npz")


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    import ksdraft.kernels.ks3_int8 as K
    from ksdraft.model.ks3 import KS3

    torch.manual_seed(4321)
    d, F, M = 128, 256, 48
    cell = KS3(d, F)
    with torch.no_grad():
        cell.up.weight.normal_(0, 0.05)
        cell.coefficients.normal_(0, 0.3)
        cell.raw_scale.add_(torch.randn(F) * 0.3)
        cell.raw_shift.normal_(0, 0.5)
    arrays = {}
    for mode in ("fp16", "fp32"):
        q = K.KS3Int8Cell(cell, group=128, nonlinear=mode).eval()
        rec = []
        orig = q._spine_features

        def spine_rec(*args, orig=orig, rec=rec):
            out = orig(*args)
            rec.append((args[0].detach().clone(), out.detach().clone()))
            return out
        q._spine_features = spine_rec
        for name, xscale in (("std1", 1.0), ("std8", 8.0)):
            rec.clear()
            g = torch.Generator().manual_seed(11 if name == "std1" else 12)
            x = torch.randn(M, d, generator=g) * xscale
            with torch.no_grad():
                y = K.KS3Int8Cell._forward_composed(q, x)
            coords, h = rec[0]
            arrays[f"{mode}/{name}/x"] = x.numpy()
            arrays[f"{mode}/{name}/coords"] = coords.reshape(M, F).numpy()
            arrays[f"{mode}/{name}/h"] = h.reshape(M, F).numpy()
            arrays[f"{mode}/{name}/y"] = y.numpy()
    q = K.KS3Int8Cell(cell, group=128, nonlinear="int8")
    for k in ("down_codes", "down_scales", "up_codes", "up_scales", "spine_codes",
              "spine_scale", "warp_scale_codes", "warp_scale_scales", "warp_shift_codes",
              "warp_shift_scales"):
        arrays[k] = getattr(q, k).numpy()
    for k in ("down", "up"):
        arrays[f"{k}_weight"] = getattr(cell, k).weight.detach().numpy()
    arrays["coefficients"] = cell.coefficients.detach().numpy()
    arrays["raw_scale"] = cell.raw_scale.detach().numpy()
    arrays["raw_shift"] = cell.raw_shift.detach().numpy()
    np.savez_compressed(OUT, **arrays)
    print("wrote", OUT, {k: v.shape for k, v in arrays.items()})


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
