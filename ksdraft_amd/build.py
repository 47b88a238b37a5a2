"""Build libksdraft_amd.so (gfx950 HIP kernels + C ABI) in-tree with hipcc.

Usage: ``python -m ksdraft_amd.build``. The library lands next to this file and is
loaded with ctypes by :mod:`ksdraft_amd._lib` (no torch C++ headers are involved).
"""

from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libksdraft_amd.so")
SOURCES = ["quant.hip", "gemm.hip", "ks3.hip", "rosa.hip", "draft.hip"]
OBJDIR = os.path.join(HERE, "_build")
# generated at build time (git-ignored): fp16 tanh table for the KS3 kernels
TANH_INC = os.path.join(CSRC, "tanh16_table.inc")

ARCH = "gfx950"

# -ffp-contract=off: HIP's default contraction would fuse separately rounded
#   multiply/add pairs of the reference contract; the kernels call fmaf() where an FMA
#   is part of the contract.
# -fhip-fp32-correctly-rounded-divide-sqrt: x/scale must be IEEE division (quant.py:50).
# -packed-fp32-ops off: no v_pk_{add,mul,fma}_f32 anywhere in the library.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-ffp-contract=off", "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if cand and (os.path.sep not in cand or os.path.exists(cand)):
            return cand
    raise RuntimeError("hipcc not found")


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        # hipcc's host pass warns about the device-only target feature; only errors fail
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stderr[-8000:]}")


def build(verbose: bool = False) -> str:
    sys.path.insert(0, CSRC)
    try:
        import gen_tanh16
    finally:
        sys.path.pop(0)
    gen_tanh16.write(TANH_INC)
    os.makedirs(OBJDIR, exist_ok=True)
    objs = [os.path.join(OBJDIR, os.path.splitext(s)[0] + ".o") for s in SOURCES]
    flags = [f for f in HIPCC_FLAGS if f != "-shared"]
    cmds = [[hipcc(), *flags, "-c", "-o", o, os.path.join(CSRC, s)]
            for s, o in zip(SOURCES, objs)]
    with ThreadPoolExecutor(len(cmds)) as ex:
        list(ex.map(lambda c: _run(c, verbose), cmds))
    tmp = LIB + ".tmp"
    _run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs], verbose)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
