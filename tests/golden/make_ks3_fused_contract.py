"""Record how Triton compiles the reference's fused KS3 kernel for AMD targets.

Run in the build container only (the reference is not present on GPU boxes):

    python tests/golden/make_ks3_fused_contract.py /root/reference

The reference's _fused_gemm_spine (ksdraft/kernels/ks3_triton.py:100-156, with the spine
helpers at :32-97) is compiled by the installed Triton for ("hip", "gfx950", 64), the
MI355X, and ("hip", "gfx1100", 32), the reference's development GPU, once per nonlinear
mode (NL 0 'fp32', 1 'fp16', 2 'int8'). Nothing is run: the kernel cannot execute here.
What the source text leaves to the backend is which multiply/add pairs Triton's default
enable_fp_fusion contracts into one fused multiply-add, and how `/` is lowered. The AMD
assembly answers both: every instruction carries the `.loc` source line of
ks3_triton.py it came from (inlined helpers included).

The fixture records, per target, mode and source line of ks3_triton.py, the count of each
floating-point VALU opcode (encoding suffixes such as _e32/_e64/_sdwa dropped) and the
literal and inline constants that line's floating-point and move instructions use. Only this
data is committed (tests/golden/ks3_fused_contract.json); the oracle's fused contract is
checked against it in tests/test_oracle_fused_contract.py.
"""

from __future__ import annotations

import collections
import json
import os
import re
import sys

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "ks3_fused_contract.json")
TARGETS = [("gfx950", 64), ("gfx1100", 32)]
# a small shape with every compile-time branch of the kernel live (two chart groups, a
# ragged row tile is not needed: the arithmetic does not depend on M, N, K)
SHAPE = {"M": 64, "N": 256, "K": 256, "G": 128, "NSCALE": 2, "BM": 16, "BN": 128, "BK": 128}
FP_OP = re.compile(r"^v_(pk_)?(fma|fmac|fmamk|fmaak|mul|add|sub|subrev|div|rcp|fma_mix|fma_mixlo|"
                   r"fma_mixhi|mac|mad|max|min|med3|rndne|trunc|cvt|ldexp|exp|log|sqrt)")


def _norm(op: str) -> str:
    return re.sub(r"_(e32|e64|sdwa|dpp|e64_dpp)$", "", op)


def _parse(asm: str, src_file: str):
    """opcode counts and constants per source line of `src_file` (by .file index)."""
    files = {}
    cur = None
    ops = collections.defaultdict(collections.Counter)
    consts = collections.defaultdict(set)
    for raw in asm.splitlines():
        s = raw.split(";")[0].strip()
        m = re.match(r"\.file\s+(\d+)\s+\"([^\"]*)\"\s+\"([^\"]*)\"", s)
        if m:
            files[int(m.group(1))] = os.path.join(m.group(2), m.group(3))
            continue
        m = re.match(r"\.loc\s+(\d+)\s+(\d+)\s+(\d+)", s)
        if m:
            cur = (int(m.group(1)), int(m.group(2)))
            continue
        if not s or s.startswith(".") or s.endswith(":") or cur is None:
            continue
        if not files.get(cur[0], "").endswith(src_file):
            continue
        parts = s.split(None, 1)
        op = _norm(parts[0])
        if not (FP_OP.match(op) or op.startswith(("s_mov", "v_mov"))):
            continue
        if FP_OP.match(op):
            ops[cur[1]][op] += 1
        if len(parts) > 1:
            for c in re.findall(r"0x[0-9a-fA-F]+|(?<![\w.])-?\d+\.\d+(?![\w.])", parts[1]):
                consts[cur[1]].add(c.lower())
    return ops, consts


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    import triton
    from triton.backends.compiler import GPUTarget
    from triton.compiler import ASTSource

    import ksdraft.kernels.ks3_triton as KT

    fn = KT._fused_gemm_spine
    sig = {"A": "*i8", "AS": "*fp16", "W": "*i8", "WS": "*fp16", "H": "*i8", "HS": "*fp16",
           "P": "*i8", "PS": "*fp16", "SC": "*fp16", "SH": "*fp16", "LUT": "*i8"}
    out = {"triton": triton.__version__, "source": "ksdraft/kernels/ks3_triton.py",
           "kernel": "_fused_gemm_spine", "shape": SHAPE, "targets": {}}
    for arch, warp in TARGETS:
        per_mode = {}
        for nl in (0, 1, 2):
            const = dict(SHAPE, NL=nl)
            full_sig = dict(sig, **{k: "constexpr" for k in const})
            src = ASTSource(fn=fn, signature=full_sig,
                            constexprs={(fn.arg_names.index(k),): v for k, v in const.items()})
            k = triton.compile(src, target=GPUTarget("hip", arch, warp), options={"num_warps": 4})
            ops, consts = _parse(k.asm["amdgcn"], "ks3_triton.py")
            per_mode[str(nl)] = {str(ln): {"ops": dict(sorted(ops[ln].items())),
                                           "consts": sorted(consts[ln])}
                                 for ln in sorted(ops)}
        out["targets"][arch] = {"wave": warp, "modes": per_mode}
    with open(OUT, "w") as f:
        json.dump(out, f, indent=1, sort_keys=True)
        f.write("\n")
    print(OUT)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
