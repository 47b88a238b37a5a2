"""CPU oracle for KSDraft's INT8 tier — TEST INFRASTRUCTURE, NOT PRODUCT CODE.

A restatement, in numpy and plain C (``ksd_oracle.c``), of the reference's arithmetic
for the hot path (reference ksdraft/kernels/{quant,gemm,linear,ks3_int8}.py,
ksdraft/model/rosa.py, ksdraft/kernels/rosa_credit_gpu.py). Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import it, and
only as the checker (or the timed CPU baseline) — never as the thing measured or
shipped. ``ksdraft_amd`` never imports it and has no CPU fallback.

Every function cites the reference file:line it restates. How each one is pinned
(reference known-answer tests, closed forms, brute force, exact rational arithmetic)
is stated in its docstring and exercised by tests/test_oracle_*.py.
"""
