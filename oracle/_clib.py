"""Build and load liboracle.so (ksd_oracle.c) with gcc. Test infrastructure only."""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "ksd_oracle.c")
LIB = os.path.join(HERE, "liboracle.so")

CFLAGS = ["-O2", "-fopenmp", "-ffp-contract=off", "-fPIC", "-shared", "-std=c11"]


def build() -> str:
    tmp = LIB + ".tmp"
    res = subprocess.run(["gcc", *CFLAGS, "-o", tmp, SRC, "-lm"],
                         capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"gcc failed building the oracle:\n{res.stderr}")
    os.replace(tmp, LIB)
    return LIB


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB) or os.path.getmtime(LIB) < os.path.getmtime(SRC):
            build()
        _lib = ctypes.CDLL(LIB)
        P, I64, I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        _lib.ksd_check_div127.argtypes = [ctypes.c_uint32, ctypes.c_uint32]
        _lib.ksd_check_div127.restype = ctypes.c_uint64
        _lib.ksd_half_to_float.argtypes = [ctypes.c_uint16]
        _lib.ksd_half_to_float.restype = ctypes.c_float
        _lib.ksd_oracle_partials.argtypes = [P, P, I64, I64, I64, I, P]
        _lib.ksd_oracle_partials.restype = None
        _lib.ksd_oracle_gemm_ordered.argtypes = [P, P, P, P, I64, I64, I64, I, P, P, I64, I, P]
        _lib.ksd_oracle_gemm_ordered.restype = None
        _lib.ksd_oracle_rosa_match.argtypes = [P, P, P, I64, I64, I, P, P, P]
        _lib.ksd_oracle_rosa_match.restype = None
        _lib.ksd_oracle_rosa_credits.argtypes = [P, P, P, P, I64, I64, I, P]
        _lib.ksd_oracle_rosa_credits.restype = None
    return _lib


def ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)
