"""The C-ABI library loads and exports every symbol include/*.h declares (CPU only).

Argument-validation paths return before any HIP call, so they are exercised here with
null device pointers; no compute runs without a GPU."""

import ctypes
import glob
import os
import re

import pytest
import torch  # noqa: F401  (binds libamdhip64 first, as the package does)

from ksdraft_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_symbols():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        src = open(h).read()
        src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
        names.update(re.findall(r"\b(ksd_\w+)\s*\(", src))
    return sorted(names)


def test_header_declares_entry_points():
    names = _declared_symbols()
    assert "ksd_w8a8_gemm_nt" in names and "ksd_quantize_lastdim" in names


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in _declared_symbols():
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, f"{name} has no ctypes prototype"


def test_abi_version_and_error_channel():
    lib = _lib.load()
    assert lib.ksd_abi_version() == 2
    rc = lib.ksd_quantize_lastdim(None, 0, 4, 128, 128, 48, None, None, None, 0.0, None)
    assert rc == 1
    buf = ctypes.create_string_buffer(256)
    lib.ksd_last_error(buf, 256)
    assert b"group" in buf.value


def test_validation_paths_without_gpu():
    lib = _lib.load()
    # K not a multiple of 128
    assert lib.ksd_w8a8_gemm_nt(None, None, None, None, 4, 4, 100, 128, None, None, 0, None) == 1
    # bad group
    assert lib.ksd_w8a8_gemm_nt(None, None, None, None, 4, 4, 128, 16, None, None, 0, None) == 1
    # bad dtype reaches the type check only on a valid shape; empty shapes are no-ops
    assert lib.ksd_quantize_lastdim(None, 9, 0, 128, 128, 128, None, None, None, 0.0, None) == 0
    assert lib.ksd_requant_transpose(None, None, 4, 4, 128, 24, None, None, None) == 1
    with pytest.raises(ValueError):
        _lib.call("ksd_w8a8_gemm_nt", None, None, None, None, 4, 4, 100, 128, None, None, 0, None)


def test_ks3_validation_paths_without_gpu():
    lib = _lib.load()
    nrb = ctypes.c_int64(-1)
    assert lib.ksd_ks3_vjp_row_blocks(300, ctypes.byref(nrb)) == 0 and nrb.value == 1
    assert lib.ksd_ks3_vjp_row_blocks(1025, ctypes.byref(nrb)) == 0 and nrb.value == 3
    assert lib.ksd_ks3_vjp_row_blocks(0, ctypes.byref(nrb)) == 0 and nrb.value == 0
    # bad group; null inputs; partials sized for the wrong block count
    assert lib.ksd_ks3_spine_fwd(None, 4, 4, None, None, None, None, None, 48,
                                 None, None, None, None, None) == 1
    assert lib.ksd_ks3_spine_fwd(None, 4, 4, None, None, None, None, None, 128,
                                 None, None, None, None, None) == 1
    assert lib.ksd_ks3_spine_fused(None, 4, 4, None, None, None, None, None, 128,
                                   None, None, None, None) == 1
    # a table workspace that is missing or misaligned is rejected before any launch
    q = ctypes.c_void_p(24)
    assert lib.ksd_ks3_spine_fwd(q, 4, 4, q, q, q, q, ctypes.c_void_p(16), 128,
                                 None, q, q, ctypes.c_void_p(8), None) == 1
    lib.ksd_last_error(buf := ctypes.create_string_buffer(256), 256)
    assert b"table" in buf.value
    p = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    assert lib.ksd_ks3_vjp(p, p, 300, 8, p, p, p, p, 128, None, None, None, None, None,
                           p, 2, None) == 1
    buf = ctypes.create_string_buffer(256)
    lib.ksd_last_error(buf, 256)
    assert b"row blocks" in buf.value
    assert lib.ksd_ks3_vjp_finalize(None, 1, 8, None, None, None, None, None, None, None) == 1
    assert lib.ksd_ks3_tanh16(None, 4, None, None) == 1
    # the one-launch projection: group 128 only, aligned operands, a table, K > 0
    a = ctypes.c_void_p(256)
    assert lib.ksd_ks3_project_fused(a, p, a, p, 64, 256, 128, p, p, p, p, q, 32,
                                     p, p, a, None) == 1
    lib.ksd_last_error(buf, 256)
    assert b"group 128" in buf.value
    assert lib.ksd_ks3_project_fused(a, p, a, p, 64, 256, 128, p, p, p, p, q, 128,
                                     p, p, None, None) == 1
    lib.ksd_last_error(buf, 256)
    assert b"table" in buf.value
    assert lib.ksd_ks3_project_fused(a, p, a, p, 64, 256, 0, p, p, p, p, q, 128,
                                     p, p, a, None) == 1
    lib.ksd_last_error(buf, 256)
    assert b"K = 0" in buf.value
    assert lib.ksd_ks3_project_fused(ctypes.c_void_p(8), p, a, p, 64, 256, 128, p, p, p, p, q,
                                     128, p, p, a, None) == 1  # A not 16-byte aligned
    assert lib.ksd_ks3_project_fused(a, p, a, p, 0, 256, 128, p, p, p, p, q, 128,
                                     p, p, a, None) == 0  # empty: nothing to launch


def test_single_hip_runtime_in_process():
    _lib.load()
    maps = open("/proc/self/maps").read()
    hips = {line.split()[-1] for line in maps.splitlines() if "libamdhip64" in line}
    assert len(hips) == 1, hips
