"""ctypes binding of libksdraft_amd.so (declared in include/ksdraft_amd.h).

The library is built in-tree by ``python -m ksdraft_amd.build``. torch is imported first
so that the library's ``libamdhip64.so.7`` dependency binds to the HIP runtime torch
already loaded (same SONAME): device pointers and hipStream_t handles are then shared.

There is no CPU or eager fallback: a missing library or a CPU tensor raises.
"""

from __future__ import annotations

import ctypes
import os

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libksdraft_amd.so")

# element type codes (KSD_F32 ... in include/ksdraft_amd.h)
F32, BF16, F16, F16_SAT = 0, 1, 2, 3
_DTYPE_CODE = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16}

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_INT = ctypes.c_int
_F = ctypes.c_float

# name -> argtypes (every symbol the header declares)
SIGNATURES = {
    "ksd_abi_version": [],
    "ksd_last_error": [ctypes.c_char_p, ctypes.c_size_t],
    "ksd_quantize_lastdim": [_P, _INT, _I64, _I64, _I64, _INT, _P, _P, _P, _F, _P],
    "ksd_dequantize_lastdim": [_P, _P, _I64, _I64, _I64, _INT, _P, _P],
    "ksd_quantize_transpose": [_P, _INT, _I64, _I64, _INT, _P, _P, _P],
    "ksd_requant_transpose": [_P, _P, _I64, _I64, _INT, _INT, _P, _P, _P],
    "ksd_quantize_dual": [_P, _INT, _I64, _I64, _INT, _INT, _P, _P, _P, _P, _P],
    "ksd_quantize_dual2": [_P, _I64, _I64, _P, _P, _P, _P, _P, _I64, _I64, _P, _P, _P, _P, _INT, _INT, _P],
    "ksd_quantize_dual_colsum": [_P, _INT, _I64, _I64, _INT, _P, _P, _P, _P, _P, _P, _I64, _P],
    "ksd_ce_row_stats": [_P, _I64, _I64, _P, _I64, _P, _P, _P, _P],
    "ksd_ce_backward_quant_dual": [_P, _I64, _I64, _P, _P, _P, _I64, _P, _INT, _P, _P, _P, _P, _P, _P],
    "ksd_adamw_requant": [_P, _P, _P, _P, _I64, _I64, _P, _F, _F, _F, _F, _F, _F, _F, _INT, _P, _P, _P],
    "ksd_adamw_requant_multi": [_P, _INT, _P, _F, _F, _F, _F, _F, _INT, _P],
    "ksd_requant_transpose_multi": [_P, _INT, _INT, _P],
    "ksd_layernorm_quant": [_P, _INT, _I64, _I64, _I64, _P, _P, _F, _INT, _P, _P, _P, _P, _P, _P],
    "ksd_embedding_gather_int8": [_P, _P, _P, _I64, _I64, _I64, _INT, _P, _INT, _P],
    "ksd_w8a8_gemm_nt": [_P, _P, _P, _P, _I64, _I64, _I64, _INT, _P, _P, _INT, _P],
    "ksd_w8a8_gemm_splits": [_I64, _I64, _I64, _INT, _P],
    "ksd_w8a8_gemm_nt_ws": [_P, _P, _P, _P, _I64, _I64, _I64, _INT, _P, _P, _INT, _P, _I64, _P],
    "ksd_w8a8_gemm_nt_ex": [_P, _P, _P, _P, _I64, _I64, _I64, _INT, _P, _P, _P, _INT, _P, _I64, _P],
    "ksd_w8a8_gemm_pair": [_P, _P, _P, _P, _I64, _I64, _I64, _P, _INT, _P, _P, _P, _P, _I64, _I64, _I64,
                           _P, _INT, _P, _I64, _P],
    "ksd_w8a8_group_partials": [_P, _P, _I64, _I64, _I64, _INT, _P, _P],
    "ksd_ks3_spine_fwd": [_P, _I64, _I64, _P, _P, _P, _P, _P, _INT, _P, _P, _P, _P, _P],
    "ksd_ks3_spine_fwd_noalloc": [_P, _I64, _I64, _P, _P, _P, _P, _P, _INT, _P, _P, _P, _P],
    "ksd_ks3_spine_fused": [_P, _I64, _I64, _P, _P, _P, _P, _P, _INT, _P, _P, _P, _P],
    "ksd_ks3_project_fused": [_P, _P, _P, _P, _I64, _I64, _I64, _P, _P, _P, _P, _P, _INT, _P, _P, _P,
                              _P],
    "ksd_ks3_spine_float": [_P, _INT, _I64, _I64, _P, _P, _P, _P, _INT, _INT, _P, _P, _P, _P],
    "ksd_ks3_vjp_row_blocks": [_I64, _P],
    "ksd_ks3_vjp": [_P, _P, _I64, _I64, _P, _P, _P, _P, _INT,
                    _P, _P, _P, _P, _P, _P, _I64, _P],
    "ksd_ks3_vjp_finalize": [_P, _I64, _I64, _P, _P, _P, _P, _P, _P, _P],
    "ksd_ks3_tanh16": [_P, _I64, _P, _P],
    "ksd_grad_handoff": [_P, _I64, _P, _P, _P],
    "ksd_rosa_shift_quant": [_P, _INT, _I64, _I64, _I64, _P, _P, _P, _INT,
                             _P, _P, _P, _P, _P, _P, _P],
    "ksd_rosa_shift_quant_dual": [_P, _INT, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _P, _P],
    "ksd_rosa_shift_backward_blocks": [_I64, _I64, _P],
    "ksd_rosa_shift_backward": [_P, _INT, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _P, _P, _P],
    "ksd_rosa_pack_bits": [_P, _INT, _I64, _I64, _I64, _P, _P],
    "ksd_rosa_pack_bits3": [_P, _P, _P, _INT, _I64, _I64, _I64, _P, _P, _P, _P],
    "ksd_transfer_cos": [_P, _P, _I64, _I64, _P, _P, _P],
    "ksd_transfer_grad": [_P, _P, _P, _P, _P, _I64, _I64, _P, _P, _INT, _P],
    "ksd_injection_update": [_P, _P, _P, _P, _P, _I64, _I64, _P, _P],
    "ksd_layernorm_backward_blocks": [_I64, _P],
    "ksd_layernorm_backward": [_P, _P, _P, _P, _P, _P, _I64, _I64, _P, _P, _P],
    "ksd_injection_update_backward": [_P, _P, _P, _P, _P, _I64, _I64, _P, _P, _P],
    "ksd_rosa_match": [_P, _P, _P, _I64, _I64, _INT, _P, _P, _P],
    "ksd_rosa_hard": [_P, _P, _I64, _I64, _I64, _P, _INT, _P],
    "ksd_rosa_credits": [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _INT, _P, _P, _P, _P],
    "ksd_rosa_credit_grads": [_P, _P, _P, _P, _INT, _P, _I64, _I64, _I64,
                              _P, _P, _P, _P, _P],
}

_lib = None


class KernelLibraryMissing(RuntimeError):
    pass


def load() -> ctypes.CDLL:
    """Load (once) and return the kernel library, with prototypes set."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise KernelLibraryMissing(
            f"{LIB_PATH} is not built; run `python -m ksdraft_amd.build` "
            "(ksdraft_amd has no CPU fallback)")
    lib = ctypes.CDLL(LIB_PATH)
    for name, args in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = ctypes.c_int
    _lib = lib
    return lib


_ERRORS = {1: ValueError, 2: TypeError, 3: RuntimeError}


def check(status: int) -> None:
    if status == 0:
        return
    buf = ctypes.create_string_buffer(512)
    load().ksd_last_error(buf, 512)
    raise _ERRORS.get(status, RuntimeError)(buf.value.decode(errors="replace"))


def call(name: str, *args) -> None:
    check(getattr(load(), name)(*args))


def require_gpu(*tensors: torch.Tensor) -> torch.device:
    """All tensors must live on one HIP device; returns it."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(
                "ksdraft_amd kernels run on the GPU only (no CPU path); got a tensor on "
                f"{t.device}")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} and {t.device}")
    if dev is None:
        raise RuntimeError("no tensor given")
    return dev


def stream_ptr(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dtype]
    except KeyError:
        raise TypeError(f"unsupported floating dtype {dtype}") from None
