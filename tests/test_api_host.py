"""Host logic of the ksdraft_amd.kernels API (CPU only): the reference's error
conditions and classes fire before any device work, and the package refuses CPU
tensors instead of falling back to a CPU path."""

import pytest
import torch

from ksdraft_amd.kernels import quant, gemm


def test_quantize_rejects_integer_input():
    # reference quant.py:39-40
    with pytest.raises(TypeError):
        quant.quantize_last_dim(torch.zeros(2, 128, dtype=torch.int32))


def test_no_cpu_fallback():
    with pytest.raises(RuntimeError, match="GPU only"):
        quant.quantize_last_dim(torch.zeros(2, 128))


def test_gemm_validation_matches_reference():
    a = torch.zeros(4, 256, dtype=torch.int8)
    s = torch.zeros(4, 2, dtype=torch.float16)
    # gemm.py:62-63
    with pytest.raises(ValueError, match="K mismatch"):
        gemm.w8a8_gemm(a, s, torch.zeros(3, 128, dtype=torch.int8), s[:3, :1])
    # gemm.py:64-67
    with pytest.raises(ValueError, match="scale group mismatch"):
        gemm.w8a8_gemm(a, s, a, s[:, :1])
    # gemm.py:69-70
    with pytest.raises(ValueError, match="exceeds"):
        gemm.w8a8_gemm(a, s[:, :1], a, s[:, :1])
    with pytest.raises(RuntimeError, match="GPU only"):
        gemm.w8a8_gemm(a, s, a, s)


def test_padded_length():
    assert quant._padded_length(100) == 128
    assert quant._padded_length(256, 32) == 256
    assert quant.GROUP_SIZE == 128 and quant.SCALE_DTYPE == torch.float16


def test_layer_norm_quantize_host_checks():
    # argument checks fire before any device work; CPU tensors are refused
    with pytest.raises(TypeError):
        quant.layer_norm_quantize(torch.zeros(2, 128, dtype=torch.int32))
    with pytest.raises(ValueError, match="group 128"):
        quant.layer_norm_quantize(torch.zeros(2, 128), group=64)
    with pytest.raises(ValueError, match="d <= 4096"):
        quant.layer_norm_quantize(torch.zeros(2, 4097))
    with pytest.raises(RuntimeError, match="GPU only"):
        quant.layer_norm_quantize(torch.zeros(2, 128))
