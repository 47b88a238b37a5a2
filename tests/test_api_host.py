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


def test_gemm_rejects_scale_rows_that_do_not_match():
    # the kernel reads scale rows by raw stride: a short scale tensor must raise before
    # any launch instead of reading past its allocation
    a = torch.zeros(4, 256, dtype=torch.int8)
    w = torch.zeros(3, 256, dtype=torch.int8)
    sa = torch.zeros(4, 2, dtype=torch.float16)
    sw = torch.zeros(3, 2, dtype=torch.float16)
    with pytest.raises(ValueError, match="a_scales shape"):
        gemm.w8a8_gemm(a, sa[:2], w, sw)
    with pytest.raises(ValueError, match="w_scales shape"):
        gemm.w8a8_gemm(a, sa, w, sw[:1])
    with pytest.raises(RuntimeError, match="GPU only"):
        gemm.w8a8_gemm(a, sa, w, sw)


def test_dequantize_scale_shapes_follow_torch_broadcasting():
    codes = torch.zeros(4, 256, dtype=torch.int8)
    # scale rows that neither match nor broadcast: torch's own broadcasting error class
    with pytest.raises(RuntimeError, match="broadcast|size"):
        quant.dequantize_last_dim(codes, torch.zeros(3, 2, dtype=torch.float16))
    # an explicit group the scales do not cover
    with pytest.raises(RuntimeError, match="broadcast|size"):
        quant.dequantize_last_dim(codes, torch.zeros(4, 2, dtype=torch.float16), group=64)
    # shapes the reference accepts by broadcasting pass the host checks (then need a GPU)
    for sc in (torch.zeros(1, 2), torch.zeros(2), torch.zeros(4, 1)):
        with pytest.raises(RuntimeError, match="GPU only"):
            g = 128 if sc.shape[-1] == 2 else None
            quant.dequantize_last_dim(codes, sc.half(), group=g)


def test_int8_linear_codes_follow_writes_the_optimizer_did_not_make():
    """Codes handed over by AdamWRequant are used only while the master is the one they
    were made from: load_state_dict, .to() and invalidate_codes() drop them (host state
    only; no kernel runs)."""
    from ksdraft_amd.kernels.linear import Int8Linear
    lin = Int8Linear(128, 4, bias=False)
    lin.weight_codes = torch.zeros(4, 128, dtype=torch.int8)
    lin.weight_scales = torch.zeros(4, 1, dtype=torch.float16)
    lin._codes_owner = object()
    lin._codes_key = (lin.weight.data_ptr(), lin.weight._version)
    assert lin._codes_current()
    with torch.no_grad():
        lin.weight.add_(1.0)                      # a versioned in-place write
    assert not lin._codes_current()
    lin._codes_key = (lin.weight.data_ptr(), lin.weight._version)
    lin.weight.data.copy_(torch.ones(4, 128))     # unversioned: needs invalidate_codes()
    lin.invalidate_codes()
    assert not lin._codes_current()
    lin._codes_key = (lin.weight.data_ptr(), lin.weight._version)
    lin.load_state_dict({"weight": torch.full((4, 128), 2.0)})
    assert not lin._codes_current()
    lin._codes_key = (lin.weight.data_ptr(), lin.weight._version)
    lin.to(torch.float32)
    assert not lin._codes_current()
    # a module no optimizer registered never skips its requantization
    lin2 = Int8Linear(128, 4, bias=False)
    lin2.weight_codes, lin2.weight_scales = lin.weight_codes, lin.weight_scales
    lin2._codes_key = (lin2.weight.data_ptr(), lin2.weight._version)
    assert not lin2._codes_current()
