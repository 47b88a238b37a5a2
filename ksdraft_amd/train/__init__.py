"""Training-side helpers the INT8 kernels call (reference ksdraft/train).

Cross entropy over the LM head's logits, ``F.cross_entropy(logits, tgt)`` of reference
ksdraft/train/__init__.py:77, with its gradient delivered straight as the two int8 operand
layouts of the int8 head backward (dY per token along the vocabulary for dX = dY.W, dY^T
per vocabulary row along the tokens for dW = dY^T.X; the recipe of
ksdraft/kernels/ks3_int8.py:403-424). The fp32 dY is never written.
"""

from __future__ import annotations

import torch

from .. import _lib
from ..kernels.gemm import w8a8_gemm, w8a8_gemm_out, w8a8_gemm_pair
from ..kernels.linear import w8a8_linear_forward_train
from ..kernels.quant import GROUP_SIZE, SCALE_DTYPE, requant_transpose, requant_transpose_multi

IGNORE_INDEX = -100  # torch.nn.functional.cross_entropy's default


def _check_logits(logits: torch.Tensor, targets: torch.Tensor, ignore_index: int,
                  check_targets: bool = True):
    dev = _lib.require_gpu(logits, targets)
    if logits.dim() != 2 or logits.dtype != torch.float32:
        raise ValueError("cross entropy expects 2-D float32 logits (rows, classes)")
    if targets.dim() != 1 or targets.shape[0] != logits.shape[0]:
        raise ValueError(f"targets of shape {tuple(targets.shape)} do not match logits "
                         f"{tuple(logits.shape)}")
    if targets.dtype != torch.int64:
        raise TypeError("targets must be int64 class indices")
    if check_targets:  # torch raises for such targets too (a host sync)
        C = logits.shape[1]
        bad = ((targets < 0) & (targets != ignore_index)) | (targets >= C)
        if bool(bad.any()):
            t = int(targets[bad][0])
            raise IndexError(f"Target {t} is out of bounds.")
    return dev


def cross_entropy_stats(logits: torch.Tensor, targets: torch.Tensor,
                        ignore_index: int = IGNORE_INDEX, check_targets: bool = True):
    """One read of the logits: (loss, row_max, row_inv_sum, n_counted).

    loss is the mean over counted rows of log(sum exp(y)) - y[t] (a 0-d fp32 tensor, NaN
    when no row counts, as torch gives); row_max / row_inv_sum feed the backward.
    ``check_targets=False`` skips the range check and its host sync (for graph capture):
    the kernels then treat an out-of-range target as an ignored row."""
    dev = _check_logits(logits, targets, ignore_index, check_targets)
    logits = logits.contiguous()
    targets = targets.contiguous()
    R, C = logits.shape
    rmax = torch.empty(R, dtype=torch.float32, device=dev)
    rinv = torch.empty(R, dtype=torch.float32, device=dev)
    rloss = torch.empty(R, dtype=torch.float32, device=dev)
    _lib.call("ksd_ce_row_stats", logits.data_ptr(), R, C, targets.data_ptr(), int(ignore_index),
              rmax.data_ptr(), rinv.data_ptr(), rloss.data_ptr(), _lib.stream_ptr(dev))
    # the rows the kernels count: a target in range and not ignored (with check_targets
    # off, an out-of-range target is an ignored row for the kernels, so it is for n too)
    C = logits.shape[1]
    n = ((targets != ignore_index) & (targets >= 0) & (targets < C)).sum().to(torch.float32)
    return rloss.sum() / n, rmax, rinv, n


def cross_entropy_grad_int8(logits: torch.Tensor, targets: torch.Tensor, row_max: torch.Tensor,
                            row_inv_sum: torch.Tensor, grad_scale: torch.Tensor,
                            ignore_index: int = IGNORE_INDEX, group: int = GROUP_SIZE,
                            return_dy: bool = False):
    """d(loss)/d(logits) = (softmax(y) - onehot(t)) * grad_scale, quantized in both layouts.

    grad_scale: a 1-element fp32 device tensor (the upstream gradient over the number of
    counted rows). Returns (codes (R, C), scales (R, C/group), codes_t (C, R), scales_t
    (C, R/group)) and, with ``return_dy``, the fp32 dY the codes were made from."""
    dev = _lib.require_gpu(logits, targets, row_max, row_inv_sum, grad_scale)
    if group != GROUP_SIZE:
        raise ValueError(f"the fused cross-entropy gradient supports group {GROUP_SIZE} only")
    logits = logits.contiguous()
    targets = targets.contiguous()
    R, C = logits.shape
    gsc = grad_scale.to(device=dev, dtype=torch.float32).reshape(1).contiguous()
    codes = torch.empty((R, C), dtype=torch.int8, device=dev)
    scales = torch.empty((R, -(-C // group)), dtype=SCALE_DTYPE, device=dev)
    codes_t = torch.empty((C, R), dtype=torch.int8, device=dev)
    scales_t = torch.empty((C, -(-R // group)), dtype=SCALE_DTYPE, device=dev)
    # shapes off the fused path (C % 8 != 0) stage dY in an fp32 buffer
    dy = torch.empty((R, C), dtype=torch.float32, device=dev) if (return_dy or C % 8) else None
    _lib.call("ksd_ce_backward_quant_dual", logits.data_ptr(), R, C, row_max.data_ptr(),
              row_inv_sum.data_ptr(), targets.data_ptr(), int(ignore_index), gsc.data_ptr(),
              group, codes.data_ptr(), scales.data_ptr(), codes_t.data_ptr(), scales_t.data_ptr(),
              0 if dy is None else dy.data_ptr(), _lib.stream_ptr(dev))
    out = (codes, scales, codes_t, scales_t)
    return (out, dy) if return_dy else out


def cross_entropy_int8(logits: torch.Tensor, targets: torch.Tensor,
                       ignore_index: int = IGNORE_INDEX, grad_output: float = 1.0,
                       group: int = GROUP_SIZE, return_dy: bool = False):
    """F.cross_entropy(logits, targets) and its int8 logits gradient in one call.

    Returns (loss, (codes, scales, codes_t, scales_t)) [, dy]."""
    loss, rmax, rinv, n = cross_entropy_stats(logits, targets, ignore_index)
    gsc = torch.as_tensor(grad_output, dtype=torch.float32, device=logits.device) / n
    res = cross_entropy_grad_int8(logits, targets, rmax, rinv, gsc, ignore_index, group, return_dy)
    if return_dy:
        ops, dy = res
        return loss, ops, dy
    return loss, res


class LinearCrossEntropyInt8(torch.autograd.Function):
    """loss = F.cross_entropy(W8A8(x, W), t) for the bias-free LM head of reference
    ksdraft/model/draft.py:39, 82 with the loss of ksdraft/train/__init__.py:77.

    Forward: the int8 head GEMM (fp32 logits) and the row statistics. Backward: the fused
    cross-entropy gradient in both int8 layouts, then dX = dY.W and dW = dY^T.X on the int8
    GEMMs. Returns fp32 gradients for x (in x's dtype) and the fp32 master weight."""

    @staticmethod
    def forward(ctx, x, weight, wq, ws, targets, ignore_index, group, wt=None):
        """wt: (codes_t, scales_t) = requant_transpose(wq, ws) when the caller has it."""
        K = x.shape[-1]
        x2 = x.reshape(-1, K)
        y, xtq, xts = w8a8_linear_forward_train(x2, wq, ws, None, group, torch.float32)
        loss, rmax, rinv, n = cross_entropy_stats(y, targets.reshape(-1), ignore_index)
        ctx.save_for_backward(y, rmax, rinv, n, targets.reshape(-1), xtq, xts, wq, ws)
        ctx.ignore_index, ctx.group, ctx.x_shape, ctx.x_dtype = ignore_index, group, x.shape, x.dtype
        ctx.wt = wt
        return loss

    @staticmethod
    def backward(ctx, grad_loss):
        y, rmax, rinv, n, t, xtq, xts, wq, ws = ctx.saved_tensors
        group = ctx.group
        gsc = grad_loss.to(torch.float32).reshape(1) / n
        gq, gs, gtq, gts = cross_entropy_grad_int8(y, t, rmax, rinv, gsc, ctx.ignore_index, group)
        dx = dw = None
        out = ctx.x_dtype if ctx.x_dtype in (torch.bfloat16, torch.float16) else torch.float32
        if ctx.needs_input_grad[0]:
            wtq, wts = ctx.wt if ctx.wt is not None else requant_transpose(wq, ws, group, group)
        if ctx.needs_input_grad[0] and ctx.needs_input_grad[1]:  # one launch for both
            dx, dw = w8a8_gemm_pair((gq, gs, wtq, wts, out), (gtq, gts, xtq, xts, torch.float32),
                                    group)
            dx = dx.reshape(ctx.x_shape)
        elif ctx.needs_input_grad[0]:
            dx = w8a8_gemm_out(gq, gs, wtq, wts, group, out_dtype=out).reshape(ctx.x_shape)
        elif ctx.needs_input_grad[1]:
            dw = w8a8_gemm(gtq, gts, xtq, xts, group)
        return dx, dw, None, None, None, None, None, None


def adamw_requant_(param: torch.Tensor, grad: torch.Tensor, exp_avg: torch.Tensor,
                   exp_avg_sq: torch.Tensor, step: int, lr: float, betas=(0.9, 0.999),
                   eps: float = 1e-8, weight_decay: float = 1e-2,
                   clip_coef: torch.Tensor | None = None, quantize: bool = True,
                   group: int = GROUP_SIZE):
    """One torch.optim.AdamW step (decoupled weight decay, amsgrad off, step already
    incremented to ``step``) on an fp32 master in place, fused with the int8 repack of the
    updated master (quantize_last_dim along the last dim, as Int8Linear._quantize_weight of
    reference ksdraft/kernels/linear.py:46-56 does on every call).

    clip_coef: optional 1-element fp32 device tensor, the factor clip_grad_norm_ would
    multiply the gradient by (the gradient itself is read, not rewritten). Returns (codes,
    scales) of the updated master, or None when ``quantize`` is False."""
    dev = _lib.require_gpu(param, grad, exp_avg, exp_avg_sq, clip_coef)
    for name, t in (("param", param), ("grad", grad), ("exp_avg", exp_avg), ("exp_avg_sq", exp_avg_sq)):
        if t.dtype != torch.float32 or not t.is_contiguous():
            raise ValueError(f"adamw_requant_: {name} must be a contiguous float32 tensor")
        if t.shape != param.shape:
            raise ValueError(f"adamw_requant_: {name} shape {tuple(t.shape)} != {tuple(param.shape)}")
    if group != GROUP_SIZE:
        raise ValueError(f"adamw_requant_ supports group {GROUP_SIZE} only")
    beta1, beta2 = betas
    K = param.shape[-1] if param.dim() >= 1 else 1
    rows = param.numel() // max(K, 1)
    # torch's python-double scalars, rounded to fp32 by the kernel's arguments
    bc1 = 1 - beta1 ** step
    bc2 = 1 - beta2 ** step
    codes = scales = None
    if quantize:
        codes = torch.empty(param.shape, dtype=torch.int8, device=dev)
        scales = torch.empty((*param.shape[:-1], -(-K // group)), dtype=SCALE_DTYPE, device=dev)
    cc = None if clip_coef is None else clip_coef.to(dtype=torch.float32).reshape(1).contiguous()
    _lib.call("ksd_adamw_requant", param.data_ptr(), grad.data_ptr(), exp_avg.data_ptr(),
              exp_avg_sq.data_ptr(), rows, K, 0 if cc is None else cc.data_ptr(),
              1 - lr * weight_decay, 1 - beta1, beta2, 1 - beta2, eps, lr / bc1, bc2 ** 0.5,
              group, 0 if codes is None else codes.data_ptr(),
              0 if scales is None else scales.data_ptr(), _lib.stream_ptr(dev))
    return None if codes is None else (codes, scales)


# KsdAdamTensor of the C ABI: six pointers, rows and K, the two per-master step scalars
_ADAM_TENSOR = None


def _adam_tensor_dtype():
    global _ADAM_TENSOR
    if _ADAM_TENSOR is None:
        import numpy as np
        _ADAM_TENSOR = np.dtype([("param", "<u8"), ("grad", "<u8"), ("exp_avg", "<u8"),
                                 ("exp_avg_sq", "<u8"), ("codes", "<u8"), ("scales", "<u8"),
                                 ("rows", "<i8"), ("K", "<i8"), ("step_size", "<f4"),
                                 ("bc2_sqrt", "<f4")])
        assert _ADAM_TENSOR.itemsize == 72
    return _ADAM_TENSOR


def adamw_requant_multi_(items, lr: float, betas=(0.9, 0.999), eps: float = 1e-8,
                         weight_decay: float = 1e-2, clip_coef: torch.Tensor | None = None,
                         group: int = GROUP_SIZE):
    """adamw_requant_ over many masters in a few launches (ksd_adamw_requant_multi).

    items: (param, grad, exp_avg, exp_avg_sq, step, quantize) per master, all fp32,
    contiguous, on one device; step is that master's incremented step count. Returns one
    (codes, scales) or None per item, as adamw_requant_ would."""
    import numpy as np
    if not items:
        return []
    if group != GROUP_SIZE:
        raise ValueError(f"adamw_requant_multi_ supports group {GROUP_SIZE} only")
    dev = _lib.require_gpu(*[t for it in items for t in it[:4]], clip_coef)
    beta1, beta2 = betas
    arr = np.zeros(len(items), dtype=_adam_tensor_dtype())
    out = []
    for i, (param, grad, exp_avg, exp_avg_sq, step, quantize) in enumerate(items):
        for name, t in (("param", param), ("grad", grad), ("exp_avg", exp_avg), ("exp_avg_sq", exp_avg_sq)):
            if t.dtype != torch.float32 or not t.is_contiguous() or t.shape != param.shape:
                raise ValueError(f"adamw_requant_multi_: {name} of item {i} must be a contiguous "
                                 f"float32 tensor of the param's shape")
        K = param.shape[-1] if param.dim() >= 1 else 1
        rows = param.numel() // max(K, 1)
        codes = scales = None
        if quantize:
            codes = torch.empty(param.shape, dtype=torch.int8, device=dev)
            scales = torch.empty((*param.shape[:-1], -(-K // group)), dtype=SCALE_DTYPE, device=dev)
        out.append(None if codes is None else (codes, scales))
        arr[i] = (param.data_ptr(), grad.data_ptr(), exp_avg.data_ptr(), exp_avg_sq.data_ptr(),
                  0 if codes is None else codes.data_ptr(), 0 if scales is None else scales.data_ptr(),
                  rows, K, lr / (1 - beta1 ** step), (1 - beta2 ** step) ** 0.5)
    cc = None if clip_coef is None else clip_coef.to(dtype=torch.float32).reshape(1).contiguous()
    _lib.call("ksd_adamw_requant_multi", arr.ctypes.data, len(items), 0 if cc is None else cc.data_ptr(),
              1 - lr * weight_decay, 1 - beta1, beta2, 1 - beta2, eps, group, _lib.stream_ptr(dev))
    return out


class AdamWRequant(torch.optim.Optimizer):
    """torch.optim.AdamW (the optimizer of reference ksdraft/train/__init__.py:114-116,
    amsgrad off) whose step also repacks int8 weights.

    Same hyper-parameters and per-parameter state ("step", "exp_avg", "exp_avg_sq") as
    torch's AdamW. ``register_int8(module)`` attaches an Int8Linear-like module: after each
    step its ``weight_codes`` / ``weight_scales`` hold quantize_last_dim of the updated
    fp32 master, from the same pass over the weight. ``step(clip_coef=...)`` takes the
    factor of clip_grad_norm_ as a device tensor instead of rescaling every gradient."""

    def __init__(self, params, lr: float = 1e-3, betas=(0.9, 0.999), eps: float = 1e-8,
                 weight_decay: float = 1e-2):
        if lr < 0 or eps < 0 or weight_decay < 0 or not (0 <= betas[0] < 1 and 0 <= betas[1] < 1):
            raise ValueError("invalid AdamW hyper-parameter")
        super().__init__(params, dict(lr=lr, betas=tuple(betas), eps=eps, weight_decay=weight_decay))
        self._int8 = {}
        self._steps = {}  # id(param) -> step count as a python int (no tensor read per step)

    def register_int8(self, module) -> None:
        """After each step the module's codes are those of its updated master. The module
        then skips its own per-call requantization until its master changes; a write to
        the master through ``.data`` (which torch does not version) must be followed by
        ``module.invalidate_codes()``. Accepts an Int8Linear (its ``weight``) or a
        trainable KS3Int8Cell (its ``master_down`` and ``master_up``, whose codes the
        cell's forward repack would otherwise rebuild every call)."""
        if hasattr(module, "master_down"):
            for name in ("down", "up"):
                self._int8[id(getattr(module, "master_" + name))] = (module, name)
        else:
            self._int8[id(module.weight)] = (module, None)
        module._codes_owner = self

    # parameters at least this large take the fused one-pass kernel; smaller ones (norms,
    # biases, gate vectors) are batched into torch's multi-tensor AdamW
    FUSED_MIN_NUMEL = 1 << 16
    # after the step, the registered masters' transposed codes (dX's operand) for modules in
    # training mode, built in a few launches rather than one per layer in the backward
    build_transposes = True

    @torch.no_grad()
    def step(self, closure=None, clip_coef: torch.Tensor | None = None):
        """One AdamW step. Registered Int8Linear masters and the other large fp32 parameters
        go through the fused update (+ int8 repack for the registered ones) kernel, a few
        launches for the whole group (clip_coef applied on load); every other parameter
        goes through torch's own multi-tensor AdamW (torch.optim.adamw with foreach), after
        one multi-tensor multiply by clip_coef, as clip_grad_norm_ does."""
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        from torch.optim.adamw import adamw as torch_adamw
        for group in self.param_groups:
            fl = ([], [], [], [], [])  # params, grads, exp_avg, exp_avg_sq, steps
            fused, regs = [], []
            for p in group["params"]:
                if p.grad is None:
                    continue
                st = self.state[p]
                if not st:
                    st["step"] = torch.tensor(0.0)
                    st["exp_avg"] = torch.zeros_like(p, memory_format=torch.preserve_format)
                    st["exp_avg_sq"] = torch.zeros_like(p, memory_format=torch.preserve_format)
                reg = self._int8.get(id(p))
                if reg is None and (p.numel() < self.FUSED_MIN_NUMEL or p.dtype != torch.float32
                                    or not p.is_contiguous() or not p.grad.is_contiguous()):
                    for lst, v in zip(fl, (p, p.grad, st["exp_avg"], st["exp_avg_sq"], st["step"])):
                        lst.append(v)
                    continue
                n = self._steps.get(id(p))
                if n is None:  # first step, or state loaded from a state_dict (a CPU tensor)
                    n = int(st["step"])
                n += 1
                self._steps[id(p)] = n
                st["step"].fill_(float(n))  # torch's AdamW state layout: a CPU scalar tensor
                fused.append((p, p.grad.contiguous(), st["exp_avg"], st["exp_avg_sq"], n, reg is not None))
                regs.append(reg)
            results = adamw_requant_multi_(fused, group["lr"], group["betas"], group["eps"],
                                           group["weight_decay"], clip_coef)
            tpairs, towners = [], []
            for (p, *_), reg, res in zip(fused, regs, results):
                if reg is None:
                    continue
                # the codes now belong to the master as it is
                mod, name = reg
                key = (p.data_ptr(), p._version)
                if name is None:
                    mod.weight_codes, mod.weight_scales = res
                    mod._codes_key = key
                else:
                    setattr(mod, name + "_codes", res[0])
                    setattr(mod, name + "_scales", res[1])
                    mod._master_codes_keys[name] = key
                if self.build_transposes and mod.training and res[0].dim() == 2:
                    tpairs.append(res)
                    towners.append((mod, name, res[0]))
            # the dX operands W^T of the next backward, for all masters in a few launches
            for (mod, name, codes), wt in zip(towners, requant_transpose_multi(tpairs)):
                if name is None:
                    mod._wt, mod._wt_src = wt, codes
                else:
                    if getattr(mod, "_master_t", None) is None:
                        mod._master_t = {}
                    mod._master_t[name] = (wt, codes)
            if fl[0]:
                if clip_coef is not None:
                    torch._foreach_mul_(fl[1], clip_coef.reshape(()).to(fl[1][0].dtype))
                beta1, beta2 = group["betas"]
                torch_adamw(fl[0], fl[1], fl[2], fl[3], [], fl[4], foreach=True,
                            amsgrad=False, beta1=beta1, beta2=beta2, lr=group["lr"],
                            weight_decay=group["weight_decay"], eps=group["eps"],
                            maximize=False)
        return loss

    def load_state_dict(self, state_dict):
        super().load_state_dict(state_dict)
        self._steps.clear()
