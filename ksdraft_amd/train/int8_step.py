"""The INT8 draft training step: the reference trainer's step
(ksdraft/train/__init__.py:145-174) on a ``to_int8(model, trainable=True)`` model.

    logits-free loss:  ce = LinearCrossEntropyInt8(output_norm(stream), tied head)
                       ts = mean over layers of 1 - cos(feature, embedding[next token])
                       loss = ce + transfer_weight * ts          (distillation_losses, :65-99)
    backward           every linear INT8 (Int8Linear / KS3Int8Cell / the head's GEMMs)
    clip               the clip_grad_norm_ factor as a device scalar: applied on load by the
                       int8 optimizer kernel, by one multi-tensor multiply for the rest
    optimizer          AdamWRequant: torch AdamW's update fused with the int8 repack of every
                       registered Int8Linear master (the head's codes included)

The teacher-KL term needs teacher top-k signals, which config 5 does not have (a synthetic
teacher hidden state drives only the ``teacher_proj`` seam); it is not part of this step.
Nothing in the step reads a value back to the host except the loss check of the
cross-entropy targets.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from ..kernels.ks3_int8 import KS3Int8Cell
from ..kernels.linear import Int8Linear
from . import IGNORE_INDEX, AdamWRequant, LinearCrossEntropyInt8


def clip_coefficient(params, max_norm: float, loss_scale: float = 1.0) -> torch.Tensor:
    """The factor torch.nn.utils.clip_grad_norm_ multiplies every gradient by:
    min(1, max_norm / (||g||_2 + 1e-6)) over all gradients, as a 1-element device tensor.
    The per-tensor norms are one multi-tensor launch (torch._foreach_norm), as in
    clip_grad_norm_'s own foreach path.

    loss_scale: the gradients hold loss_scale * g (a power of two, so the scaling and the
    norm's division by it are exact); the factor returned then applies the unscaling too:
    min(1, max_norm / (||g|| + 1e-6)) / loss_scale."""
    grads = [p.grad for p in params if p.grad is not None]
    norms = torch._foreach_norm(grads, 2.0)
    total = torch.linalg.vector_norm(torch.stack(norms))
    if loss_scale != 1.0:
        total = total / loss_scale
    coef = torch.clamp(max_norm / (total + 1e-6), max=1.0)
    if loss_scale != 1.0:
        coef = coef / loss_scale
    return coef.reshape(1)


def _check_loss_scale(s: float) -> float:
    s = float(s)
    m, e = math.frexp(s)
    if not (s > 0 and m == 0.5):
        raise ValueError(f"loss_scale must be a positive power of two, got {s}")
    return s


def transfer_space_loss(features, embedding_weight: torch.Tensor, tgt: torch.Tensor,
                        sparse_row_grad: bool = False):
    """distillation_losses' transfer term (train/__init__.py:79-85). On the GPU the
    per-layer cosines and their gradients are two HIP row kernels per layer
    (kernels.draft.TransferSpaceLoss); the normalized target embeddings stay torch ops.
    sparse_row_grad: the gather embedding_weight[tgt] returns its row gradients as a sparse
    gradient, which autograd adds into the tied head's dense one (the same values as the
    dense embedding backward), instead of a dense (V, d) gradient."""
    if sparse_row_grad and embedding_weight.requires_grad:
        from ..kernels.embedding import gather_rows_sparse_grad
        rows = gather_rows_sparse_grad(embedding_weight, tgt)
    else:
        rows = embedding_weight[tgt]
    tgt_emb = F.normalize(rows.float(), dim=-1)
    if tgt_emb.is_cuda and len(features) and all(f.is_cuda for f in features):
        from ..kernels.draft import TransferSpaceLoss
        d = tgt_emb.shape[-1]
        return TransferSpaceLoss.apply(tgt_emb.reshape(-1, d), *features)
    ts = 0.0
    for f in features:
        ts = ts + (1 - (F.normalize(f.float(), dim=-1) * tgt_emb).sum(-1)).mean()
    return ts / max(1, len(features))


class Int8DraftTrainer:
    """One optimizer step per ``step(tokens, teacher_states)`` on an INT8 draft model.

    tokens (B, T + 1): inputs tokens[:, :-1], targets tokens[:, 1:] (train/__init__.py:152).
    The model must come from ``to_int8(model, trainable=True)`` (its head is an Int8Linear
    tied to the embedding).

    loss_scale (a power of two, default 1): backward runs on loss_scale * loss and the
    optimizer step divides it out again (through the clip factor). The int8 gradient
    operands are per-group symmetric codes, so scaling by a power of two leaves every code
    unchanged wherever the group's fp16 scale stays a normal number, and gives codes to the
    groups whose scale would otherwise clamp to the 2^-24 minimum and round to zero (a
    mean loss over 8192 tokens at random init has most vocabulary groups of the logits'
    gradient near 1e-9)."""

    def __init__(self, model, lr: float = 3e-4, betas=(0.9, 0.999), eps: float = 1e-8,
                 weight_decay: float = 0.01, grad_clip: float = 1.0,
                 transfer_weight: float = 0.5, loss_scale: float = 1.0):
        if not isinstance(getattr(model, "head", None), Int8Linear):
            raise ValueError("Int8DraftTrainer needs to_int8(model, trainable=True)")
        self.model = model
        self.grad_clip = grad_clip
        self.transfer_weight = transfer_weight
        self.loss_scale = _check_loss_scale(loss_scale)
        self.opt = AdamWRequant(model.parameters(), lr=lr, betas=betas, eps=eps,
                                weight_decay=weight_decay)
        for mod in model.modules():
            if isinstance(mod, Int8Linear) or (isinstance(mod, KS3Int8Cell) and mod.trainable):
                self.opt.register_int8(mod)
        # the float embedding's lookups return sparse row gradients, which autograd adds
        # into the tied head's dense dW
        model.sparse_embedding_grad = True

    def loss(self, tokens: torch.Tensor, teacher_states: torch.Tensor | None = None):
        """(loss, ce, transfer) as device tensors, with the graph for backward."""
        model = self.model
        inp, tgt = tokens[:, :-1], tokens[:, 1:]
        h, features = model.backbone(inp, teacher_states)
        ts = transfer_space_loss(features, model.embedding.weight, tgt, sparse_row_grad=True)
        head = model.head
        if not head._codes_current():
            head._quantize_weight()
        ce = LinearCrossEntropyInt8.apply(h, head.weight, head.weight_codes, head.weight_scales,
                                          tgt.reshape(-1), IGNORE_INDEX, 128, head.current_transpose())
        return ce + self.transfer_weight * ts, ce, ts

    def backward(self, loss: torch.Tensor):
        """Gradients of loss_scale * loss (the scale is exact: a power of two)."""
        self.opt.zero_grad(set_to_none=True)
        (loss * self.loss_scale if self.loss_scale != 1.0 else loss).backward()

    def optimizer_step(self):
        coef = clip_coefficient(self.model.parameters(), self.grad_clip, self.loss_scale)
        self.opt.step(clip_coef=coef)

    def step(self, tokens: torch.Tensor, teacher_states: torch.Tensor | None = None):
        self.model.train()
        loss, ce, ts = self.loss(tokens, teacher_states)
        self.backward(loss)
        self.optimizer_step()
        return loss.detach(), ce.detach(), ts.detach()
