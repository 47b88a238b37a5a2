"""Int8 embedding gather (the staged int8-embedding surface of the reference's INT8 tier:
ksdraft/model/int8_convert.py:9-12 keeps the embedding float and names the per-row-scale
int8 embedding as a separate surface).

The table is quantized per row in GS groups along d exactly as the tied head's weight is
(quantize_last_dim, reference ksdraft/kernels/quant.py:30-52), so one set of codes serves
both the head GEMM and the lookup. ``embedding_gather_int8`` returns the looked-up rows
dequantized (code * scale, exact in fp32). ``Int8Embedding`` is an nn.Embedding drop-in
(fp32 master ``weight``) whose backward is the float embedding's: the scatter-add of the
upstream gradient into the master (straight through the quantization).
"""

from __future__ import annotations

import torch
from torch import nn

from .. import _lib
from .quant import GROUP_SIZE, SCALE_DTYPE, quantize_last_dim

_OUT = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16, torch.float16: _lib.F16}


def embedding_gather_int8(codes: torch.Tensor, scales: torch.Tensor, ids: torch.Tensor,
                          group: int = GROUP_SIZE, out_dtype: torch.dtype = torch.float32,
                          check_ids: bool = True) -> torch.Tensor:
    """codes (V, d) int8, scales (V, ceil(d/group)) fp16, ids (...) int -> (..., d)."""
    dev = _lib.require_gpu(codes, scales, ids)
    if codes.dim() != 2 or codes.dtype != torch.int8:
        raise ValueError("codes must be a 2-D int8 table (V, d)")
    V, d = codes.shape
    if scales.dtype != SCALE_DTYPE or scales.shape != (V, -(-d // group)):
        raise ValueError(f"scales must be ({V}, {-(-d // group)}) float16")
    if ids.dtype not in (torch.int64, torch.int32):
        raise TypeError("ids must be integer token indices")
    code = _OUT.get(out_dtype)
    if code is None:
        raise TypeError(f"unsupported output dtype {out_dtype}")
    flat = ids.reshape(-1).to(torch.int64).contiguous()
    if check_ids and flat.numel():  # nn.Embedding raises for such ids (a host sync)
        bad = (flat < 0) | (flat >= V)
        if bool(bad.any()):
            raise IndexError(f"index {int(flat[bad][0])} is out of range for {V} rows")
    out = torch.empty((flat.numel(), d), dtype=out_dtype, device=dev)
    codes, scales = codes.contiguous(), scales.contiguous()  # outlive the enqueued kernel
    _lib.call("ksd_embedding_gather_int8", codes.data_ptr(),
              scales.data_ptr(), flat.data_ptr(), flat.numel(), V, d, group,
              out.data_ptr(), code, _lib.stream_ptr(dev))
    return out.reshape(*ids.shape, d)


class _RowGather(torch.autograd.Function):
    """weight[ids] (F.embedding) whose backward returns a sparse (COO) gradient: the
    upstream rows summed per distinct id, one entry per distinct row.

    A tied weight (embedding lookups beside the LM head) receives a dense gradient from the
    head; autograd adds the sparse row sums into it (one pass over the dense tensor) instead
    of zero-filling and adding a dense (V, d) gradient per lookup. The values are the dense
    embedding backward's: the upstream rows are summed per distinct id by torch's embedding
    backward over a compact table of the distinct ids (sorted, in position order), found
    without a host sync. Slots past the distinct count carry id 0 and zero sums, so adding
    them leaves row 0 unchanged. When the sparse gradient is the weight's only one, its
    .grad is sparse; the caller that uses this lookup (Int8DraftTrainer) always has the
    head's dense gradient on the same weight."""

    @staticmethod
    def forward(ctx, weight, ids):
        ctx.save_for_backward(ids)
        ctx.shape = weight.shape
        return torch.nn.functional.embedding(ids, weight)

    @staticmethod
    def backward(ctx, grad):
        (ids,) = ctx.saved_tensors
        V, d = ctx.shape
        flat = ids.reshape(-1)
        n = flat.numel()
        sid, order = torch.sort(flat, stable=True)
        head = torch.ones(n, dtype=torch.bool, device=flat.device)
        head[1:] = sid[1:] != sid[:-1]
        slot = torch.cumsum(head, 0) - 1
        inv = torch.empty_like(slot)
        inv[order] = slot
        uids = torch.zeros(n, dtype=torch.int64, device=flat.device)
        uids[slot] = sid
        sums = torch.ops.aten.embedding_dense_backward(grad.reshape(-1, d), inv, n, -1, False)
        return torch.sparse_coo_tensor(uids[None], sums, (V, d), check_invariants=False), None


def gather_rows_sparse_grad(weight: torch.Tensor, ids: torch.Tensor) -> torch.Tensor:
    """F.embedding(ids, weight) with a sparse row-sum gradient for ``weight``."""
    return _RowGather.apply(weight, ids)


class _Int8EmbeddingFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, ids, weight, codes, scales, group):
        ctx.save_for_backward(ids)
        ctx.num_weights = weight.shape[0]
        return embedding_gather_int8(codes, scales, ids, group, torch.float32)

    @staticmethod
    def backward(ctx, grad):
        (ids,) = ctx.saved_tensors
        dw = torch.ops.aten.embedding_dense_backward(grad.contiguous(), ids, ctx.num_weights,
                                                     -1, False)
        return None, dw, None, None, None


class Int8Embedding(nn.Module):
    """nn.Embedding(V, d) with an int8 GS128 lookup. The fp32 master ``weight`` stays
    authoritative: the codes are rebuilt every call unless ``codes_from`` (an Int8Linear
    tied to the same weight, e.g. the LM head) holds codes of the master as it is now."""

    def __init__(self, num_embeddings: int, embedding_dim: int, group: int = GROUP_SIZE):
        super().__init__()
        self.num_embeddings = num_embeddings
        self.embedding_dim = embedding_dim
        self.group = group
        self.weight = nn.Parameter(torch.zeros(num_embeddings, embedding_dim))
        self.codes_from = None

    @classmethod
    def from_float(cls, module: nn.Embedding, group: int = GROUP_SIZE) -> "Int8Embedding":
        emb = cls(module.num_embeddings, module.embedding_dim, group)
        emb.weight = module.weight  # the same master (a tied head keeps its tie)
        return emb

    def _codes(self):
        src = self.codes_from
        if (src is not None and src.weight is self.weight and src._codes_current()
                and self.group == GROUP_SIZE):
            return src.weight_codes, src.weight_scales
        return quantize_last_dim(self.weight.detach().float(), self.group)

    def forward(self, ids: torch.Tensor) -> torch.Tensor:
        codes, scales = self._codes()
        return _Int8EmbeddingFunction.apply(ids, self.weight, codes, scales, self.group)
