"""KSDraftModel — tied embedding, input norm, DraftBlocks, output norm, tied head
(mirror of reference ksdraft/model/draft.py:25-88).

The optional teacher seam adds ``teacher_proj(teacher_states)`` to the stream after the
input norm (draft.py:73-79). The head is tied to the embedding after any device move
(draft.py:49-51). ``backbone`` returns the output-normed stream that the head projects;
the INT8 training step feeds it to the fused int8 head + cross-entropy instead of
materialising the logits' gradient.
"""

from __future__ import annotations

import torch
from torch import nn

from ..config import KSDraftConfig
from .block import DraftBlock


class KSDraftModel(nn.Module):
    def __init__(self, config: KSDraftConfig | None = None, teacher_dim: int = 0,
                 device: torch.device | str | None = None, skip_init: bool = False):
        super().__init__()
        cfg = config or KSDraftConfig()
        self.config = cfg
        self.teacher_dim = teacher_dim
        self.embedding = nn.Embedding(cfg.vocab_size, cfg.d_model)
        self.input_norm = nn.LayerNorm(cfg.d_model)
        self.blocks = nn.ModuleList([DraftBlock(cfg, i) for i in range(cfg.layers)])
        self.output_norm = nn.LayerNorm(cfg.d_model)
        self.head = nn.Linear(cfg.d_model, cfg.vocab_size, bias=False)
        self.teacher_proj = nn.Linear(teacher_dim, cfg.d_model, bias=False) if teacher_dim else None
        if device is not None:
            self.to(device)
        self.head.weight = self.embedding.weight
        if not skip_init:
            nn.init.uniform_(self.embedding.weight, -1e-4, 1e-4)
            if self.teacher_proj is not None:
                nn.init.zeros_(self.teacher_proj.weight)

    def backbone(self, tokens: torch.Tensor, teacher_states: torch.Tensor | None = None):
        """tokens (B, T) -> (output_norm(stream) (B, T, d), per-layer features)."""
        if getattr(self, "sparse_embedding_grad", False) and type(self.embedding) is nn.Embedding:
            from ..kernels.embedding import gather_rows_sparse_grad
            e = gather_rows_sparse_grad(self.embedding.weight, tokens)
        else:
            e = self.embedding(tokens)
        x = self.input_norm(e)
        if teacher_states is not None:
            if self.teacher_proj is None:
                raise ValueError("teacher_states passed but teacher_dim=0 at construction")
            x = x + self.teacher_proj(teacher_states.to(self.teacher_proj.weight.dtype))
        prev = None
        features = []
        for block in self.blocks:
            x, prev = block(x, prev)
            features.append(prev)
        return self.output_norm(x), features

    def forward(self, tokens: torch.Tensor, teacher_states: torch.Tensor | None = None):
        """tokens (B, T) -> (logits (B, T, V), per-layer transfer features)."""
        h, features = self.backbone(tokens, teacher_states)
        return self.head(h), features

    def param_counts(self) -> dict:
        core = self.config.layers * self.config.layer_params() + self.config.embedding_params()
        extras = sum(p.numel() for p in self.parameters()) - core
        return {"core": core, "extras": extras, "total": core + extras}
