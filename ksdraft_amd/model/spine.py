"""DSpine gated adjacent injection (mirror of reference ksdraft/model/spine.py:38-68).

    p_t  = feature_up(feature_down(z_t))                 this layer's predicted feature
    g_t  = sigmoid(gate_q(z_t) + gate_p(p_{t-1}) + b)
    z'_t = z_t + g_t * inject(p_{t-1})

with p_{-1} = 0, or position 0 seeded from the previous layer's prediction. The gates and
the injection are low-rank pairs (rank 32; the feature pair rank 64) whose up-projections
start at zero. ``to_int8`` keeps these surfaces in float (the reference's conversion
doctrine, int8_convert.py:1-16): at rank 32/64 the reduction is shorter than one 128-wide
quantization group. On the GPU the float injection runs as one autograd function
(kernels.draft.FusedInjection: the gated update in one HIP pass, p_prev never
materialised, split-K weight gradients); on the CPU, as torch ops.
"""

from __future__ import annotations

import torch
from torch import nn
import torch.nn.functional as F


class _LowRank(nn.Module):
    def __init__(self, width: int, rank: int):
        super().__init__()
        self.down = nn.Linear(width, rank, bias=False)
        self.up = nn.Linear(rank, width, bias=False)
        nn.init.zeros_(self.up.weight)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.up(self.down(x))


class AdjacentInjection(nn.Module):
    fused = True  # GPU, fp32: kernels.draft.FusedInjection (False: the torch composition)

    def __init__(self, width: int, rank: int = 32, feature_rank: int = 64):
        super().__init__()
        self.width = width
        self.feature_down = nn.Linear(width, feature_rank, bias=False)
        self.feature_up = nn.Linear(feature_rank, width, bias=False)
        self.gate_q = _LowRank(width, rank)
        self.gate_p = _LowRank(width, rank)
        self.gate_bias = nn.Parameter(torch.zeros(width))
        self.inject = _LowRank(width, rank)

    def extra_repr(self) -> str:
        return f"width={self.width}"

    def _use_fused(self, z: torch.Tensor) -> bool:
        ranks = (self.gate_q.down.out_features, self.gate_p.down.out_features,
                 self.inject.down.out_features)
        return (self.fused and z.is_cuda and z.dim() == 3 and z.dtype == torch.float32
                and ranks == (32, 32, 32)
                and all(p.dtype == torch.float32 for p in self.parameters()))

    def predicted_feature(self, z: torch.Tensor) -> torch.Tensor:
        return self.feature_up(self.feature_down(z))

    def forward(self, z: torch.Tensor, prev_layer_feature: torch.Tensor | None = None):
        """(z', p): the injected stream and this layer's predicted feature.

        The low-rank maps that read the same input run as one GEMM with their weights
        stacked (z: feature_down and gate_q.down; p_prev: gate_p.down and inject.down),
        and gate_q(z) + gate_p(p_prev) as one GEMM over the concatenated rank: the same
        sums as spine.py:62-68, in one pass over each (M, d) operand instead of two."""
        if not isinstance(self.feature_down, nn.Linear):
            # INT8 surfaces (to_int8(int8_injection=True)): each low-rank map is its own
            # W8A8 GEMM, composed as spine.py:62-68 writes it
            p = self.predicted_feature(z)
            p_prev = F.pad(p, (0, 0, 1, 0))[:, :-1, :]
            if prev_layer_feature is not None:
                p_prev = torch.cat([prev_layer_feature[:, :1, :], p_prev[:, 1:, :]], dim=1)
            gate = torch.sigmoid(self.gate_q(z) + self.gate_p(p_prev) + self.gate_bias)
            return z + gate * self.inject(p_prev), p
        if self._use_fused(z):
            from ..kernels.draft import FusedInjection
            prev0 = None if prev_layer_feature is None else prev_layer_feature[:, :1, :]
            return FusedInjection.apply(
                z.contiguous(), prev0, self.feature_down.weight, self.gate_q.down.weight,
                self.feature_up.weight, self.gate_p.down.weight, self.inject.down.weight,
                self.gate_q.up.weight, self.gate_p.up.weight, self.gate_bias,
                self.inject.up.weight)
        r1 = self.feature_down.out_features
        zd = F.linear(z, torch.cat([self.feature_down.weight, self.gate_q.down.weight]))
        p = self.feature_up(zd[..., :r1])
        p_prev = F.pad(p, (0, 0, 1, 0))[:, :-1, :]
        if prev_layer_feature is not None:
            p_prev = torch.cat([prev_layer_feature[:, :1, :], p_prev[:, 1:, :]], dim=1)
        r2 = self.gate_p.down.out_features
        pd = F.linear(p_prev, torch.cat([self.gate_p.down.weight, self.inject.down.weight]))
        pre = F.linear(torch.cat([zd[..., r1:], pd[..., :r2]], dim=-1),
                       torch.cat([self.gate_q.up.weight, self.gate_p.up.weight], dim=1),
                       self.gate_bias)
        return z + torch.sigmoid(pre) * self.inject.up(pd[..., r2:]), p
