"""The float KS3 spine decoder (mirror of reference ksdraft/model/ks3.py:66-117).

It is the float tier of the FFN and the constructor input of ``KS3Int8Cell``: the down/up
projections, the six spine coefficients per chart and the warp's raw scale and shift,
with the reference's initialisation (coefficients ~ N(0, 0.05), raw_scale 0.75, raw_shift
0, down ~ N(0, d**-0.5), up zero so a fresh block is the identity, ks3.py:85-90). The
INT8 tier replaces it with ``KS3Int8Cell`` (``to_int8``); its own forward is the float
reference, evaluated by torch in fp32 (fp64 for a double model).
"""

from __future__ import annotations

import torch
from torch import nn
from torch.nn import functional as F


def spine_horner(t: torch.Tensor, z: torch.Tensor, coefficients: torch.Tensor):
    """ks3.py:33-48: the Hermite cubic in t and the Chebyshev warp in z, nested."""
    p0, p1, p2, p3, p4, p5 = coefficients.unbind(-1)
    cubic = 2.0 * p0 - 2.0 * p1 + p2 + p3
    quadratic = -3.0 * p0 + 3.0 * p1 - 2.0 * p2 - p3
    spine = ((cubic * t + quadratic) * t + p2) * t + p0
    warped = ((4.0 * p5 * z + 2.0 * p4) * z - 3.0 * p5) * z - p4
    return spine, warped


class KS3(nn.Module):
    def __init__(self, d_model: int, num_charts: int | None = None, subspace_rank: int = 1):
        super().__init__()
        charts = num_charts if num_charts is not None else round(d_model * 368 / 96)
        self.d_model = d_model
        self.num_charts = charts
        self.subspace_rank = subspace_rank
        self.features = charts * subspace_rank
        self.down = nn.Linear(d_model, self.features, bias=False)
        self.up = nn.Linear(self.features, d_model, bias=False)
        shape = (charts, 6) if subspace_rank == 1 else (charts, subspace_rank, 6)
        self.coefficients = nn.Parameter(torch.empty(shape))
        self.raw_scale = nn.Parameter(torch.full((charts,), 0.75))
        self.raw_shift = nn.Parameter(torch.zeros(charts))
        nn.init.normal_(self.coefficients, std=0.05)
        nn.init.normal_(self.down.weight, std=d_model ** -0.5)
        nn.init.zeros_(self.up.weight)

    def extra_repr(self) -> str:
        return (f"d_model={self.d_model}, num_charts={self.num_charts}, "
                f"subspace_rank={self.subspace_rank}")

    def warp_scale(self) -> torch.Tensor:
        return F.softplus(self.raw_scale.float()) + 1e-4

    def warp_shift(self) -> torch.Tensor:
        return 0.5 * torch.tanh(self.raw_shift.float())

    def forward(self, x: torch.Tensor, residual: torch.Tensor | None = None) -> torch.Tensor:
        if residual is not None:
            return residual + self.forward(x)
        coords = self.down(x)
        gdt = torch.float64 if coords.dtype == torch.float64 else torch.float32
        h = coords.to(gdt).clamp(-65504.0, 65504.0)
        h = h.reshape(*x.shape[:-1], self.num_charts, self.subspace_rank)
        t = 4.0 * torch.tanh(h.mean(-1, keepdim=True) / 4.0)
        z = torch.tanh(self.warp_scale()[:, None] * (t + self.warp_shift()[:, None]))
        coeffs = self.coefficients.to(gdt).reshape(self.num_charts, self.subspace_rank, 6)
        spine, warped = spine_horner(t, z, coeffs)
        feats = F.relu(h + spine + warped).square()
        return self.up(feats.flatten(-2).to(self.up.weight.dtype))
