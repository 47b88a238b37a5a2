"""DraftBlock — Rosa mixer, DSpine injection, KS3 (mirror of reference
ksdraft/model/block.py:24-42):

    h     = x + Rosa(LN_attn(x))
    h, p  = AdjacentInjection(h, p_prev_layer)
    y     = h + KS3(LN_ffn(h))

Both residual adds are passed to the mixer and the cell as ``residual=``: the INT8 surfaces
add them in their output GEMM's store, the float ones add them after. On the GPU each
pre-norm is kernels.draft.ResidualLayerNorm, whose backward also takes the residual
branch's gradient (one pass instead of LayerNorm's backward plus autograd's add).
"""

from __future__ import annotations

import torch
from torch import nn

from .ks3 import KS3
from .rosa import RosaMixer
from .spine import AdjacentInjection


class DraftBlock(nn.Module):
    def __init__(self, config, layer: int):
        super().__init__()
        d = config.d_model
        self.layer = layer
        self.ln_attn = nn.LayerNorm(d)
        self.rosa = RosaMixer(d, config.rosa_streams, config.rosa_bits)
        self.injection = AdjacentInjection(d)
        self.ln_ffn = nn.LayerNorm(d)
        self.ffn = KS3(d, config.ks3_charts or None)

    @staticmethod
    def _norm(ln: nn.LayerNorm, x: torch.Tensor):
        """(ln(x), x as the residual operand)."""
        if (x.is_cuda and x.dtype == torch.float32 and x.shape[-1] % 256 == 0
                and x.shape[-1] <= 2048 and ln.elementwise_affine
                and ln.weight.dtype == torch.float32 and torch.is_grad_enabled()):
            from ..kernels.draft import ResidualLayerNorm
            return ResidualLayerNorm.apply(x.contiguous(), ln.weight, ln.bias, ln.eps)
        return ln(x), x

    def forward(self, x: torch.Tensor, prev_layer_feature: torch.Tensor | None = None):
        # the two residual adds ride in the output projections' stores (INT8 surfaces)
        y, res = self._norm(self.ln_attn, x)
        h = self.rosa(y, residual=res)
        h, feature = self.injection(h, prev_layer_feature)
        y, res = self._norm(self.ln_ffn, h)
        return self.ffn(y, residual=res), feature
