"""DraftBlock — Rosa mixer, DSpine injection, KS3 (mirror of reference
ksdraft/model/block.py:24-42):

    h     = x + Rosa(LN_attn(x))
    h, p  = AdjacentInjection(h, p_prev_layer)
    y     = h + KS3(LN_ffn(h))

Both residual adds are passed to the mixer and the cell as ``residual=``: the INT8 surfaces
add them in their output GEMM's store, the float ones add them after.
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

    def forward(self, x: torch.Tensor, prev_layer_feature: torch.Tensor | None = None):
        # the two residual adds ride in the output projections' stores (INT8 surfaces)
        h = self.rosa(self.ln_attn(x), residual=x)
        h, feature = self.injection(h, prev_layer_feature)
        return self.ffn(self.ln_ffn(h), residual=h), feature
