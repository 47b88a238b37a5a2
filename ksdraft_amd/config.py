"""Draft model shape (mirror of reference ksdraft/config.py:36-110).

The fields and parameter formulas the model and the INT8 tier read: vocabulary, depth,
width, Rosa streams and bits, KS3 charts (0 means round(d_model * 368 / 96),
config.py:79-83). The per-layer counts follow config.py:71-91: Rosa 4ds + 4d + 4s, KS3
c(2d + 6) + 2c, and the tied embedding V * d.
"""

from __future__ import annotations

from dataclasses import dataclass

VALID_DTYPES = ("int8", "bf16", "fp32")
KS3_CHARTS_PER_WIDTH = 368 / 96


@dataclass
class KSDraftConfig:
    vocab_size: int = 150_144
    layers: int = 24
    d_model: int = 1792
    head_size: int = 64
    rosa_streams: int = 597
    rosa_bits: int = 1
    ks3_charts: int = 0
    block_len: int = 16
    anchor_stride: int = 64
    dtype: str = "int8"
    tie_word_embeddings: bool = True

    def __post_init__(self) -> None:
        if self.dtype not in VALID_DTYPES:
            raise ValueError(f"dtype must be one of {VALID_DTYPES}, got {self.dtype!r}")
        if not 1 <= self.rosa_bits <= 64:
            raise ValueError("rosa_bits must be in [1, 64] (Rosa packed symbol width)")

    @property
    def n_heads(self) -> int:
        return self.d_model // self.head_size

    @property
    def charts(self) -> int:
        return self.ks3_charts or round(self.d_model * KS3_CHARTS_PER_WIDTH)

    def rosa_params(self) -> int:
        d, s = self.d_model, self.rosa_streams
        return 4 * d * s + 4 * d + 4 * s

    def ks3_params(self) -> int:
        d, c = self.d_model, self.charts
        return c * (2 * d + 6) + 2 * c

    def layer_params(self) -> int:
        return self.rosa_params() + self.ks3_params()

    def embedding_params(self) -> int:
        n = self.vocab_size * self.d_model
        return n if self.tie_word_embeddings else 2 * n

    def total_params(self) -> int:
        return self.layers * self.layer_params() + self.embedding_params()


def baseline_config() -> KSDraftConfig:
    """The BASELINE config-5 draft: 24 layers, d 1536, 512 streams, 5888 charts."""
    return KSDraftConfig(vocab_size=150_144, layers=24, d_model=1536, rosa_streams=512,
                         ks3_charts=5888)
