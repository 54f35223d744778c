"""Model configuration (restates ``TransformerConfig``, ``torch_transformer_benchmark.py:106-133``)."""

from __future__ import annotations

from dataclasses import dataclass


@dataclass(frozen=True)
class TransformerConfig:
    batch_size: int
    seq_len: int
    d_model: int
    num_heads: int
    ffn_dim: int
    num_layers: int
    causal: bool

    def validate(self) -> None:
        """Raise ``ValueError`` for the same conditions as the reference's ``validate``."""
        if self.batch_size <= 0:
            raise ValueError("batch_size must be positive")
        if self.seq_len <= 0:
            raise ValueError("seq_len must be positive")
        if self.d_model <= 0:
            raise ValueError("d_model must be positive")
        if self.num_heads <= 0:
            raise ValueError("num_heads must be positive")
        if self.d_model % self.num_heads != 0:
            raise ValueError(
                f"d_model ({self.d_model}) must be divisible by num_heads ({self.num_heads})"
            )
        if self.ffn_dim <= 0:
            raise ValueError("ffn_dim must be positive")
        if self.num_layers <= 0:
            raise ValueError("num_layers must be positive")

    @property
    def head_dim(self) -> int:
        return self.d_model // self.num_heads

    @property
    def tokens(self) -> int:
        return self.batch_size * self.seq_len


# The five benchmark configurations this build is measured on (all causal).
BENCHMARK_CONFIGS = {
    "cfg1": TransformerConfig(64, 128, 128, 4, 128, 4, True),
    "cfg2": TransformerConfig(64, 1024, 128, 4, 128, 4, True),
    "cfg3": TransformerConfig(128, 256, 32, 2, 64, 2, True),
    "cfg4": TransformerConfig(16, 2048, 512, 8, 2048, 6, True),
    "cfg5": TransformerConfig(512, 4096, 256, 8, 1024, 4, True),
}
