"""Decoder hyper-parameters (internal/config/config.go:31-49)."""
from __future__ import annotations

from dataclasses import dataclass, field


@dataclass(frozen=True)
class DecoderConfig:
    hidden: int
    inter: int
    layers: int
    heads: int
    kv_heads: int
    head_dim: int
    vocab: int
    eps: float = 1e-6          # config.go:80 default
    rope_theta: float = 10000  # config.go:77 default
    mrope_section: tuple = field(default=(16, 24, 24))  # model.go:882 default

    @property
    def q_rows(self) -> int:
        return self.heads * self.head_dim

    @property
    def kv_rows(self) -> int:
        return self.kv_heads * self.head_dim


# The 0.3B ERNIE text decoder the benchmarks are quoted on: 18 layers, hidden
# 1024, 16 query heads / 2 KV heads of 128, SwiGLU 3072, vocab 103424,
# RMSNorm eps 1e-5, RoPE theta 500000.
ERNIE_0P3B = DecoderConfig(hidden=1024, inter=3072, layers=18, heads=16, kv_heads=2, head_dim=128, vocab=103424,
                           eps=1e-5, rope_theta=500000.0)
