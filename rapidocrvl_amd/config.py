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


def load_config_json(path: str) -> dict:
    """config.Load (internal/config/config.go:51-84): config.json of a model
    directory (or the file itself) with the loader's defaults — head_dim =
    hidden/heads, kv heads = heads, rope_theta 10000, rms_norm_eps 1e-6."""
    import json
    import os

    if os.path.isdir(path):
        path = os.path.join(path, "config.json")
    if os.path.getsize(path) > 16 << 20:
        raise ValueError(f"config.json too large: {path}")
    with open(path, "rb") as f:
        raw = f.read()

    def no_dups(pairs):
        keys = [k for k, _ in pairs]
        if len(set(keys)) != len(keys):
            raise ValueError(f"{path}: duplicate key")
        return dict(pairs)

    c = json.loads(raw, object_pairs_hook=no_dups)
    if not c.get("head_dim") and c.get("num_attention_heads"):
        c["head_dim"] = c.get("hidden_size", 0) // c["num_attention_heads"]
    if not c.get("num_key_value_heads"):
        c["num_key_value_heads"] = c.get("num_attention_heads", 0)
    c["rope_theta"] = c.get("rope_theta") or 10000.0
    c["rms_norm_eps"] = c.get("rms_norm_eps") or 1e-6
    return c


def decoder_config(c: dict) -> DecoderConfig:
    """The decoder's hyper-parameters from a loaded config.json; the rotary
    sections come from rope_scaling.mrope_section when present
    (initTextRoPE, internal/model/model.go:877-885)."""
    sections = ((c.get("rope_scaling") or {}).get("mrope_section") or (16, 24, 24))
    return DecoderConfig(hidden=c["hidden_size"], inter=c["intermediate_size"], layers=c["num_hidden_layers"],
                         heads=c["num_attention_heads"], kv_heads=c["num_key_value_heads"], head_dim=c["head_dim"],
                         vocab=c["vocab_size"], eps=float(c["rms_norm_eps"]), rope_theta=float(c["rope_theta"]),
                         mrope_section=tuple(sections))
