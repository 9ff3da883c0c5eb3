"""Seeded synthetic ERNIE weights and inputs.

Weights are N(0, 0.02) f32, rounded to bf16 (round to nearest even) and read
back as f32 — the exact ``bits<<16`` decode of internal/safetensors
(safetensors.go:776-790) — then row-quantized with the library's own
Q8/Q6/Q4 encoders (the converter path, internal/gguf/convert.go:207-291).
Norm weights are 1 + N(0, 0.02) (bf16-rounded) so activations keep a
realistic scale; the embedding table is N(0, 0.02) bf16.
Each matrix draws from numpy's PCG64 seeded with (seed, layer, role).
"""
from __future__ import annotations

import numpy as np

from . import lib
from .config import DecoderConfig

ROLES = ("q", "k", "v", "o", "gate", "up", "down")
_ROLE_ID = {r: i for i, r in enumerate(ROLES)}


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round f32 to bf16 (nearest, ties to even) and back.  In place on a
    copy in uint32: for every finite f32 the bits plus 0x8000 stay below 2^32."""
    a = np.array(x, dtype=np.float32, copy=True, order="C")
    b = a.view(np.uint32)
    r = (b >> 16) & 1
    r += 0x7FFF
    b += r
    b &= 0xFFFF0000
    return a


def normal(shape, seed, std=0.02):
    rng = np.random.default_rng(seed)
    return bf16_round(rng.standard_normal(shape, dtype=np.float32) * np.float32(std))


def shape_of(cfg: DecoderConfig, role: str):
    return {
        "q": (cfg.q_rows, cfg.hidden), "k": (cfg.kv_rows, cfg.hidden), "v": (cfg.kv_rows, cfg.hidden),
        "o": (cfg.hidden, cfg.q_rows), "gate": (cfg.inter, cfg.hidden), "up": (cfg.inter, cfg.hidden),
        "down": (cfg.hidden, cfg.inter),
    }[role]


def quant_matrix(w, qtype, tie=lib.TIE_HALF_AWAY):
    s, p = lib.quantize_rows(qtype, w, tie)
    return (qtype, s, p, w.shape[1])


def make_weights(cfg: DecoderConfig, qtype: int, seed: int = 0, tie: int = lib.TIE_HALF_AWAY,
                 lm_qtype: int | None = None):
    """dict: layers[i][role] = (qtype, scales, packed, cols), ln1/ln2, lm_head, final_norm, embed."""
    lm_qtype = qtype if lm_qtype is None else lm_qtype
    layers = []
    for li in range(cfg.layers):
        lw = {}
        for role in ROLES:
            w = normal(shape_of(cfg, role), [seed, li, _ROLE_ID[role]])
            lw[role] = quant_matrix(w, qtype, tie)
        lw["ln1"] = bf16_round(1.0 + normal(cfg.hidden, [seed, li, 100]))
        lw["ln2"] = bf16_round(1.0 + normal(cfg.hidden, [seed, li, 101]))
        layers.append(lw)
    lm = normal((cfg.vocab, cfg.hidden), [seed, 1000, 0])
    out = {
        "layers": layers,
        "lm_head": quant_matrix(lm, lm_qtype, tie),
        "final_norm": bf16_round(1.0 + normal(cfg.hidden, [seed, 1000, 1])),
        "embed": normal((cfg.vocab, cfg.hidden), [seed, 1000, 2]),
    }
    return out


_CKPT_ROLE = {"q": "self_attn.q_proj", "k": "self_attn.k_proj", "v": "self_attn.v_proj", "o": "self_attn.o_proj",
              "gate": "mlp.gate_proj", "up": "mlp.up_proj", "down": "mlp.down_proj"}


def make_checkpoint(cfg: DecoderConfig, seed: int = 0) -> dict:
    """The f32 (bf16-exact) tensors ``make_weights`` quantizes, under the
    checkpoint's names (preloadTextWeights, internal/model/model.go:2861-2885);
    converting them reproduces ``make_weights(cfg, q, seed, TIE_AMD64)``."""
    out = {}
    for li in range(cfg.layers):
        pre = f"model.layers.{li}."
        for role in ROLES:
            out[pre + _CKPT_ROLE[role] + ".weight"] = normal(shape_of(cfg, role), [seed, li, _ROLE_ID[role]])
        out[pre + "input_layernorm.weight"] = bf16_round(1.0 + normal(cfg.hidden, [seed, li, 100]))
        out[pre + "post_attention_layernorm.weight"] = bf16_round(1.0 + normal(cfg.hidden, [seed, li, 101]))
    out["lm_head.weight"] = normal((cfg.vocab, cfg.hidden), [seed, 1000, 0])
    out["model.norm.weight"] = bf16_round(1.0 + normal(cfg.hidden, [seed, 1000, 1]))
    out["model.embed_tokens.weight"] = normal((cfg.vocab, cfg.hidden), [seed, 1000, 2])
    return out


def config_json(cfg: DecoderConfig) -> dict:
    """config.json fields of a decoder configuration (internal/config/config.go:31-49)."""
    return {"vocab_size": cfg.vocab, "hidden_size": cfg.hidden, "intermediate_size": cfg.inter,
            "num_hidden_layers": cfg.layers, "num_attention_heads": cfg.heads, "num_key_value_heads": cfg.kv_heads,
            "head_dim": cfg.head_dim, "rms_norm_eps": cfg.eps, "rope_theta": cfg.rope_theta,
            "rope_scaling": {"mrope_section": list(cfg.mrope_section)}, "vision_config": {"num_hidden_layers": 0}}


def prompt_ids(n: int, seed: int = 0, high: int = 100000):
    """Token ids drawn uniformly from [0, high) with the given seed."""
    return np.random.default_rng(seed).integers(0, high, size=n, dtype=np.int64).astype(np.int32)


def image_embeds(n: int, hidden: int, seed: int = 0):
    """Synthetic visual-token rows, N(0, 1) f32."""
    return np.random.default_rng([seed, 7]).standard_normal((n, hidden), dtype=np.float32)
