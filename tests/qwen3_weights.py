"""Seeded random-init Qwen3 weights shared by the fixture script and the tests.

Every tensor is drawn by toyinfer_amd.synth (SplitMix64 + Box-Muller, the
same bits on every machine) and rounded to bf16, so a fixture needs to store
only the seed and the token ids.
"""
from __future__ import annotations

import numpy as np

from toyinfer_amd import synth

LAYER_SHAPES = ("input_layernorm", "q_proj", "k_proj", "v_proj", "q_norm", "k_norm", "o_proj",
                "post_attention_layernorm", "gate_proj", "up_proj", "down_proj")


def layer_shapes(cfg: dict) -> dict:
    qd, kv = cfg["num_q_heads"] * cfg["head_dim"], cfg["num_kv_heads"] * cfg["head_dim"]
    H, F = cfg["hidden_size"], cfg["intermediate_size"]
    return {"input_layernorm": (H,), "q_proj": (qd, H), "k_proj": (kv, H), "v_proj": (kv, H),
            "q_norm": (cfg["head_dim"],), "k_norm": (cfg["head_dim"],), "o_proj": (H, qd),
            "post_attention_layernorm": (H,), "gate_proj": (F, H), "up_proj": (F, H),
            "down_proj": (H, F)}


def bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def scaled_bits(seed: int, name: str, shape, std: float) -> np.ndarray:
    """bf16 bits of std * N(0, 1) (the N(0, 1) draw rounded to bf16 first)."""
    return synth.scale_bf16(synth.normal_bf16(seed, name, shape), std)


def weight_bits(cfg: dict, seed: int, proj_std: float, embed_std: float, norm_range,
                tied: bool) -> dict:
    """bf16 bit patterns: {"layers": [{name: bits}], "embed_tokens", "norm",
    "lm_head"} (lm_head is the embedding array itself when tied).

    Projections ~ proj_std * N(0, 1), embeddings ~ embed_std * N(0, 1), norm
    weights ~ U(norm_range) (or all ones when norm_range is None)."""
    shapes = layer_shapes(cfg)

    def norm_w(name, shp):
        if norm_range is None:
            return synth.f32_to_bf16_bits(np.ones(shp, np.float32))
        return synth.uniform_bf16(seed, name, shp, norm_range[0], norm_range[1])

    out = {"layers": []}
    for l in range(cfg["num_layers"]):
        out["layers"].append({n: (norm_w(f"{l}.{n}", shp) if len(shp) == 1
                                  else scaled_bits(seed, f"{l}.{n}", shp, proj_std))
                              for n, shp in shapes.items()})
    V, H = cfg["vocab_size"], cfg["hidden_size"]
    out["embed_tokens"] = scaled_bits(seed, "embed", (V, H), embed_std)
    out["norm"] = norm_w("norm", (H,))
    out["lm_head"] = out["embed_tokens"] if tied else scaled_bits(seed, "lm_head", (V, H),
                                                                  proj_std)
    return out


def to_f32(bits: dict) -> dict:
    """The same dict with float32 arrays (bf16-valued) for the CPU references."""
    out = {"layers": [{n: bits_to_f32(b) for n, b in lw.items()} for lw in bits["layers"]]}
    for n in ("embed_tokens", "norm"):
        out[n] = bits_to_f32(bits[n])
    out["lm_head"] = (out["embed_tokens"] if bits["lm_head"] is bits["embed_tokens"]
                      else bits_to_f32(bits["lm_head"]))
    return out
