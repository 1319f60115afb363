"""Write tests/golden/qwen3_tiny.npz: logits of a small random-init Qwen3 from an
implementation independent of oracle/ (run on the CPU; torch and transformers
required, so this runs in the build container only).

Two float64 torch forwards written from the model's equations (not from the
oracle's code):

* ``exact``: no rounding anywhere.  It is checked here against
  transformers' Qwen3ForCausalLM (eager attention, float64, same weights).
  transformers computes RMSNorm statistics and the attention softmax in
  float32 even in a float64 model, which bounds the agreement near 1e-6 of
  the logit scale; the check asks for 1e-5 of it, while a structural slip
  moves logits by a sizeable fraction of that scale.  That pins the
  equations themselves (RMSNorm with
  weight, per-head q/k RMSNorm before RoPE, rotate-half RoPE with
  theta ** (-2i/D), causal GQA with query head h reading KV head
  h // (Hq/Hkv), SwiGLU, tied lm-head, final norm).
* ``rounded``: the same equations with every op output rounded to bf16 at
  the points where the reference engine stores bf16 tensors
  (src/transformer.cpp:327-481 prefill, :483-628 decode): input norm,
  q/k/v projections, q/k norm, RoPE, attention output, o-projection,
  residual add, post-attention norm, gate/up, SwiGLU, down projection,
  residual add, final norm; logits stay wide.  The oracle's
  Qwen3Reference (fp32 with the same rounding points) is pinned to this.

The fixture stores the config, the weight seed, the token ids and both
logit sets (prefill = last prompt token, then teacher-forced decode steps).

    python tests/golden/make_qwen3_golden.py
"""
from __future__ import annotations

import json
import math
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from tests import qwen3_weights as QW  # noqa: E402

CFG = dict(num_layers=2, hidden_size=256, num_q_heads=4, num_kv_heads=2, head_dim=128,
           intermediate_size=512, vocab_size=1000, max_seq_len=64, max_prefill_tokens=32,
           rms_norm_eps=1e-6, rope_theta=1e6)
SEED = 71
INIT = dict(proj_std=0.05, embed_std=1.0, norm_range=(0.8, 1.2), tied=True)
PROMPT = 13
DECODE = 3


def bf16(x: torch.Tensor) -> torch.Tensor:
    """Round a float64 tensor to the nearest bf16 value (ties to even)."""
    return x.to(torch.float32).to(torch.bfloat16).to(torch.float64)


class Forward64:
    """Qwen3 forward in float64 from the equations; `rnd` is applied to every
    stored activation (identity for the exact forward, bf16 for the rounded)."""

    def __init__(self, cfg, w, rnd):
        self.c, self.w, self.rnd = cfg, w, rnd
        L, msl = cfg["num_layers"], cfg["max_seq_len"]
        self.kc = torch.zeros(L, msl, cfg["num_kv_heads"], cfg["head_dim"], dtype=torch.float64)
        self.vc = torch.zeros_like(self.kc)
        d = cfg["head_dim"]
        # The rotary angle is a float32 product in the reference
        # (src/decode.cu:35-50 inv_freq, src/prefill.cu:185-208 angle) and in
        # transformers; cos and sin of that angle are taken in float64 here.
        self.inv = (1.0 / cfg["rope_theta"] ** (torch.arange(0, d, 2, dtype=torch.float64) / d)
                    ).to(torch.float32)

    def norm(self, x, w):
        return x / torch.sqrt((x * x).mean(-1, keepdim=True) + self.c["rms_norm_eps"]) * w

    def rope(self, x, pos):
        """x [T][H][D] at positions pos [T]: pairs (i, i + D/2)."""
        ang = (pos[:, None].to(torch.float32) * self.inv[None, :]).to(torch.float64)
        c, s = torch.cos(ang)[:, None, :], torch.sin(ang)[:, None, :]
        h = x.shape[-1] // 2
        x1, x2 = x[..., :h], x[..., h:]
        return torch.cat([x1 * c - x2 * s, x2 * c + x1 * s], -1)

    def attention(self, q, l, pos0, T):
        """q [T][Hq][D] against cache rows 0 .. pos0+T-1, causal."""
        hq, hkv, d = self.c["num_q_heads"], self.c["num_kv_heads"], self.c["head_dim"]
        n = pos0 + T
        k = self.kc[l, :n].repeat_interleave(hq // hkv, 1)   # [n][Hq][D]
        v = self.vc[l, :n].repeat_interleave(hq // hkv, 1)
        s = torch.einsum("thd,nhd->htn", q, k) / math.sqrt(d)
        qpos = torch.arange(pos0, pos0 + T)[:, None]
        s = s.masked_fill(torch.arange(n)[None, :] > qpos, float("-inf"))
        return torch.einsum("htn,nhd->thd", torch.softmax(s, -1), v)

    def layer(self, l, x, pos0):
        c, W, r = self.c, self.w["layers"][l], self.rnd
        T = x.shape[0]
        hq, hkv, d = c["num_q_heads"], c["num_kv_heads"], c["head_dim"]
        xn = r(self.norm(x, W["input_layernorm"]))
        q = r(xn @ W["q_proj"].T).view(T, hq, d)
        k = r(xn @ W["k_proj"].T).view(T, hkv, d)
        v = r(xn @ W["v_proj"].T).view(T, hkv, d)
        pos = torch.arange(pos0, pos0 + T)
        q = r(self.rope(r(self.norm(q, W["q_norm"])), pos))
        k = r(self.rope(r(self.norm(k, W["k_norm"])), pos))
        self.kc[l, pos0:pos0 + T] = k
        self.vc[l, pos0:pos0 + T] = v
        o = r(self.attention(q, l, pos0, T)).reshape(T, hq * d)
        x = r(x + r(o @ W["o_proj"].T))
        xn = r(self.norm(x, W["post_attention_layernorm"]))
        g, u = r(xn @ W["gate_proj"].T), r(xn @ W["up_proj"].T)
        h = r(g * torch.sigmoid(g) * u)
        return r(x + r(h @ W["down_proj"].T))

    def forward(self, ids, pos0):
        x = self.w["embed_tokens"][torch.as_tensor(np.asarray(ids, np.int64))]
        for l in range(self.c["num_layers"]):
            x = self.layer(l, x, pos0)
        xn = self.rnd(self.norm(x[-1:], self.w["norm"]))
        return (xn @ self.w["lm_head"].T)[0]


def torch_weights(wf32):
    t = lambda a: torch.from_numpy(np.asarray(a, np.float64))  # noqa: E731
    out = {"layers": [{n: t(a) for n, a in lw.items()} for lw in wf32["layers"]]}
    for n in ("embed_tokens", "norm", "lm_head"):
        out[n] = t(wf32[n])
    return out


def transformers_logits(cfg, w, ids_all, prompt):
    """transformers' Qwen3ForCausalLM in float64 on the same weights: logits
    at the last prompt position and at each later position (one forward over
    the whole sequence; causal masking makes them the decode-step logits)."""
    from transformers import Qwen3Config, Qwen3ForCausalLM

    hc = Qwen3Config(vocab_size=cfg["vocab_size"], hidden_size=cfg["hidden_size"],
                     intermediate_size=cfg["intermediate_size"],
                     num_hidden_layers=cfg["num_layers"],
                     num_attention_heads=cfg["num_q_heads"],
                     num_key_value_heads=cfg["num_kv_heads"], head_dim=cfg["head_dim"],
                     rms_norm_eps=cfg["rms_norm_eps"],
                     rope_parameters={"rope_type": "default", "rope_theta": cfg["rope_theta"]},
                     max_position_embeddings=cfg["max_seq_len"], tie_word_embeddings=True,
                     attention_bias=False, hidden_act="silu")
    model = Qwen3ForCausalLM(hc).to(torch.float64)
    model.config._attn_implementation = "eager"
    sd = {"model.embed_tokens.weight": w["embed_tokens"], "model.norm.weight": w["norm"],
          "lm_head.weight": w["lm_head"]}
    names = {"input_layernorm": "input_layernorm", "post_attention_layernorm":
             "post_attention_layernorm", "q_proj": "self_attn.q_proj", "k_proj": "self_attn.k_proj",
             "v_proj": "self_attn.v_proj", "o_proj": "self_attn.o_proj",
             "q_norm": "self_attn.q_norm", "k_norm": "self_attn.k_norm",
             "gate_proj": "mlp.gate_proj", "up_proj": "mlp.up_proj", "down_proj": "mlp.down_proj"}
    for l, lw in enumerate(w["layers"]):
        for n, hf in names.items():
            sd[f"model.layers.{l}.{hf}.weight"] = lw[n]
    missing, unexpected = model.load_state_dict(sd, strict=False)
    assert not unexpected and all("rotary" in m for m in missing), (missing, unexpected)
    model.eval()
    with torch.no_grad():
        out = model(torch.as_tensor(np.asarray(ids_all, np.int64))[None]).logits[0]
    return out[prompt - 1:]


def main():
    bits = QW.weight_bits(CFG, SEED, **INIT)
    w = torch_weights(QW.to_f32(bits))
    rng = np.random.default_rng(SEED)
    ids = rng.integers(0, CFG["vocab_size"], size=PROMPT + DECODE).astype(np.uint32)

    sets = {}
    for name, rnd in (("exact", lambda x: x), ("rounded", bf16)):
        f = Forward64(CFG, w, rnd)
        rows = [f.forward(ids[:PROMPT], 0)]
        for s in range(DECODE):
            rows.append(f.forward(ids[PROMPT + s:PROMPT + s + 1], PROMPT + s))
        sets[name] = torch.stack(rows).numpy()

    hf = transformers_logits(CFG, w, ids, PROMPT).numpy()
    dx = np.abs(hf - sets["exact"]).max()
    scale = np.abs(sets["exact"]).max()
    print(f"transformers vs exact float64 forward: max |diff| {dx:.3g} (max |logit| {scale:.3g})")
    assert dx < 1e-5 * scale, "the float64 forward does not match transformers' Qwen3"
    dr = np.abs(sets["rounded"] - sets["exact"])
    print(f"bf16 rounding points move the logits by max {dr.max():.3g}, mean {dr.mean():.3g} "
          f"(logit std {sets['exact'].std():.3g})")

    np.savez_compressed(os.path.join(HERE, "qwen3_tiny.npz"),
                        config=np.array(json.dumps(CFG)), init=np.array(json.dumps(INIT)),
                        seed=np.array(SEED), ids=ids, prompt=np.array(PROMPT),
                        logits_exact=sets["exact"], logits_rounded=sets["rounded"],
                        transformers_max_diff=np.array(dx))
    print("wrote qwen3_tiny.npz")


if __name__ == "__main__":
    main()
