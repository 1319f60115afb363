"""Write the golden fixtures under tests/golden/ (run on the CPU; torch required).

Expected values come from an implementation independent of oracle/: torch
on the CPU in float64 (attention, softmax, RMSNorm sums) with torch's own
float32 -> bfloat16 conversion for the rounding steps.  Inputs come from the
reference tests' deterministic case formulas (restated in oracle/, used here
only as an input generator; these fixtures store their inputs as bf16 bit
patterns, so the check does not depend on libm) and from toyinfer_amd.synth's
seeded normals (these store the seed and a SHA-256 of the input bits, which
the tests regenerate and verify).

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import os
import sys

import hashlib

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402  (input generators only)
from toyinfer_amd import synth  # noqa: E402


def to_bits(x: torch.Tensor) -> np.ndarray:
    return x.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def from_bits(b: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(torch.bfloat16).float()


def sha(*arrays) -> np.ndarray:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return np.array(h.hexdigest())


def flash_fp64(q, k, v):
    """Causal GQA attention in float64: q [S][Hq][D], k/v [S][Hkv][D]."""
    s, hq, d = q.shape
    g = hq // k.shape[1]
    q64, k64, v64 = q.double(), k.double().repeat_interleave(g, 1), v.double().repeat_interleave(g, 1)
    sc = torch.einsum("shd,thd->hst", q64, k64) / np.sqrt(d)
    sc = sc.masked_fill(torch.triu(torch.ones(s, s, dtype=torch.bool), 1), float("-inf"))
    p = torch.softmax(sc, -1)
    return torch.einsum("hst,thd->shd", p, v64)


def decode_fp64(q, k, v, pos, msl):
    """Single-sequence decode: q [Hq][D], k/v [MSL][Hkv][D] -> (score [Hq][MSL]
    probabilities with zeros past pos, o [Hq][D])."""
    hq, d = q.shape
    g = hq // k.shape[1]
    kk = k[: pos + 1].double().repeat_interleave(g, 1)
    vv = v[: pos + 1].double().repeat_interleave(g, 1)
    sc = torch.einsum("hd,thd->ht", q.double(), kk) / np.sqrt(d)
    p = torch.softmax(sc, -1)
    score = torch.zeros(hq, msl, dtype=torch.float64)
    score[:, : pos + 1] = p
    return score, torch.einsum("ht,thd->hd", p, vv)


def qknorm_rope(x, gamma, theta, eps):
    """x [T][H][D] float (bf16 values) -> RMSNorm -> bf16 -> RoPE -> bf16."""
    t, h, d = x.shape
    inv = 1.0 / torch.sqrt((x.double() ** 2).sum(-1, keepdim=True) / d + eps)
    y = (x.double() * inv * gamma.double()).float().to(torch.bfloat16).float()
    i = torch.arange(d // 2, dtype=torch.float32)
    f = (1.0 / torch.pow(torch.tensor(theta, dtype=torch.float64), 2.0 * i.double() / d)).float()
    ang = (torch.arange(t, dtype=torch.float32)[:, None] * f[None, :]).double()
    c, s_ = torch.cos(ang)[:, None, :], torch.sin(ang)[:, None, :]
    re, im = y[..., : d // 2].double(), y[..., d // 2:].double()
    out = torch.cat([re * c - im * s_, im * c + re * s_], -1)
    return out.float().to(torch.bfloat16).float()


def main():
    out = {}
    # Prefill: the reference's cases (tests/test_flash_attention_v1_bf16.cu:113-131).
    cases = [("seq1_gqa", 2, 1, 64, 1, 0.07, 0.03, 1.0, 1.0, 1.0),
             ("exact_kv_tile", 4, 4, 64, 32, 0.05, 0.021, 1.0, 1.0, 1.0),
             ("gqa_tail_tiles", 8, 2, 128, 37, 0.033, 0.017, 1.0, 1.0, 1.0),
             ("multi_kv_tile", 6, 3, 128, 65, 0.028, 0.019, 1.0, 1.0, 1.0),
             ("large_magnitude", 4, 2, 64, 19, 0.061, 0.027, 12.0, 10.0, 1.7)]
    for name, hq, hkv, d, s, qp, kvp, qs, ks, vs in cases:
        q, k, v = (torch.from_numpy(a) for a in oracle.make_flash_case(hq, hkv, d, s, qp, kvp,
                                                                        qs, ks, vs))
        qb, kb, vb = to_bits(q), to_bits(k), to_bits(v)
        o = flash_fp64(from_bits(qb), from_bits(kb), from_bits(vb))
        out[f"prefill_{name}"] = dict(q=qb, k=kb, v=vb, o=o.float().numpy(), o_bf16=to_bits(o.float()))
    q, k, v = (torch.from_numpy(a) for a in oracle.make_causal_focus_case())
    qb, kb, vb = to_bits(q), to_bits(k), to_bits(v)
    o = flash_fp64(from_bits(qb), from_bits(kb), from_bits(vb))
    out["prefill_causal_focus"] = dict(q=qb, k=kb, v=vb, o=o.float().numpy(),
                                       o_bf16=to_bits(o.float()))
    # Config 1: S=128, 16/8, D=128, seeded N(0,1).
    qb = synth.normal_bf16(1, "q", (128, 16, 128))
    kb = synth.normal_bf16(1, "k", (128, 8, 128))
    vb = synth.normal_bf16(1, "v", (128, 8, 128))
    o = flash_fp64(from_bits(qb), from_bits(kb), from_bits(vb))
    out["prefill_config1"] = dict(seed=np.array(1), inputs_sha256=sha(qb, kb, vb),
                                  o_bf16=to_bits(o.float()))

    # Decode: the reference's cases (tests/test_attention_bf16.cu:84-91).
    for name, hq, hkv, d, pos, msl, qp, kvp in [("pos0_gqa", 2, 1, 64, 0, 5, 0.07, 0.03),
                                                ("full_kv", 4, 4, 64, 6, 7, 0.05, 0.025),
                                                ("tiled_seq", 8, 2, 128, 37, 40, 0.03, 0.017)]:
        q, k, v = (torch.from_numpy(a) for a in oracle.make_attention_case(hq, hkv, d, msl, qp, kvp))
        qb, kb, vb = to_bits(q), to_bits(k), to_bits(v)
        score, o = decode_fp64(from_bits(qb), from_bits(kb), from_bits(vb), pos, msl)
        out[f"decode_{name}"] = dict(q=qb, k=kb, v=vb, pos=np.array(pos), score=score.float().numpy(),
                                     o=o.float().numpy(), o_bf16=to_bits(o.float()))
    # Decode, seeded: B=2 sequences of length 300 and 77, 8/2 heads, D=128.
    qb = synth.normal_bf16(5, "q", (2, 8, 128))
    kb = synth.normal_bf16(5, "k", (2, 300, 2, 128))
    vb = synth.normal_bf16(5, "v", (2, 300, 2, 128))
    lens = np.array([300, 77], np.uint32)
    os_ = [decode_fp64(from_bits(qb[i]), from_bits(kb[i]), from_bits(vb[i]), int(lens[i]) - 1,
                       300)[1] for i in range(2)]
    o = torch.stack(os_)
    out["decode_seeded"] = dict(seed=np.array(5), inputs_sha256=sha(qb, kb, vb), lens=lens,
                                o=o.float().numpy(), o_bf16=to_bits(o.float()))

    # Fused QK-RMSNorm + RoPE + attention, small (S=96, 4/2 heads, D=128).
    s, hq, hkv, d = 96, 4, 2, 128
    qb = synth.normal_bf16(9, "q", (s, hq, d))
    kb = synth.normal_bf16(9, "k", (s, hkv, d))
    vb = synth.normal_bf16(9, "v", (s, hkv, d))
    gq = synth.uniform_bf16(9, "gamma_q", (d,), 0.9, 1.1)
    gk = synth.uniform_bf16(9, "gamma_k", (d,), 0.9, 1.1)
    qn = qknorm_rope(from_bits(qb), from_bits(gq), 1e6, 1e-6)
    kn = qknorm_rope(from_bits(kb), from_bits(gk), 1e6, 1e-6)
    o = flash_fp64(qn, kn, from_bits(vb))
    out["fused_small"] = dict(seed=np.array(9), inputs_sha256=sha(qb, kb, vb, gq, gk),
                              k_norm_rope=to_bits(kn), q_norm_rope=to_bits(qn),
                              o_bf16=to_bits(o.float()), eps=np.array(1e-6, np.float32),
                              theta=np.array(1e6, np.float32))

    for name, arrays in out.items():
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **arrays)
        print(f"{path}: {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main()
