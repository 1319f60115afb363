"""The HIP path against the committed golden fixtures (torch float64 values,
tests/golden/make_golden.py), independently of the oracle."""
import hashlib
import os

import numpy as np
import pytest
import torch

from tests import helpers as H
from toyinfer_amd import attn, synth

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def gold(name):
    return np.load(os.path.join(GOLD, name + ".npz"))


def sha(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def prefill(qb, kb, vb, dev, algo):
    s, hq, d = qb.shape
    q, k, v = H.to_dev_bf16(qb, dev), H.to_dev_bf16(kb, dev), H.to_dev_bf16(vb, dev)
    o = torch.empty((s, hq, d), dtype=torch.bfloat16, device=dev)
    attn.flash_attention_algo_bf16(q, k, v, o, hq, kb.shape[1], d, s, algo)
    H.sync()
    return H.bf16_bits_to_f32(H.from_dev_bf16(o))


@pytest.mark.parametrize("algo", [attn.ALGO_SPLIT_KEYS, attn.ALGO_ROW_TILES, attn.ALGO_SPLIT_PAIRS, attn.ALGO_ROW_PAIRS])
@pytest.mark.parametrize("name", ["seq1_gqa", "exact_kv_tile", "gqa_tail_tiles", "multi_kv_tile",
                                  "large_magnitude", "causal_focus"])
def test_prefill_reference_cases_vs_golden(dev, name, algo):
    g = gold("prefill_" + name)
    got = prefill(g["q"], g["k"], g["v"], dev, algo)
    H.check_bar(got, H.bf16_bits_to_f32(g["o_bf16"]), name)


@pytest.mark.parametrize("algo", [attn.ALGO_SPLIT_KEYS, attn.ALGO_ROW_TILES, attn.ALGO_SPLIT_PAIRS, attn.ALGO_ROW_PAIRS])
def test_prefill_config1_vs_golden(dev, algo):
    g = gold("prefill_config1")
    sd = int(g["seed"])
    qb = synth.normal_bf16(sd, "q", (128, 16, 128))
    kb = synth.normal_bf16(sd, "k", (128, 8, 128))
    vb = synth.normal_bf16(sd, "v", (128, 8, 128))
    assert sha(qb, kb, vb) == str(g["inputs_sha256"])
    got = prefill(qb, kb, vb, dev, algo)
    mx, mn = H.check_bar(got, H.bf16_bits_to_f32(g["o_bf16"]), "config1")
    print(f"[golden] config1 algo={algo} max-abs {mx:.3g} mean-abs {mn:.3g}", flush=True)


@pytest.mark.parametrize("name", ["pos0_gqa", "full_kv", "tiled_seq"])
def test_decode_reference_cases_vs_golden(dev, name):
    g = gold("decode_" + name)
    hq, d = g["q"].shape
    msl, hkv = g["k"].shape[0], g["k"].shape[1]
    pos = int(g["pos"])
    score = torch.full((hq, msl), 7.0, dtype=torch.float32, device=dev)
    ob = torch.full((hq, d), -7.0, dtype=torch.float32, device=dev)
    o = torch.full((hq, d), 3.0, dtype=torch.bfloat16, device=dev)
    attn.attention_bf16(H.to_dev_bf16(g["q"], dev), H.to_dev_bf16(g["k"], dev),
                        H.to_dev_bf16(g["v"], dev), score, ob, o, hq, hkv, d, pos, msl)
    H.sync()
    H.check_close(score.cpu().numpy(), g["score"], 5e-3, 5e-3, name + " score")
    H.check_close(ob.cpu().numpy(), g["o"], 5e-2, 5e-2, name + " o_buffer")
    H.check_bar(H.bf16_bits_to_f32(H.from_dev_bf16(o)), H.bf16_bits_to_f32(g["o_bf16"]), name)


def test_decode_batched_vs_golden(dev):
    g = gold("decode_seeded")
    sd = int(g["seed"])
    qb = synth.normal_bf16(sd, "q", (2, 8, 128))
    kb = synth.normal_bf16(sd, "k", (2, 300, 2, 128))
    vb = synth.normal_bf16(sd, "v", (2, 300, 2, 128))
    assert sha(qb, kb, vb) == str(g["inputs_sha256"])
    q, k, v = H.to_dev_bf16(qb, dev), H.to_dev_bf16(kb, dev), H.to_dev_bf16(vb, dev)
    lens = torch.tensor(g["lens"].astype(np.int32), device=dev)
    o = torch.empty((2, 8, 128), dtype=torch.bfloat16, device=dev)
    s = attn.decode_default_splits(2, 8, 2, 128, 300)
    ws = attn.decode_workspace(2, 8, 128, s, dev)
    attn.decode_attention_bf16(q, k, v, o, 2, 8, 2, 128, lens, 300, 300 * 2 * 128, s, ws)
    H.sync()
    H.check_bar(H.bf16_bits_to_f32(H.from_dev_bf16(o)), H.bf16_bits_to_f32(g["o_bf16"]),
                "decode seeded")


def test_fused_prefill_vs_golden(dev):
    g = gold("fused_small")
    sd, s, hq, hkv, d = int(g["seed"]), 96, 4, 2, 128
    qb = synth.normal_bf16(sd, "q", (s, hq, d))
    kb = synth.normal_bf16(sd, "k", (s, hkv, d))
    vb = synth.normal_bf16(sd, "v", (s, hkv, d))
    gq = synth.uniform_bf16(sd, "gamma_q", (d,), 0.9, 1.1)
    gk = synth.uniform_bf16(sd, "gamma_k", (d,), 0.9, 1.1)
    assert sha(qb, kb, vb, gq, gk) == str(g["inputs_sha256"])
    f = torch.empty(d // 2, dtype=torch.float32, device=dev)
    attn.precompute_freq_f32(f, d, float(g["theta"]))
    table = torch.empty((s, d // 2, 2), dtype=torch.float32, device=dev)
    attn.rope_cos_sin_f32(table, f, s, d)
    q, k, v = H.to_dev_bf16(qb, dev), H.to_dev_bf16(kb, dev), H.to_dev_bf16(vb, dev)
    o = torch.empty((s, hq, d), dtype=torch.bfloat16, device=dev)
    k_out = torch.empty_like(k)
    attn.prefill_qknorm_rope_attention_bf16(q, k, v, o, k_out, H.to_dev_bf16(gq, dev),
                                            H.to_dev_bf16(gk, dev), table, float(g["eps"]),
                                            hq, hkv, d, s)
    H.sync()
    H.check_bar(H.bf16_bits_to_f32(H.from_dev_bf16(k_out)),
                H.bf16_bits_to_f32(g["k_norm_rope"]), "K_out")
    H.check_bar(H.bf16_bits_to_f32(H.from_dev_bf16(o)), H.bf16_bits_to_f32(g["o_bf16"]),
                "fused O")
