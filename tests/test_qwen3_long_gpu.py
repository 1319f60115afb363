"""The model harness where the one-token attention pass gives its splits
slices that follow the device length (more cache rows than splits x 128),
at widths that take the block-cooperative decode GEMV's single-read RMSNorm
staging (inputs of 4097..8192 elements).

Geometry: one layer, hidden 5120 (Qwen3-14B's width), 64 query / 64 KV heads,
D=128, SwiGLU 6144, vocab 512, tied embeddings; bf16 weights 0.02 * N(0, 1),
norm weights 1; max_seq_len 2048.  With 64 KV heads one sequence fills the
resident workgroup slots with 12 splits (768 slots on 256 CUs), so 12 x 128
rows < 2048 and the slices follow the length: at a 1700-token prompt each
split holds about 142 rows, its four waves walk more than one 32-row chunk
each (the next chunk's loads in flight), the new token's k/v row is swapped
into the last split's later chunk, and V past the length is zeroed.  The
decode GEMVs see inputs of 5120 (hidden), 8192 (q heads x D) and 6144
(SwiGLU) elements.  The prompt itself runs the fused QK-norm + RoPE
128-row prefill kernel (896 workgroups).

A direct model and a graph-replayed model take the same prompt and 3 greedy
steps: both against the oracle's forward (bars as for configuration 5,
tests/test_qwen3_config5_gpu.py), and graph == direct bit for bit.
"""
import numpy as np
import pytest
import torch

import oracle
from tests import helpers as H
from tests import qwen3_weights as QW
from toyinfer_amd import attn, qwen3

pytestmark = pytest.mark.gpu

LOGIT_MAX_ABS = 0.1
LOGIT_MEAN_ABS = 0.02

LONG = dict(num_layers=1, hidden_size=5120, num_q_heads=64, num_kv_heads=64, head_dim=128,
            intermediate_size=6144, vocab_size=512, max_seq_len=2048, max_prefill_tokens=1700,
            rms_norm_eps=1e-6, rope_theta=1e6)
SEED = 97


def check_logits(got, exp, label):
    assert np.isfinite(got).all(), f"{label}: non-finite logits"
    d = np.abs(got.astype(np.float64) - exp)
    print(f"  {label}: max {d.max():.4f} mean {d.mean():.5f} (std {exp.std():.3f})", flush=True)
    assert d.max() <= LOGIT_MAX_ABS and d.mean() <= LOGIT_MEAN_ABS, \
        f"{label}: max {d.max():.3g} mean {d.mean():.3g}"


def test_length_following_slices_and_wide_gemv_vs_oracle(dev):
    splits = attn.decode_default_splits(1, LONG["num_q_heads"], LONG["num_kv_heads"],
                                        LONG["head_dim"], LONG["max_seq_len"])
    print(f"[step] long-cache model: {splits} splits, max_seq_len {LONG['max_seq_len']}",
          flush=True)
    assert splits * 128 < LONG["max_seq_len"], "this device would take the fixed-slice path"
    T, steps = 1700, 3
    assert -(-T // splits) > 4 * 32, "each wave should walk more than one chunk"
    print("[step] weights (host draw + upload)", flush=True)
    bits = QW.weight_bits(LONG, SEED, proj_std=0.02, embed_std=0.02, norm_range=None, tied=True)
    dw = {"layers": [{n: H.to_dev_bf16(b, dev) for n, b in lw.items()} for lw in bits["layers"]]}
    dw["embed_tokens"] = H.to_dev_bf16(bits["embed_tokens"], dev)
    dw["norm"] = H.to_dev_bf16(bits["norm"], dev)
    dw["lm_head"] = dw["embed_tokens"]
    host = QW.to_f32(bits)
    host["inv_freq"] = oracle.inv_freq(LONG["head_dim"], LONG["rope_theta"])
    H.sync()

    ids = np.random.default_rng(SEED).integers(0, LONG["vocab_size"], T).astype(np.uint32)
    id_t = torch.from_numpy(ids.view(np.int32)).to(dev)
    direct = qwen3.Qwen3(qwen3.Config(**LONG), dw)
    graph = qwen3.Qwen3(qwen3.Config(**LONG), dw)
    print("[step] prefill 1700 (two models)", flush=True)
    direct.prefill(id_t, T)
    graph.prefill(id_t, T)
    got = direct.logits_host()
    assert np.array_equal(got.view(np.uint32), graph.logits_host().view(np.uint32))
    print("[step] oracle forward of 1700 tokens", flush=True)
    ref = oracle.Qwen3Reference(dict(LONG, max_seq_len=T + steps + 1), host)
    check_logits(got, ref.forward(ids, 0), "prefill")
    toks = direct.tokens_host(T + 1)
    assert toks[T] == oracle.argmax(got), "prefill pick"
    for s in range(steps):
        print(f"[step] decode step {s} (direct and graph)", flush=True)
        direct.decode(1, False)
        graph.decode(1, True)
        got = direct.logits_host()
        assert np.array_equal(got.view(np.uint32), graph.logits_host().view(np.uint32)), \
            f"step {s}: graph != direct"
        toks = direct.tokens_host(T + s + 2)
        assert np.array_equal(toks, graph.tokens_host(T + s + 2))
        check_logits(got, ref.forward([toks[T + s]], T + s), f"step {s}")
        assert toks[T + s + 1] == oracle.argmax(got), f"step {s} pick"
    assert direct.position_host() == graph.position_host() == T + steps
    direct.close()
    graph.close()
