"""The model harness at configuration 5's full geometry: random-init
Qwen3-0.6B (28 layers, hidden 1024, 16/8 heads, D=128, SwiGLU 3072, vocab
151936, tied embeddings; bf16 weights 0.02 * N(0, 1), norm weights 1).

* A 48-token prefill and 4 greedy decode steps (direct and graph) against the
  oracle's forward (oracle.Qwen3Reference, itself pinned to an independent
  float64 forward that matches transformers' Qwen3): each step's logits
  within LOGIT_MAX_ABS / LOGIT_MEAN_ABS, the device pick = argmax of the
  device logits, the oracle fed the tokens the device chose.
* The 1371-token prompt of config 5 and 2 graph decode steps against the
  same oracle forward.
* After a 1371-token prefill, 12 decode steps from a captured graph and 12
  direct steps give identical tokens and logits.

Bars: the oracle and the float64 forward with the same bf16 rounding points
differ by max 0.041, mean 0.0069 on these logits (std 0.64; fp32 vs fp64
sums flip a bf16 activation now and then and 28 layers carry the flips);
the GPU's own reduction orders do the same, so the bars are about 2.5x that.
"""
import numpy as np
import pytest
import torch

import oracle
from tests import helpers as H
from tests import qwen3_weights as QW
from toyinfer_amd import qwen3

pytestmark = pytest.mark.gpu

LOGIT_MAX_ABS = 0.1
LOGIT_MEAN_ABS = 0.02

CFG5 = dict(num_layers=28, hidden_size=1024, num_q_heads=16, num_kv_heads=8, head_dim=128,
            intermediate_size=3072, vocab_size=151936, max_seq_len=1400,
            max_prefill_tokens=1371, rms_norm_eps=1e-6, rope_theta=1e6)
SEED = 91


@pytest.fixture(scope="module")
def weights5(dev):
    print("[step] config-5 weights (host draw + upload)", flush=True)
    bits = QW.weight_bits(CFG5, SEED, proj_std=0.02, embed_std=0.02, norm_range=None, tied=True)
    dw = {"layers": [{n: H.to_dev_bf16(b, dev) for n, b in lw.items()} for lw in bits["layers"]]}
    dw["embed_tokens"] = H.to_dev_bf16(bits["embed_tokens"], dev)
    dw["norm"] = H.to_dev_bf16(bits["norm"], dev)
    dw["lm_head"] = dw["embed_tokens"]
    host = QW.to_f32(bits)
    host["inv_freq"] = oracle.inv_freq(CFG5["head_dim"], CFG5["rope_theta"])
    H.sync()
    return host, dw


def ids_dev(ids, dev):
    return torch.from_numpy(np.ascontiguousarray(ids, np.uint32).view(np.int32)).to(dev)


def check_logits(got, exp, label):
    assert np.isfinite(got).all(), f"{label}: non-finite logits"
    d = np.abs(got.astype(np.float64) - exp)
    print(f"  {label}: max {d.max():.4f} mean {d.mean():.5f} (std {exp.std():.3f})", flush=True)
    assert d.max() <= LOGIT_MAX_ABS and d.mean() <= LOGIT_MEAN_ABS, \
        f"{label}: max {d.max():.3g} mean {d.mean():.3g}"


@pytest.mark.parametrize("graph", [False, True])
def test_config5_prefill_and_decode_vs_oracle(dev, weights5, graph):
    print(f"[step] config-5 prefill 48 + 4 decode steps, graph={graph}", flush=True)
    host, dw = weights5
    T, steps = 48, 4
    ids = np.random.default_rng(SEED + int(graph)).integers(0, CFG5["vocab_size"], T)
    ids = ids.astype(np.uint32)
    m = qwen3.Qwen3(qwen3.Config(**CFG5), dw)
    id_t = ids_dev(ids, dev)
    m.prefill(id_t, T)
    got = m.logits_host()
    ref = oracle.Qwen3Reference(dict(CFG5, max_seq_len=T + steps + 1), host)
    check_logits(got, ref.forward(ids, 0), "prefill")
    toks = m.tokens_host(T + 1)
    assert np.array_equal(toks[:T], ids)
    assert toks[T] == oracle.argmax(got), "prefill pick"
    for s in range(steps):
        m.decode(1, graph)
        got = m.logits_host()
        toks = m.tokens_host(T + s + 2)
        check_logits(got, ref.forward([toks[T + s]], T + s), f"step {s}")
        assert toks[T + s + 1] == oracle.argmax(got), f"step {s} pick"
    assert m.position_host() == T + steps
    m.close()


def test_config5_full_prompt_and_decode_vs_oracle(dev, weights5):
    """Configuration 5's own prompt length (src/transformer.cpp:327-481 runs
    the 1371-token prompt): every layer's attention goes through the
    persistent split-over-keys prefill kernel in more than one round, and the
    prefill projections through the 128 x 192 / 64 x 64 GEMM tiles; then two
    graph-replayed decode steps over the 1371-row cache."""
    print("[step] config-5 1371-token prefill + 2 graph decode steps vs oracle", flush=True)
    host, dw = weights5
    T, steps = 1371, 2
    ids = np.random.default_rng(SEED + 11).integers(0, CFG5["vocab_size"], T).astype(np.uint32)
    m = qwen3.Qwen3(qwen3.Config(**CFG5), dw)
    id_t = ids_dev(ids, dev)
    m.prefill(id_t, T)
    got = m.logits_host()
    print("[step] oracle forward of 1371 tokens", flush=True)
    ref = oracle.Qwen3Reference(dict(CFG5, max_seq_len=T + steps + 1), host)
    check_logits(got, ref.forward(ids, 0), "prefill 1371")
    toks = m.tokens_host(T + 1)
    assert np.array_equal(toks[:T], ids)
    assert toks[T] == oracle.argmax(got), "prefill pick"
    for s in range(steps):
        m.decode(1, True)
        got = m.logits_host()
        toks = m.tokens_host(T + s + 2)
        check_logits(got, ref.forward([toks[T + s]], T + s), f"step {s}")
        assert toks[T + s + 1] == oracle.argmax(got), f"step {s} pick"
    assert m.position_host() == T + steps
    m.close()


def test_config5_graph_equals_direct_after_long_prefill(dev, weights5):
    print("[step] config-5 1371-token prefill, graph vs direct decode", flush=True)
    _, dw = weights5
    T, steps = 1371, 12
    ids = np.random.default_rng(SEED + 7).integers(0, CFG5["vocab_size"], T).astype(np.uint32)
    id_t = ids_dev(ids, dev)
    a = qwen3.Qwen3(qwen3.Config(**CFG5), dw)
    b = qwen3.Qwen3(qwen3.Config(**CFG5), dw)
    for m in (a, b):
        m.prefill(id_t, T)
    la, lb = a.logits_host(), b.logits_host()
    assert np.array_equal(la.view(np.uint32), lb.view(np.uint32)), "prefill is deterministic"
    a.decode(steps, False)
    b.decode(5, True)
    b.decode(steps - 5, True)
    assert np.array_equal(a.tokens_host(T + steps + 1), b.tokens_host(T + steps + 1))
    assert np.array_equal(a.logits_host().view(np.uint32), b.logits_host().view(np.uint32))
    assert a.position_host() == b.position_host() == T + steps
    a.close()
    b.close()
