"""The model harness at Qwen3-8B's layer widths (hidden 4096, 32/8 heads,
D=128, SwiGLU 12288; one layer, vocab 4096, tied embeddings; bf16 weights
0.02 * N(0, 1), norm weights 1): a 24-token prefill and 3 greedy decode
steps, direct and from a captured graph, against the oracle's forward.

These widths take the decode projections down paths the 0.6B geometry does
not: inputs of 4096 elements (eight 16-byte chunks per lane in the one-token
GEMV, its largest register form) and the 12288-element input of the down
projection (the block-cooperative GEMV, for inputs over 4096).

Bars as for configuration 5 (tests/test_qwen3_config5_gpu.py): the oracle
and the device round the same activations to bf16 at the same points, and
their fp32 reduction orders differ.
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

WIDE = dict(num_layers=1, hidden_size=4096, num_q_heads=32, num_kv_heads=8, head_dim=128,
            intermediate_size=12288, vocab_size=4096, max_seq_len=64, max_prefill_tokens=32,
            rms_norm_eps=1e-6, rope_theta=1e6)
SEED = 93


@pytest.fixture(scope="module")
def weights_wide(dev):
    print("[step] wide weights (host draw + upload)", flush=True)
    bits = QW.weight_bits(WIDE, SEED, proj_std=0.02, embed_std=0.02, norm_range=None, tied=True)
    dw = {"layers": [{n: H.to_dev_bf16(b, dev) for n, b in lw.items()} for lw in bits["layers"]]}
    dw["embed_tokens"] = H.to_dev_bf16(bits["embed_tokens"], dev)
    dw["norm"] = H.to_dev_bf16(bits["norm"], dev)
    dw["lm_head"] = dw["embed_tokens"]
    host = QW.to_f32(bits)
    host["inv_freq"] = oracle.inv_freq(WIDE["head_dim"], WIDE["rope_theta"])
    H.sync()
    return host, dw


def check_logits(got, exp, label):
    assert np.isfinite(got).all(), f"{label}: non-finite logits"
    d = np.abs(got.astype(np.float64) - exp)
    print(f"  {label}: max {d.max():.4f} mean {d.mean():.5f} (std {exp.std():.3f})", flush=True)
    assert d.max() <= LOGIT_MAX_ABS and d.mean() <= LOGIT_MEAN_ABS, \
        f"{label}: max {d.max():.3g} mean {d.mean():.3g}"


# max_seq_len 64: the attention pass gives each split a fixed 128-row slice of
# the cache and requests it before the device length arrives; 16384 (more
# rows than 96 splits x 128): slices follow the length instead.
@pytest.mark.parametrize("msl", [64, 16384])
@pytest.mark.parametrize("graph", [False, True])
def test_wide_prefill_and_decode_vs_oracle(dev, weights_wide, graph, msl):
    print(f"[step] wide prefill 24 + 3 decode steps, graph={graph}, max_seq_len={msl}", flush=True)
    host, dw = weights_wide
    T, steps = 24, 3
    ids = np.random.default_rng(SEED + int(graph)).integers(0, WIDE["vocab_size"], T)
    ids = ids.astype(np.uint32)
    m = qwen3.Qwen3(qwen3.Config(**dict(WIDE, max_seq_len=msl)), dw)
    id_t = torch.from_numpy(ids.view(np.int32)).to(dev)
    m.prefill(id_t, T)
    got = m.logits_host()
    ref = oracle.Qwen3Reference(dict(WIDE, max_seq_len=T + steps + 1), host)
    check_logits(got, ref.forward(ids, 0), "prefill")
    toks = m.tokens_host(T + 1)
    assert toks[T] == oracle.argmax(got), "prefill pick"
    for s in range(steps):
        m.decode(1, graph)
        got = m.logits_host()
        toks = m.tokens_host(T + s + 2)
        check_logits(got, ref.forward([toks[T + s]], T + s), f"step {s}")
        assert toks[T + s + 1] == oracle.argmax(got), f"step {s} pick"
    assert m.position_host() == T + steps
    m.close()
