"""Decode parity: the split-K HIP path through the C ABI vs the CPU oracle.

Reference-contract cases follow tests/test_attention_bf16.cu:84-91 (dirty
score/O_buffer/O, tolerances 5e-3 / 5e-2 / 5e-2) and the graph replay of
tests/test_cuda_graph_pos.cu:94-219; the batched entry point is checked at
the benchmark shapes (B=8 L=4096 and B=1 L=32768, Qwen3-8B heads), with
ragged lengths, explicit split counts and run-to-run determinism.
"""
import numpy as np
import pytest
import torch

import oracle
from tests import helpers as H
from toyinfer_amd import attn, synth

pytestmark = pytest.mark.gpu


def dirty_buffers(hq, d, msl, dev):
    """Pre-filled outputs as tests/test_attention_bf16.cu:23-33 builds them."""
    i = np.arange(hq * msl)
    score = (10.0 - 0.1 * (i % 17)).astype(np.float32).reshape(hq, msl)
    j = np.arange(hq * d)
    ob = (-7.0 + 0.05 * (j % 23)).astype(np.float32).reshape(hq, d)
    o = oracle.f32_to_bf16((3.0 - 0.08 * (j % 19)).astype(np.float32)).reshape(hq, d)
    return H.to_dev_f32(score, dev), H.to_dev_f32(ob, dev), H.to_dev_bf16(o, dev)


def check_compat(score_d, ob_d, o_d, q, k, v, pos, msl, label):
    exp_score, exp_ob, exp_o = oracle.decode_attention(q, k, v, pos, msl)
    score = score_d.cpu().numpy()
    ob = ob_d.cpu().numpy()
    o = H.bf16_bits_to_f32(H.from_dev_bf16(o_d))
    H.check_close(score, exp_score, 5e-3, 5e-3, label + " score")
    assert np.all(score[:, pos + 1:] == 0.0), label + ": score past pos not zeroed"
    H.check_close(ob, exp_ob, 5e-2, 5e-2, label + " o_buffer")
    H.check_close(o, H.bf16_bits_to_f32(exp_o), 5e-2, 5e-2, label + " output")
    H.check_bar(o, H.bf16_bits_to_f32(exp_o), label + " output")


# tests/test_attention_bf16.cu:84-91 (label, Hq, Hkv, D, pos, MSL, q_phase, kv_phase)
REF_CASES = [
    ("pos0 gqa", 2, 1, 64, 0, 5, 0.07, 0.03),
    ("full-kv", 4, 4, 64, 6, 7, 0.05, 0.025),
    ("tiled-seq", 8, 2, 128, 37, 40, 0.03, 0.017),
    # Long caches: the split partials then live in score rows (several splits).
    ("long msl", 32, 8, 128, 777, 1000, 0.03, 0.017),
    ("long msl d64", 16, 4, 64, 2999, 3001, 0.021, 0.013),
    # Room past the length for the partials: the split pass also stores the
    # raw scores, and the score pass rescales them.
    ("long msl raw scores", 32, 8, 128, 1200, 4096, 0.03, 0.017),
    ("long msl raw scores d64", 16, 4, 64, 700, 2200, 0.021, 0.013),
]


@pytest.mark.parametrize("case", REF_CASES, ids=[c[0] for c in REF_CASES])
def test_reference_contract(dev, case):
    label, hq, hkv, d, pos, msl, qp, kvp = case
    print(f"[decode] reference contract {label}", flush=True)
    qf, kf, vf = oracle.make_attention_case(hq, hkv, d, msl, qp, kvp)
    qb, kb, vb = oracle.f32_to_bf16(qf), oracle.f32_to_bf16(kf), oracle.f32_to_bf16(vf)
    q, k, v = oracle.bf16_to_f32(qb), oracle.bf16_to_f32(kb), oracle.bf16_to_f32(vb)
    score, ob, o = dirty_buffers(hq, d, msl, dev)
    attn.attention_bf16(H.to_dev_bf16(qb, dev), H.to_dev_bf16(kb, dev), H.to_dev_bf16(vb, dev),
                        score, ob, o, hq, hkv, d, pos, msl)
    H.sync()
    check_compat(score, ob, o, q, k, v, pos, msl, label)


@pytest.mark.parametrize("hq,hkv,d,msl,positions", [
    (2, 1, 64, 5, (0, 3)),             # tests/test_cuda_graph_pos.cu:95-96
    (32, 8, 128, 2048, (0, 1500, 37)),  # several splits, partials in score rows
])
def test_graph_replay(dev, hq, hkv, d, msl, positions):
    """Capture attention_bf16_graph once, replay with a new device pos each time."""
    print(f"[decode] graph replay {hq}/{hkv} D={d} msl={msl}", flush=True)
    qf, kf, vf = oracle.make_attention_case(hq, hkv, d, msl, 0.07, 0.03)
    qb, kb, vb = oracle.f32_to_bf16(qf), oracle.f32_to_bf16(kf), oracle.f32_to_bf16(vf)
    q, k, v = oracle.bf16_to_f32(qb), oracle.bf16_to_f32(kb), oracle.bf16_to_f32(vb)
    qd, kd, vd = H.to_dev_bf16(qb, dev), H.to_dev_bf16(kb, dev), H.to_dev_bf16(vb, dev)
    score = torch.ones((hq, msl), dtype=torch.float32, device=dev)
    ob = torch.full((hq, d), -2.0, dtype=torch.float32, device=dev)
    o = torch.full((hq, d), 0.5, dtype=torch.bfloat16, device=dev)
    pos_d = torch.zeros(1, dtype=torch.int32, device=dev)
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        attn.attention_bf16_graph(qd, kd, vd, score, ob, o, hq, hkv, d, pos_d, msl, stream)
    H.sync()
    with torch.cuda.graph(graph, stream=stream):
        attn.attention_bf16_graph(qd, kd, vd, score, ob, o, hq, hkv, d, pos_d, msl, stream)
    for pos in positions:
        pos_d.fill_(pos)
        H.sync()
        graph.replay()
        H.sync()
        check_compat(score, ob, o, q, k, v, pos, msl, f"graph pos={pos}")


def test_reference_contract_engine_cache(dev):
    """The engine's cache size (--max_seq_len=40960, the reference's
    experiment scripts) at Qwen3-8B heads: direct calls at pos 0, 32767 and
    40959, then attention_bf16_graph captured once and replayed at pos
    32767, 0 and 40959 (the partials then sit in the score rows, ~96
    splits).  score, O_buffer and O against the oracle, zero tail checked."""
    hq, hkv, d, msl = 32, 8, 128, 40960
    print(f"[decode] reference contract at msl={msl}", flush=True)
    qf, kf, vf = oracle.make_attention_case(hq, hkv, d, msl, 0.03, 0.017)
    qb, kb, vb = oracle.f32_to_bf16(qf), oracle.f32_to_bf16(kf), oracle.f32_to_bf16(vf)
    q, k, v = oracle.bf16_to_f32(qb), oracle.bf16_to_f32(kb), oracle.bf16_to_f32(vb)
    qd, kd, vd = H.to_dev_bf16(qb, dev), H.to_dev_bf16(kb, dev), H.to_dev_bf16(vb, dev)
    for pos in (0, 32767, msl - 1):
        score, ob, o = dirty_buffers(hq, d, msl, dev)
        attn.attention_bf16(qd, kd, vd, score, ob, o, hq, hkv, d, pos, msl)
        H.sync()
        check_compat(score, ob, o, q, k, v, pos, msl, f"direct pos={pos}")
    score, ob, o = dirty_buffers(hq, d, msl, dev)
    pos_d = torch.zeros(1, dtype=torch.int32, device=dev)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        attn.attention_bf16_graph(qd, kd, vd, score, ob, o, hq, hkv, d, pos_d, msl, stream)
    H.sync()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        attn.attention_bf16_graph(qd, kd, vd, score, ob, o, hq, hkv, d, pos_d, msl, stream)
    for pos in (32767, 0, msl - 1):
        pos_d.fill_(pos)
        H.sync()
        graph.replay()
        H.sync()
        check_compat(score, ob, o, q, k, v, pos, msl, f"graph pos={pos}")


@pytest.mark.parametrize("hq,hkv,d,msl,positions", [
    (2, 1, 64, 5, (0, 3, 4)),               # one split: partials in O_buffer / O rows
    (8, 2, 128, 40, (37, 0)),
    (16, 4, 64, 3001, (2999, 0, 1234)),     # several splits, 4-byte-aligned score rows
    (32, 8, 128, 40960, (32767, 0, 40959)),  # the engine's cache size
])
def test_graph_lean(dev, hq, hkv, d, msl, positions):
    """attention_bf16_graph_lean (the engine's call site, score as scratch):
    captured once, replayed at each device position; O and O_buffer against
    the oracle at the contract's tolerances, O at the north-star bar."""
    print(f"[decode] lean graph {hq}/{hkv} D={d} msl={msl}", flush=True)
    qf, kf, vf = oracle.make_attention_case(hq, hkv, d, msl, 0.03, 0.017)
    qb, kb, vb = oracle.f32_to_bf16(qf), oracle.f32_to_bf16(kf), oracle.f32_to_bf16(vf)
    q, k, v = oracle.bf16_to_f32(qb), oracle.bf16_to_f32(kb), oracle.bf16_to_f32(vb)
    qd, kd, vd = H.to_dev_bf16(qb, dev), H.to_dev_bf16(kb, dev), H.to_dev_bf16(vb, dev)
    score, ob, o = dirty_buffers(hq, d, msl, dev)
    pos_d = torch.zeros(1, dtype=torch.int32, device=dev)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        attn.attention_bf16_graph_lean(qd, kd, vd, score, ob, o, hq, hkv, d, pos_d, msl, stream)
    H.sync()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        attn.attention_bf16_graph_lean(qd, kd, vd, score, ob, o, hq, hkv, d, pos_d, msl, stream)
    for pos in positions:
        pos_d.fill_(pos)
        H.sync()
        graph.replay()
        H.sync()
        _, exp_ob, exp_o = oracle.decode_attention(q, k, v, pos, msl)
        got_o = H.bf16_bits_to_f32(H.from_dev_bf16(o))
        H.check_close(ob.cpu().numpy(), exp_ob, 5e-2, 5e-2, f"lean pos={pos} o_buffer")
        H.check_close(got_o, H.bf16_bits_to_f32(exp_o), 5e-2, 5e-2, f"lean pos={pos} output")
        H.check_bar(got_o, H.bf16_bits_to_f32(exp_o), f"lean pos={pos} output")
        # O is O_buffer rounded to bf16, as in the contract.
        assert np.array_equal(H.from_dev_bf16(o), oracle.f32_to_bf16(ob.cpu().numpy()))


def run_batched(qb, kb, vb, lens, dev, splits=0, seq_lens_on_device=False):
    b, hq, d = qb.shape
    cap, hkv = kb.shape[1], kb.shape[2]
    q, k, v = H.to_dev_bf16(qb, dev), H.to_dev_bf16(kb, dev), H.to_dev_bf16(vb, dev)
    o = torch.full((b, hq, d), 9.0, dtype=torch.bfloat16, device=dev)
    L = int(max(lens))
    s = splits or attn.decode_default_splits(b, hq, hkv, d, L)
    ws = attn.decode_workspace(b, hq, d, s, dev)
    lens_d = (torch.tensor(np.asarray(lens, np.int32), device=dev)
              if seq_lens_on_device else None)
    attn.decode_attention_bf16(q, k, v, o, b, hq, hkv, d, lens_d, L, cap * hkv * d, s, ws)
    H.sync()
    return H.from_dev_bf16(o)


def batched_inputs(seed, b, cap, hq, hkv, d):
    return (synth.normal_bf16(seed, "q", (b, hq, d)),
            synth.normal_bf16(seed, "k", (b, cap, hkv, d)),
            synth.normal_bf16(seed, "v", (b, cap, hkv, d)))


@pytest.mark.parametrize("b,L,hq,hkv,d", [
    (8, 4096, 32, 8, 128),   # config 3
    (1, 32768, 32, 8, 128),  # north-star decode
    (4, 1371, 16, 8, 128),   # Qwen3-0.6B heads
    (2, 333, 8, 8, 64),
    (3, 1, 6, 3, 128),
    (2, 17, 12, 2, 64),
])
def test_batched_vs_oracle(dev, b, L, hq, hkv, d):
    print(f"[decode] batched B={b} L={L} {hq}/{hkv} D={d}", flush=True)
    qb, kb, vb = batched_inputs(100 + L, b, L, hq, hkv, d)
    lens = [L] * b
    exp = oracle.round_bf16(oracle.decode_batched(qb, kb, vb, lens))
    got = H.bf16_bits_to_f32(run_batched(qb, kb, vb, lens, dev))
    mx, mn = H.check_bar(got, exp, f"B={b} L={L}")
    print(f"[decode] max-abs {mx:.3g} mean-abs {mn:.3g}", flush=True)


def test_ragged_lengths_on_device(dev):
    b, cap, hq, hkv, d = 6, 700, 32, 8, 128
    qb, kb, vb = batched_inputs(7, b, cap, hq, hkv, d)
    lens = [1, 16, 17, 128, 129, 700]
    exp = oracle.round_bf16(oracle.decode_batched(qb, kb, vb, lens))
    got = H.bf16_bits_to_f32(run_batched(qb, kb, vb, lens, dev, seq_lens_on_device=True))
    H.check_bar(got, exp, "ragged")


@pytest.mark.parametrize("splits", [1, 3, 8, 40])
def test_split_count_invariance(dev, splits):
    b, L, hq, hkv, d = 2, 4000, 32, 8, 128
    qb, kb, vb = batched_inputs(9, b, L, hq, hkv, d)
    exp = oracle.round_bf16(oracle.decode_batched(qb, kb, vb, [L] * b))
    got = H.bf16_bits_to_f32(run_batched(qb, kb, vb, [L] * b, dev, splits=splits))
    H.check_bar(got, exp, f"splits={splits}")


def test_deterministic(dev):
    qb, kb, vb = batched_inputs(10, 8, 2048, 32, 8, 128)
    a = run_batched(qb, kb, vb, [2048] * 8, dev)
    b2 = run_batched(qb, kb, vb, [2048] * 8, dev)
    assert np.array_equal(a, b2)


def test_workspace_reused_across_shapes(dev):
    """One workspace, filled with garbage first, serves calls of different shapes in turn."""
    shapes = [(4, 3000, 32, 8, 128), (1, 20000, 16, 8, 128), (3, 77, 6, 3, 64),
              (4, 3000, 32, 8, 128)]
    big = max(attn.decode_workspace_bytes(b, hq, d, attn.decode_default_splits(b, hq, hkv, d, L))
              for b, L, hq, hkv, d in shapes)
    ws = torch.full((big,), 0x7F, dtype=torch.uint8, device=dev)
    for i, (b, L, hq, hkv, d) in enumerate(shapes):
        qb, kb, vb = batched_inputs(40 + i, b, L, hq, hkv, d)
        q, k, v = H.to_dev_bf16(qb, dev), H.to_dev_bf16(kb, dev), H.to_dev_bf16(vb, dev)
        o = torch.empty((b, hq, d), dtype=torch.bfloat16, device=dev)
        s = attn.decode_default_splits(b, hq, hkv, d, L)
        attn.decode_attention_bf16(q, k, v, o, b, hq, hkv, d, None, L, L * hkv * d, s, ws)
        H.sync()
        exp = oracle.round_bf16(oracle.decode_batched(qb, kb, vb, [L] * b))
        H.check_bar(H.bf16_bits_to_f32(H.from_dev_bf16(o)), exp, f"shape {i}")


def test_kv_permutation_invariance(dev):
    """Decode attends to a set: permuting cached rows leaves O unchanged
    (up to fp32 summation order)."""
    b, L, hq, hkv, d = 1, 1000, 16, 8, 128
    qb, kb, vb = batched_inputs(12, b, L, hq, hkv, d)
    perm = np.random.default_rng(0).permutation(L)
    a = H.bf16_bits_to_f32(run_batched(qb, kb, vb, [L], dev))
    p = H.bf16_bits_to_f32(run_batched(qb, kb[:, perm].copy(), vb[:, perm].copy(), [L], dev))
    H.check_bar(p, a, "permuted", max_abs=8e-3, mean_abs=5e-4)


def test_workspace_too_small_is_rejected(dev):
    qb, kb, vb = batched_inputs(13, 1, 256, 8, 8, 128)
    q, k, v = H.to_dev_bf16(qb, dev), H.to_dev_bf16(kb, dev), H.to_dev_bf16(vb, dev)
    o = torch.empty((1, 8, 128), dtype=torch.bfloat16, device=dev)
    ws = torch.empty(64, dtype=torch.uint8, device=dev)
    with pytest.raises(attn.ToyInferError) as e:
        attn.decode_attention_bf16(q, k, v, o, 1, 8, 8, 128, None, 256, 256 * 8 * 128, 4, ws)
    assert e.value.status == attn.ERR_WORKSPACE


def test_cache_rows_past_length_are_not_read(dev):
    """Cache rows at and after each sequence's length hold NaN; outputs stay exact."""
    b, cap, hq, hkv, d = 3, 600, 32, 8, 128
    qb, kb, vb = batched_inputs(14, b, cap, hq, hkv, d)
    lens = [1, 300, 517]
    kn, vn = kb.copy(), vb.copy()
    for i, L in enumerate(lens):
        kn[i, L:] = 0x7FC0
        vn[i, L:] = 0x7FC0
    exp = oracle.round_bf16(oracle.decode_batched(qb, kb, vb, lens))
    got = H.bf16_bits_to_f32(run_batched(qb, kn, vn, lens, dev, seq_lens_on_device=True))
    H.check_bar(got, exp, "NaN past length")
