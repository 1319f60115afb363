"""Prefill parity: the HIP kernel through the C ABI vs the CPU oracle.

Cases follow tests/test_flash_attention_v1_bf16.cu:108-131 (deterministic
sin/cos inputs, its tolerances), then seeded N(0,1) inputs at the benchmark
shapes, ragged lengths, every GQA ratio the reference exercises, and
invariants that hold at any size.
"""
import numpy as np
import pytest
import torch

import oracle
from tests import helpers as H
from toyinfer_amd import attn, synth

pytestmark = pytest.mark.gpu


ALGOS = [attn.ALGO_SPLIT_KEYS, attn.ALGO_ROW_TILES, attn.ALGO_SPLIT_PAIRS, attn.ALGO_ROW_PAIRS]


def run_prefill(q_bits, k_bits, v_bits, dev, algo=attn.ALGO_AUTO):
    s, hq, d = q_bits.shape
    hkv = k_bits.shape[1]
    q = H.to_dev_bf16(q_bits, dev)
    k = H.to_dev_bf16(k_bits, dev)
    v = H.to_dev_bf16(v_bits, dev)
    o = torch.full((s, hq, d), -3.0, dtype=torch.bfloat16, device=dev)
    if algo == attn.ALGO_AUTO:
        attn.flash_attention_v1_bf16(q, k, v, o, hq, hkv, d, s)
    else:
        attn.flash_attention_algo_bf16(q, k, v, o, hq, hkv, d, s, algo)
    H.sync()
    return H.from_dev_bf16(o)


# tests/test_flash_attention_v1_bf16.cu:113-131: (label, Hq, Hkv, D, S,
# q_phase, kv_phase, scales, atol=rtol)
REF_CASES = [
    ("seq1 gqa", 2, 1, 64, 1, 0.07, 0.03, (1.0, 1.0, 1.0), 7e-2),
    ("exact-kv-tile", 4, 4, 64, 32, 0.05, 0.021, (1.0, 1.0, 1.0), 7e-2),
    ("gqa tail-tiles", 8, 2, 128, 37, 0.033, 0.017, (1.0, 1.0, 1.0), 7e-2),
    ("multi-kv-tile", 6, 3, 128, 65, 0.028, 0.019, (1.0, 1.0, 1.0), 7e-2),
    ("large-magnitude", 4, 2, 64, 19, 0.061, 0.027, (12.0, 10.0, 1.7), 1.2),
]


@pytest.mark.parametrize("algo", [attn.ALGO_AUTO] + ALGOS)
@pytest.mark.parametrize("case", REF_CASES, ids=[c[0] for c in REF_CASES])
def test_reference_cases(dev, case, algo):
    label, hq, hkv, d, s, qp, kvp, (qs, ks_, vs), tol = case
    print(f"[prefill] reference case {label} algo={algo}", flush=True)
    q, k, v = oracle.make_flash_case(hq, hkv, d, s, qp, kvp, qs, ks_, vs)
    qb, kb, vb = oracle.f32_to_bf16(q), oracle.f32_to_bf16(k), oracle.f32_to_bf16(v)
    exp = oracle.round_bf16(oracle.flash_reference(qb, kb, vb))
    got = H.bf16_bits_to_f32(run_prefill(qb, kb, vb, dev, algo))
    H.check_close(got, exp, tol, tol, label)
    H.check_bar(got, exp, label)


def test_causal_focus_case(dev):
    """tests/test_flash_attention_v1_bf16.cu:11-45, tolerance 9e-2."""
    q, k, v = oracle.make_causal_focus_case()
    qb, kb, vb = oracle.f32_to_bf16(q), oracle.f32_to_bf16(k), oracle.f32_to_bf16(v)
    exp = oracle.round_bf16(oracle.flash_reference(qb, kb, vb))
    got = H.bf16_bits_to_f32(run_prefill(qb, kb, vb, dev))
    H.check_close(got, exp, 9e-2, 9e-2, "causal-focus")
    H.check_bar(got, exp, "causal-focus")


def seeded(seed, s, hq, hkv, d):
    return (synth.normal_bf16(seed, "q", (s, hq, d)), synth.normal_bf16(seed, "k", (s, hkv, d)),
            synth.normal_bf16(seed, "v", (s, hkv, d)))


@pytest.mark.parametrize("algo", ALGOS)
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("hq,hkv", [(2, 1), (4, 4), (6, 3), (8, 2), (6, 2)])
@pytest.mark.parametrize("s", [1, 2, 31, 33, 63, 64, 65, 127, 129, 200])
def test_ragged_shapes(dev, s, hq, hkv, d, algo):
    print(f"[prefill] ragged S={s} Hq={hq} Hkv={hkv} D={d} algo={algo}", flush=True)
    qb, kb, vb = seeded(11 + s, s, hq, hkv, d)
    exp = oracle.round_bf16(oracle.flash_reference(qb, kb, vb))
    got = H.bf16_bits_to_f32(run_prefill(qb, kb, vb, dev, algo))
    H.check_bar(got, exp, f"S={s} {hq}/{hkv} D={d} algo={algo}")


@pytest.mark.parametrize("algo", ALGOS)
@pytest.mark.parametrize("s", [1, 45, 128, 200])
def test_rows_past_s_are_not_read(dev, s, algo):
    """K/V memory right after row S-1 holds NaN; no output may see it."""
    hq, hkv, d = 8, 2, 128
    qb, kb, vb = seeded(21 + s, s, hq, hkv, d)
    nan = np.full((130, hkv, d), 0x7FC0, np.uint16)
    k_full = H.to_dev_bf16(np.concatenate([kb, nan]), dev)
    v_full = H.to_dev_bf16(np.concatenate([vb, nan]), dev)
    q = H.to_dev_bf16(qb, dev)
    o = torch.empty((s, hq, d), dtype=torch.bfloat16, device=dev)
    attn.flash_attention_algo_bf16(q, k_full[:s], v_full[:s], o, hq, hkv, d, s, algo)
    H.sync()
    got = H.bf16_bits_to_f32(H.from_dev_bf16(o))
    exp = oracle.round_bf16(oracle.flash_reference(qb, kb, vb))
    H.check_bar(got, exp, f"NaN tail S={s} algo={algo}")


def test_config1_seeded(dev):
    """Config 1 shape (S=128, 16/8, D=128), seeded N(0,1), vs oracle."""
    qb, kb, vb = seeded(1, 128, 16, 8, 128)
    exp = oracle.round_bf16(oracle.flash_reference(qb, kb, vb))
    got = H.bf16_bits_to_f32(run_prefill(qb, kb, vb, dev))
    H.check_bar(got, exp, "config1")


@pytest.mark.parametrize("algo", [attn.ALGO_AUTO] + ALGOS)
def test_config2_full(dev, algo):
    """Config 2 (S=1371, 16/8, D=128): every output element vs the oracle."""
    print(f"[prefill] config2 S=1371 algo={algo}", flush=True)
    qb, kb, vb = seeded(2, 1371, 16, 8, 128)
    exp = oracle.round_bf16(oracle.flash_reference(qb, kb, vb))
    got = H.bf16_bits_to_f32(run_prefill(qb, kb, vb, dev, algo))
    mx, mn = H.check_bar(got, exp, "config2")
    print(f"[prefill] config2 max-abs {mx:.3g} mean-abs {mn:.3g}", flush=True)


def extreme_case(kind, s, hq, hkv, d):
    """Scores far outside what a fixed softmax reference could hold.

    "negative"/"positive": every key row is -u / +u and every query row 12u,
    so each row's scores are all equal, about -/+226 in log2 units here
    (2^226 overflows fp32; 2^-226 underflows): the output is the mean of V
    over the row's visible keys.  "wide": q, k ~ 4 N(0,1), score spread of
    about +-80 in log2 units within a row.
    """
    v = synth.normal_bf16(31, "v", (s, hkv, d))
    if kind == "wide":
        q = oracle.f32_to_bf16(4.0 * oracle.bf16_to_f32(synth.normal_bf16(31, "q", (s, hq, d))))
        k = oracle.f32_to_bf16(4.0 * oracle.bf16_to_f32(synth.normal_bf16(31, "k", (s, hkv, d))))
        return q, k, v
    u = oracle.bf16_to_f32(synth.normal_bf16(31, "u", (d,)))
    sign = -1.0 if kind == "negative" else 1.0
    q = oracle.f32_to_bf16(np.broadcast_to(12.0 * u, (s, hq, d)).astype(np.float32))
    k = oracle.f32_to_bf16(np.broadcast_to(sign * u, (s, hkv, d)).astype(np.float32))
    return q, k, v


@pytest.mark.parametrize("algo", ALGOS)
@pytest.mark.parametrize("kind", ["negative", "positive", "wide"])
def test_extreme_scores(dev, kind, algo):
    """Rows whose scores overflow or underflow exp2 without a running maximum
    (the kernels' reference for the exponentials moves only when a tile's
    probabilities would leave range): vs the oracle and, for equal scores,
    vs the prefix mean of V."""
    s, hq, hkv, d = 700, 4, 2, 128
    print(f"[prefill] extreme scores {kind} algo={algo}", flush=True)
    qb, kb, vb = extreme_case(kind, s, hq, hkv, d)
    got = H.bf16_bits_to_f32(run_prefill(qb, kb, vb, dev, algo))
    exp = oracle.round_bf16(oracle.flash_reference(qb, kb, vb))
    H.check_bar(got, exp, f"{kind} algo={algo}")
    if kind != "wide":
        vf = oracle.bf16_to_f32(vb).astype(np.float64)
        mean = np.cumsum(vf, axis=0) / np.arange(1, s + 1)[:, None, None]
        mean = np.repeat(mean, hq // hkv, axis=1)
        H.check_bar(got, oracle.round_bf16(mean.astype(np.float32)), f"{kind} prefix mean")


@pytest.mark.parametrize("s,hq,hkv,d", [(3000, 32, 8, 128), (2600, 16, 4, 64)])
def test_algos_agree_at_long_s(dev, s, hq, hkv, d):
    """Both kernels agree closely on problems with several times more query
    tiles than the split kernel keeps resident (its workgroups then walk
    several work items each)."""
    print(f"[prefill] split vs rows S={s} {hq}/{hkv} D={d}", flush=True)
    qb, kb, vb = seeded(3, s, hq, hkv, d)
    a = H.bf16_bits_to_f32(run_prefill(qb, kb, vb, dev, attn.ALGO_SPLIT_KEYS))
    b = H.bf16_bits_to_f32(run_prefill(qb, kb, vb, dev, attn.ALGO_ROW_TILES))
    c = H.bf16_bits_to_f32(run_prefill(qb, kb, vb, dev, attn.ALGO_SPLIT_PAIRS))
    H.check_bar(a, b, "split vs rows", max_abs=1.6e-2, mean_abs=3e-4)
    H.check_bar(c, b, "split pairs vs rows", max_abs=1.6e-2, mean_abs=3e-4)


@pytest.mark.parametrize("s,hq,hkv,d", [(700, 8, 2, 128), (1000, 32, 8, 128), (333, 16, 4, 64),
                                         (129, 4, 2, 128), (4096, 32, 8, 128), (4100, 32, 8, 128),
                                         (2049, 16, 4, 64)])
def test_row_pairs_equal_row_tiles_bitwise(dev, s, hq, hkv, d):
    """The 128-row kernel with a GQA head pair per workgroup computes every
    row as the single-head kernel does (same tiles in the same order): the
    outputs are equal bit for bit."""
    print(f"[prefill] row pairs vs row tiles S={s} {hq}/{hkv} D={d}", flush=True)
    qb, kb, vb = seeded(9, s, hq, hkv, d)
    a = run_prefill(qb, kb, vb, dev, attn.ALGO_ROW_TILES)
    b = run_prefill(qb, kb, vb, dev, attn.ALGO_ROW_PAIRS)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("algo", ALGOS)
def test_deterministic(dev, algo):
    qb, kb, vb = seeded(5, 700, 8, 2, 128)
    a = run_prefill(qb, kb, vb, dev, algo)
    b = run_prefill(qb, kb, vb, dev, algo)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("algo", ALGOS)
def test_gqa_equals_mha_with_repeated_kv(dev, algo):
    """GQA output == the output on K/V heads repeated (bitwise): G times (MHA)
    for the kernels that run each head alone, twice (G = 2) for the pair
    kernels, whose workgroups hold a head pair."""
    qb, kb, vb = seeded(6, 300, 8, 2, 128)
    rep = 2 if algo in (attn.ALGO_SPLIT_PAIRS, attn.ALGO_ROW_PAIRS) else 4
    gqa = run_prefill(qb, kb, vb, dev, algo)
    mha = run_prefill(qb, np.repeat(kb, rep, axis=1), np.repeat(vb, rep, axis=1), dev, algo)
    assert np.array_equal(gqa, mha)


@pytest.mark.parametrize("algo", ALGOS)
def test_row0_is_v_row0(dev, algo):
    """Causal row 0 attends only to key 0: O[0] == V[0] exactly."""
    qb, kb, vb = seeded(7, 96, 4, 2, 64)
    got = run_prefill(qb, kb, vb, dev, algo)
    assert np.array_equal(got[0], np.repeat(vb[0], 2, axis=0))


@pytest.mark.parametrize("algo", ALGOS)
def test_prefix_independence(dev, algo):
    """Causality: rows < S' of a length-S run equal a length-S' run."""
    qb, kb, vb = seeded(8, 400, 8, 2, 128)
    full = run_prefill(qb, kb, vb, dev, algo)
    part = run_prefill(qb[:257].copy(), kb[:257].copy(), vb[:257].copy(), dev, algo)
    assert np.array_equal(full[:257], part)


def test_rejects_bad_arguments(dev):
    q = torch.zeros((4, 4, 128), dtype=torch.bfloat16, device=dev)
    k = torch.zeros((4, 3, 128), dtype=torch.bfloat16, device=dev)
    with pytest.raises(attn.ToyInferError) as e:
        attn.flash_attention_v1_bf16(q, k, k, q, 4, 3, 128, 4)
    assert e.value.status == attn.ERR_INVALID_ARGUMENT
    with pytest.raises(attn.ToyInferError) as e:
        attn.flash_attention_v1_bf16(q, k, k, q, 4, 4, 96, 4)
    assert e.value.status == attn.ERR_UNSUPPORTED
