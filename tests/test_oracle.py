"""Pins the CPU oracle (oracle/) on the CPU, before it is trusted as the checker.

Each oracle function is checked against something other than its own
formula: the golden fixtures (torch float64, tests/golden/make_golden.py),
closed forms, invariants, brute force in numpy float64, torch's SDPA, and
the literal cases held by the reference's own tests.
"""
import hashlib
import os

import numpy as np
import pytest

import oracle
from tests import helpers as H
from toyinfer_amd import synth

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def gold(name):
    return np.load(os.path.join(GOLD, name + ".npz"))


def sha(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def bf16_ulp_diff(a_bits, b_bits):
    """|a - b| in units of one bf16 ulp at the larger magnitude (2^-7 relative
    upper bound), with differences under 1e-6 absolute counted as 0."""
    a, b = H.bf16_bits_to_f32(a_bits), H.bf16_bits_to_f32(b_bits)
    diff = np.abs(a.astype(np.float64) - b)
    ulp = np.maximum(np.abs(a), np.abs(b)).astype(np.float64) * 2.0 ** -7
    return np.where(diff <= 1e-6, 0, np.ceil(diff / np.maximum(ulp, 1e-30))).astype(np.int64)


# ------------------------------------------------------------------ bf16

def test_bf16_rounding_matches_torch():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(0)
    specials = np.array([0.0, -0.0, 1.0, -1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 1.0 + 2 ** -9,
                         1.0 + 2 ** -9 + 2 ** -20, 3.0e38, 3.4028235e38, 1e-40, -1e-42,
                         np.inf, -np.inf, 65504.0, 1e-30], np.float32)
    ties = (np.arange(1 << 16, dtype=np.uint32) << 16 | 0x8000).view(np.float32)  # exact ties
    vals = np.concatenate([specials, ties[np.isfinite(ties)],
                           rng.standard_normal(200000).astype(np.float32) * 10 ** rng.uniform(
                               -30, 30, 200000).astype(np.float32)])
    ours = oracle.f32_to_bf16(vals)
    ref = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, ref)
    nan = oracle.f32_to_bf16(np.array([np.nan, -np.nan], np.float32))
    assert np.all((nan & 0x7F80) == 0x7F80) and np.all(nan & 0x7F)
    assert np.array_equal(synth.f32_to_bf16_bits(vals), ours)


# --------------------------------------------------------------- prefill

PREFILL_CASES = ["seq1_gqa", "exact_kv_tile", "gqa_tail_tiles", "multi_kv_tile",
                 "large_magnitude", "causal_focus"]


@pytest.mark.parametrize("name", PREFILL_CASES)
def test_flash_vs_golden(name):
    g = gold("prefill_" + name)
    o = oracle.flash_reference(g["q"], g["k"], g["v"])
    scale = max(1.0, float(np.abs(g["o"]).max()))
    assert np.abs(o - g["o"]).max() <= 2e-6 * scale
    ulps = bf16_ulp_diff(oracle.f32_to_bf16(o), g["o_bf16"])
    assert ulps.max() <= 1 and (ulps > 0).mean() < 1e-3


def test_case_generators_reproduce_golden_inputs():
    """The restated case formulas give the inputs the fixtures were made from."""
    q, k, v = oracle.make_flash_case(6, 3, 128, 65, 0.028, 0.019)
    g = gold("prefill_multi_kv_tile")
    assert np.array_equal(oracle.f32_to_bf16(q), g["q"])
    assert np.array_equal(oracle.f32_to_bf16(k), g["k"])
    assert np.array_equal(oracle.f32_to_bf16(v), g["v"])


def test_flash_config1_vs_golden():
    g = gold("prefill_config1")
    qb = synth.normal_bf16(int(g["seed"]), "q", (128, 16, 128))
    kb = synth.normal_bf16(int(g["seed"]), "k", (128, 8, 128))
    vb = synth.normal_bf16(int(g["seed"]), "v", (128, 8, 128))
    assert sha(qb, kb, vb) == str(g["inputs_sha256"]), "synthetic generator drifted"
    ulps = bf16_ulp_diff(oracle.f32_to_bf16(oracle.flash_reference(qb, kb, vb)), g["o_bf16"])
    assert ulps.max() <= 1 and (ulps > 0).mean() < 1e-3


def test_flash_matches_torch_sdpa():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(1)
    s, hq, hkv, d = 50, 6, 2, 64
    q, k, v = (oracle.round_bf16(rng.standard_normal(sh).astype(np.float32))
               for sh in [(s, hq, d), (s, hkv, d), (s, hkv, d)])
    ours = oracle.flash_reference(q, k, v)
    tq = torch.from_numpy(q).double().permute(1, 0, 2)
    tk = torch.from_numpy(k).double().repeat_interleave(3, 1).permute(1, 0, 2)
    tv = torch.from_numpy(v).double().repeat_interleave(3, 1).permute(1, 0, 2)
    ref = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, is_causal=True)
    assert np.abs(ours - ref.permute(1, 0, 2).numpy()).max() < 2e-6


def test_flash_brute_force_tiny():
    rng = np.random.default_rng(2)
    s, hq, hkv, d = 7, 4, 2, 8
    q, k, v = (rng.standard_normal(sh).astype(np.float32) for sh in
               [(s, hq, d), (s, hkv, d), (s, hkv, d)])
    ours = oracle.flash_reference(q, k, v)
    for t in range(s):
        for h in range(hq):
            kv = h // 2
            sc = np.array([np.dot(q[t, h].astype(np.float64), k[j, kv]) for j in range(t + 1)])
            w = np.exp(sc / np.sqrt(d) - (sc / np.sqrt(d)).max())
            w /= w.sum()
            exp = (w[:, None] * v[: t + 1, kv].astype(np.float64)).sum(0)
            assert np.abs(ours[t, h] - exp).max() < 1e-6


def test_flash_row0_is_v0_and_constant_keys_give_prefix_mean():
    rng = np.random.default_rng(3)
    s, hq, hkv, d = 40, 4, 2, 32
    q = rng.standard_normal((s, hq, d)).astype(np.float32)
    v = rng.standard_normal((s, hkv, d)).astype(np.float32)
    k = np.repeat(rng.standard_normal((1, hkv, d)).astype(np.float32), s, 0)
    o = oracle.flash_reference(q, k, v)
    assert np.array_equal(o[0], np.repeat(v[0], 2, 0))
    prefix_mean = np.cumsum(v.astype(np.float64), 0) / np.arange(1, s + 1)[:, None, None]
    assert np.abs(o - np.repeat(prefix_mean, 2, 1)).max() < 1e-5


def test_flash_dominant_key_selects_its_value():
    s, hq, hkv, d = 12, 2, 1, 16
    q = np.zeros((s, hq, d), np.float32)
    q[:, :, 0] = 40.0
    k = np.zeros((s, hkv, d), np.float32)
    k[:, 0, 0] = np.arange(s, dtype=np.float32)    # score grows by 40/4 per key
    v = np.random.default_rng(4).standard_normal((s, hkv, d)).astype(np.float32)
    o = oracle.flash_reference(q, k, v)
    # query t sees keys 0..t; key t wins by >= 10 nats over key t-1
    assert np.abs(o[:, 0] - v[:, 0]).max() < 1e-3


def test_flash_gqa_equals_mha_and_shift_invariance():
    rng = np.random.default_rng(5)
    s, hq, hkv, d = 30, 8, 2, 64
    q, k, v = (rng.standard_normal(sh).astype(np.float32) for sh in
               [(s, hq, d), (s, hkv, d), (s, hkv, d)])
    a = oracle.flash_reference(q, k, v)
    b = oracle.flash_reference(q, np.repeat(k, 4, 1), np.repeat(v, 4, 1))
    assert np.array_equal(a, b)
    u = rng.standard_normal((1, hkv, d)).astype(np.float32)  # adds q.u to every score of q
    c = oracle.flash_reference(q, k + u, v)
    assert np.abs(a - c).max() < 1e-5


def test_flash_row_subset_matches_full():
    rng = np.random.default_rng(6)
    s, hq, hkv, d = 90, 4, 1, 32
    q, k, v = (rng.standard_normal(sh).astype(np.float32) for sh in
               [(s, hq, d), (s, hkv, d), (s, hkv, d)])
    full = oracle.flash_reference(q, k, v)
    rows = [0, 5, 61, 89]
    part = oracle.flash_reference(q, k, v, rows=rows)
    assert np.array_equal(part[rows], full[rows])
    assert np.isnan(part[1]).all()


# ---------------------------------------------------------------- decode

@pytest.mark.parametrize("name", ["pos0_gqa", "full_kv", "tiled_seq"])
def test_decode_vs_golden(name):
    g = gold("decode_" + name)
    q, k, v = (oracle.bf16_to_f32(g[x]) for x in "qkv")
    pos, msl = int(g["pos"]), g["score"].shape[1]
    score, ob, o = oracle.decode_attention(q, k, v, pos, msl)
    assert np.abs(score - g["score"]).max() < 1e-6
    assert np.all(score[:, pos + 1:] == 0)
    assert np.abs(ob - g["o"]).max() < 2e-6
    ulps = bf16_ulp_diff(o, g["o_bf16"])
    assert ulps.max() <= 1


def test_decode_batched_vs_golden():
    g = gold("decode_seeded")
    sd = int(g["seed"])
    qb = synth.normal_bf16(sd, "q", (2, 8, 128))
    kb = synth.normal_bf16(sd, "k", (2, 300, 2, 128))
    vb = synth.normal_bf16(sd, "v", (2, 300, 2, 128))
    assert sha(qb, kb, vb) == str(g["inputs_sha256"])
    o = oracle.decode_batched(qb, kb, vb, g["lens"])
    assert np.abs(o - g["o"]).max() < 2e-6


def test_softmax_reference_literal_cases():
    """tests/test_softmax_f32_kernel.cu:42-60, against scipy in float64."""
    from scipy.special import softmax

    rng_i = np.arange(24)
    mixed = (-2.5 + 0.37 * np.sin((rng_i + 1) * 0.19) + 0.11 * (rng_i % 7)).astype(np.float32)
    cases = [(2, 0, 5, np.array([1.25, -9.0, 3.0, 4.0, -2.0, -0.5, 7.0, -1.0, 2.0, 3.0],
                                np.float32)),
             (3, 5, 8, mixed),
             (2, 4, 7, np.array([80.0, 81.5, 79.25, 90.0, 88.0, -3.0, 4.0, -45.0, -44.5, -46.25,
                                 -41.0, -42.0, 6.0, -7.0], np.float32))]
    for hq, pos, msl, sc in cases:
        sc = sc.reshape(hq, msl)
        out = oracle.decode_softmax(sc, pos)
        exp = softmax(sc[:, : pos + 1].astype(np.float64), axis=1)
        assert np.abs(out[:, : pos + 1] - exp).max() < 1e-6
        assert np.array_equal(out[:, pos + 1:], sc[:, pos + 1:])
        assert np.abs(out[:, : pos + 1].sum(1) - 1).max() < 1e-6


def test_decode_qk_accumulates_onto_initial_score():
    """tests/test_gqa_qk_gemv_bf16_kernel.cu:25-31: scores add onto a dirty buffer."""
    q, k, _ = oracle.make_attention_case(8, 2, 128, 12, 0.03, 0.017)
    q, k = oracle.round_bf16(q), oracle.round_bf16(k)
    init = (-0.45 + 0.03 * ((np.arange(8 * 12) * 7) % 13)).astype(np.float32).reshape(8, 12)
    out = oracle.decode_qk_scores(q, k, init, 9, 12)
    exp = init.astype(np.float64).copy()
    for h in range(8):
        for t in range(10):
            exp[h, t] += np.dot(q[h].astype(np.float64), k[t, h // 4]) / np.sqrt(128)
    assert np.abs(out - exp).max() < 1e-5


def test_decode_apply_accumulates_onto_initial_o():
    """tests/test_apply_score2v_f32_kernel.cu:59-75 (single-tile case)."""
    _, _, v = oracle.make_attention_case(4, 2, 64, 8, 0.04, 0.02)
    v = oracle.round_bf16(v)
    score = np.zeros((4, 8), np.float32)
    for h in range(4):
        for t in range(4):
            score[h, t] = 0.12 + 0.03 * ((h + t) % 5)
    init = (0.6 - 0.04 * ((np.arange(4 * 64) * 3) % 17)).astype(np.float32).reshape(4, 64)
    out = oracle.decode_apply(score, v, init, 3)
    exp = init.astype(np.float64) + np.einsum("ht,thd->hd", score[:, :4].astype(np.float64),
                                              np.repeat(v[:4], 2, 1).astype(np.float64))
    assert np.abs(out - exp).max() < 1e-5


def test_decode_equals_last_prefill_row_and_is_permutation_invariant():
    rng = np.random.default_rng(7)
    L, hq, hkv, d = 60, 8, 2, 64
    q = oracle.round_bf16(rng.standard_normal((L, hq, d)).astype(np.float32))
    k = oracle.round_bf16(rng.standard_normal((L, hkv, d)).astype(np.float32))
    v = oracle.round_bf16(rng.standard_normal((L, hkv, d)).astype(np.float32))
    pre = oracle.flash_reference(q, k, v)[L - 1]
    _, ob, _ = oracle.decode_attention(q[L - 1], k, v, L - 1, L)
    assert np.abs(pre - ob).max() < 1e-5
    perm = rng.permutation(L)
    _, obp, _ = oracle.decode_attention(q[L - 1], k[perm], v[perm], L - 1, L)
    assert np.abs(ob - obp).max() < 1e-5


# ------------------------------------------------ QK-norm, RoPE, inv_freq

def test_inv_freq_closed_forms():
    f = oracle.inv_freq(128, 1e6)
    assert f[0] == 1.0
    exp = 1.0 / np.power(1e6, 2.0 * np.arange(64) / 128)
    assert np.abs(f / exp - 1).max() < 1e-6
    assert np.all(oracle.inv_freq(258, 1.0) == 1.0)      # theta 1 (reference case)
    assert np.allclose(oracle.inv_freq(2, 2.0), [1.0])


def test_rmsnorm_constant_row_and_vs_float64():
    w = oracle.round_bf16(np.linspace(0.9, 1.1, 64).astype(np.float32))
    x = np.full(64, -0.75, np.float32)
    y = oracle.multi_rmsnorm(x, w, 64, 1e-6)
    assert np.abs(y - oracle.round_bf16(-w / np.sqrt(1 + 1e-6 / 0.5625))).max() == 0
    x, w = oracle.make_rmsnorm_case(4, 128, 4 * 128, 0.09, 0.05)
    xq, wq = oracle.round_bf16(x), oracle.round_bf16(w)
    y = oracle.multi_rmsnorm(xq, wq, 128, 1e-5).reshape(4, 128)
    x64 = xq.reshape(4, 128).astype(np.float64)
    exp = x64 / np.sqrt((x64 ** 2).mean(1, keepdims=True) + 1e-5) * wq
    ulps = bf16_ulp_diff(oracle.f32_to_bf16(y), oracle.f32_to_bf16(exp.astype(np.float32)))
    assert ulps.max() <= 1


def test_rope_position0_identity_and_vs_float64():
    qk, f = oracle.make_rope_case(4, 128, 4 * 128, 0.021, 0.0)
    f = oracle.inv_freq(128, 10000.0)
    x = oracle.round_bf16(qk).reshape(1, 4, 128)
    assert np.array_equal(oracle.rope(x, f, 1, 4, 128), x)
    x5 = np.repeat(x, 37, 0)
    out = oracle.rope(x5, f, 37, 4, 128)
    ang = (np.arange(37, dtype=np.float32)[:, None] * f[None, :]).astype(np.float64)
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    re, im = x5[..., :64].astype(np.float64), x5[..., 64:].astype(np.float64)
    exp = np.concatenate([re * c - im * s, im * c + re * s], -1).astype(np.float32)
    assert bf16_ulp_diff(oracle.f32_to_bf16(out), oracle.f32_to_bf16(exp)).max() <= 1


def test_qk_norm_rope_and_fused_attention_vs_golden():
    g = gold("fused_small")
    sd = int(g["seed"])
    s, hq, hkv, d = 96, 4, 2, 128
    qb = synth.normal_bf16(sd, "q", (s, hq, d))
    kb = synth.normal_bf16(sd, "k", (s, hkv, d))
    vb = synth.normal_bf16(sd, "v", (s, hkv, d))
    gq = synth.uniform_bf16(sd, "gamma_q", (d,), 0.9, 1.1)
    gk = synth.uniform_bf16(sd, "gamma_k", (d,), 0.9, 1.1)
    assert sha(qb, kb, vb, gq, gk) == str(g["inputs_sha256"])
    f = oracle.inv_freq(d, float(g["theta"]))
    kn = oracle.qk_norm_rope(oracle.bf16_to_f32(kb), oracle.bf16_to_f32(gk), f, float(g["eps"]))
    qn = oracle.qk_norm_rope(oracle.bf16_to_f32(qb), oracle.bf16_to_f32(gq), f, float(g["eps"]))
    # A 1-ulp difference after the norm's rounding (float32 vs float64 sums)
    # enters both inputs of a rotation, so 2 ulps can appear after RoPE.
    for ours, ref in [(kn, g["k_norm_rope"]), (qn, g["q_norm_rope"])]:
        ulps = bf16_ulp_diff(oracle.f32_to_bf16(ours), ref)
        assert ulps.max() <= 2 and (ulps > 0).mean() < 5e-3
    o = oracle.round_bf16(oracle.flash_reference(qn, kn, oracle.bf16_to_f32(vb)))
    H.check_bar(o, H.bf16_bits_to_f32(g["o_bf16"]), "fused oracle vs golden",
                max_abs=1e-2, mean_abs=2e-4)


# ------------------------------------------------------------ projections

def test_gemv_case_generators_literal_values():
    """The case generators against the formulas of tests/gemv_test_common.h:33-48
    and tests/test_batch_gemv_proj_bf16.cu:31-49 evaluated in float64."""
    import math
    x, w = oracle.make_gemv_case(5, 7, 0.17, 0.01)
    for i in (0, 3, 6):
        e = 0.45 * math.sin((i + 1) * 0.17) - 0.18 * math.cos((i + 3) * 0.17 * 0.7) + 0.01 * (i % 5)
        assert abs(x[i] - e) < 1e-6
    for r, c in ((0, 0), (4, 6), (2, 5)):
        e = (0.35 * math.cos((r + 1) * (c + 1) * 0.01) + 0.22 * math.sin((r + c + 3) * 0.006)
             - 0.015 * ((r * 7 + c * 3) % 9))
        assert abs(w[r, c] - e) < 1e-6
    h, w = oracle.make_batch_gemv_case(3, 4, 6, 0.19, 0.12)
    for b, c in ((0, 0), (2, 5), (1, 3)):
        idx = b * 6 + c
        e = (0.47 * math.sin((idx + 1) * 0.19) - 0.18 * math.cos((idx + c + 3) * 0.19 * 0.9)
             + 0.02 * ((b + c) % 6))
        assert abs(h[b, c] - e) < 1e-6
    for r, c in ((0, 0), (3, 5)):
        e = (0.33 * math.cos((r + 1) * (c + 1) * 0.12) + 0.21 * math.sin((r + 2) * (c + 3) * 0.06)
             - 0.012 * ((r * 5 + c * 7) % 11))
        assert abs(w[r, c] - e) < 1e-6


def test_gemv_vs_float64_and_closed_forms():
    """Float accumulation in column order stays within float rounding of the
    float64 product; unit rows pick one element exactly; token rows are
    independent; the OpenMP split gives the same bits."""
    x, w = oracle.make_gemv_case(513, 514, 0.05, 0.004)
    y = oracle.gemv(w, x)
    ref = w.astype(np.float64) @ x.astype(np.float64)
    bound = 514 * 2.0 ** -23 * (np.abs(w).astype(np.float64) @ np.abs(x).astype(np.float64))
    assert (np.abs(y - ref) <= bound + 1e-30).all()
    eye = np.zeros((4, 514), np.float32)
    for k, col in enumerate((0, 7, 300, 513)):
        eye[k, col] = 1.0
    assert np.array_equal(oracle.gemv(eye, x), x[[0, 7, 300, 513]])
    xs = np.stack([x, -x, 2 * x])
    ys = oracle.gemv(w, xs)
    assert np.array_equal(ys[0], y) and np.array_equal(ys[1], -y) and np.array_equal(ys[2], 2 * y)
    assert np.array_equal(oracle.gemv(w, xs, nthreads=4), ys)


@pytest.mark.parametrize("T,M,N", [(16, 5, 1), (37, 67, 129), (130, 9, 514), (64, 64, 3072)])
def test_gemv_token_vector_path_equals_scalar_sums(T, M, N):
    """16+ tokens run 16 tokens per vector lane-set; each lane must repeat the
    scalar in-order float sum exactly: compare with one-token calls (the
    scalar loop) bit for bit, across ragged token and row tails, and with a
    float64 bound."""
    rng = np.random.default_rng(T * 1000 + M)
    w = oracle.round_bf16(rng.standard_normal((M, N)).astype(np.float32))
    x = oracle.round_bf16(rng.standard_normal((T, N)).astype(np.float32))
    y = oracle.gemv(w, x, nthreads=3)
    ys = np.stack([oracle.gemv(w, x[t]) for t in range(T)])
    assert np.array_equal(y.view(np.uint32), ys.view(np.uint32))
    ref = x.astype(np.float64) @ w.astype(np.float64).T
    bound = N * 2.0 ** -23 * (np.abs(x).astype(np.float64) @ np.abs(w).astype(np.float64).T)
    assert (np.abs(y - ref) <= bound + 1e-30).all()


# ------------------------------------------------- rest of a decoder layer

def test_layer_op_case_generators_literal_values():
    """Case formulas of tests/rmsnorm_test_common.h:33-41,
    tests/swiglu_test_common.h:33-42, tests/add_test_common.h:36-50 and
    tests/test_batch_rmsnorm_bf16.cu:31-44 evaluated in float64."""
    import math
    x, w = oracle.make_rmsnorm_row_case(258, 264, 0.11, 0.07)
    for i in (0, 100, 257):
        e = 0.48 * math.sin((i + 1) * 0.11) - 0.22 * math.cos((i + 3) * 0.11 * 0.7) + 0.013 * (i % 7)
        assert abs(x[i] - e) < 1e-6
        e = 0.72 + 0.18 * math.sin((i + 5) * 0.07) - 0.04 * ((i * 3) % 5)
        assert abs(w[i] - e) < 1e-6
    assert abs(x[260] - (-0.75 + 0.05 * 2)) < 1e-6 and abs(w[263] - (0.95 - 0.03 * 5)) < 1e-6
    g, u = oracle.make_swiglu_case(514, 520, 0.08, 0.05)
    for i in (0, 513):
        assert abs(g[i] - (0.9 * math.sin((i + 1) * 0.08) - 0.7 * math.cos((i + 3) * 0.04))) < 1e-6
        assert abs(u[i] - (0.42 * math.cos((i + 5) * 0.05) - 0.31 * math.sin((i + 1) * 0.04)
                           - 0.02 * (i % 6))) < 1e-6
    assert abs(g[515] - (-1.2 + 0.07)) < 1e-6
    r, h = oracle.make_add_case(514, 520, 0.09, 0.07, 0.6)
    for i in (0, 513):
        assert abs(r[i] - (0.23 * math.sin((i + 1) * 0.09) - 0.08 * math.cos((i + 5) * 0.063)
                           + 0.01 * (i % 5))) < 1e-6
        assert abs(h[i] - (-0.27 * math.cos((i + 3) * 0.07) + 0.19 * math.sin((i + 1) * 0.042)
                           - 0.012 * ((i * 7) % 9))) < 1e-6
    assert abs(r[514] - 0.6) < 1e-6 and abs(h[519] - (-0.6 - 0.1)) < 1e-6
    xb, wb = oracle.make_batch_row_rmsnorm_case(3, 32, 0.08, 0.12)
    for b, i in ((0, 0), (2, 31)):
        idx = b * 32 + i
        e = (0.43 * math.sin((idx + 1) * 0.08) - 0.27 * math.cos((i + 2) * 0.08 * 0.4)
             + 0.02 * ((b + i) % 7))
        assert abs(xb[b, i] - e) < 1e-6


def test_residual_add_and_swiglu_vs_torch_bf16():
    """Residual add against torch's bf16 addition (float sum, one rounding),
    SwiGLU against torch's silu in float64 then bf16 (within one bf16 step),
    plus closed forms: silu(0) = 0, silu(g) -> g for large g, -> 0 for very
    negative g."""
    import torch
    rng = np.random.default_rng(7)
    h = oracle.round_bf16(rng.normal(size=4096).astype(np.float32))
    r = oracle.round_bf16(rng.normal(size=4096).astype(np.float32))
    exp = (torch.from_numpy(h).to(torch.bfloat16) + torch.from_numpy(r).to(torch.bfloat16))
    assert np.array_equal(oracle.residual_add(h, r), exp.float().numpy())
    g = oracle.round_bf16(rng.normal(scale=3.0, size=4096).astype(np.float32))
    u = oracle.round_bf16(rng.normal(size=4096).astype(np.float32))
    ref = torch.from_numpy(u).double() * torch.nn.functional.silu(torch.from_numpy(g).double())
    ref_b = ref.float().to(torch.bfloat16).float().numpy()
    got = oracle.swiglu(g, u)
    step = np.maximum(np.abs(ref_b), 1e-30) * 2.0 ** -7
    assert (np.abs(got - ref_b) <= step + 1e-12).all()
    z = np.zeros(4, np.float32)
    assert np.array_equal(oracle.swiglu(z, np.ones(4, np.float32)), z)
    big = np.array([20.0, 40.0], np.float32)
    assert np.array_equal(oracle.swiglu(big, np.array([1.0, 0.5], np.float32)),
                          oracle.round_bf16(np.array([20.0, 20.0], np.float32)))
    assert np.abs(oracle.swiglu(-big, np.ones(2, np.float32))).max() < 1e-6


def test_argmax_first_maximum_and_nan():
    """First index of the maximum (numpy.argmax on NaN-free input); NaN never
    wins; nothing above -FLT_MAX gives UINT32_MAX."""
    rng = np.random.default_rng(8)
    for n in (1, 7, 1000, 151936):
        x = rng.normal(size=n).astype(np.float32)
        assert oracle.argmax(x) == int(np.argmax(x))
    x = np.array([1.0, 5.0, 5.0, 2.0], np.float32)
    assert oracle.argmax(x) == 1
    x = np.array([np.nan, -1.0, np.nan, 3.0, np.nan], np.float32)
    assert oracle.argmax(x) == 3
    assert oracle.argmax(np.array([-np.inf, np.nan], np.float32)) == 0xFFFFFFFF



# ------------------------------------------------------------ sampling
# oracle.sample_topk_topp restates src/sampler.cpp:18-67 with the draw u given.

def test_sample_known_answers():
    """Hand-computed: logits [2, 1, 0, -1], T = 1, top_k = 3 gives
    p = e^(2,1,0) / (e^2 + e + 1) = (0.6652, 0.2447, 0.0900); cumulative
    0.6652, 0.9100, 1."""
    lg = np.array([2, 1, 0, -1], np.float32)
    e = np.exp(np.array([2.0, 1.0, 0.0]))
    tok, order, probs, kept = oracle.sample_topk_topp(lg, 1.0, 3, 0.8, 0.5)
    assert list(order) == [0, 1, 2] and kept == 2 and tok == 0
    np.testing.assert_allclose(probs, e / e.sum(), rtol=1e-6)
    assert oracle.sample_topk_topp(lg, 1.0, 3, 0.8, 0.9)[0] == 1    # coin 0.819 > 0.665
    for u in (0.0, 0.5, 0.99):                                          # top_p 0.5 keeps one
        assert oracle.sample_topk_topp(lg, 1.0, 3, 0.5, u)[:4:3] == (0, 1)
    assert oracle.sample_topk_topp(lg, 1.0, 3, 1.0, 0.95)[0] == 2       # coin 0.95 > 0.910
    assert oracle.sample_topk_topp(lg, 1.0, 3, 0.0, 0.99)[0] == 0       # top_p 0: first only


def test_sample_greedy_paths():
    """|T| < 1e-3 or top_k == 1: the reference's argmax (first maximum,
    strict '>' from -FLT_MAX; none for all -inf)."""
    lg = np.array([1, 3, 3, 2], np.float32)
    for T, k in ((0.0, 20), (5e-4, 20), (1.0, 1), (0.7, 1)):
        assert oracle.sample_topk_topp(lg, T, k, 0.95, 0.7)[0] == 1
    assert oracle.sample_topk_topp(np.full(5, -np.inf, np.float32), 0.0, 5, 0.9, 0.5)[0] == 0xFFFFFFFF


@pytest.mark.parametrize("T", [0.5, 0.7, 1.3])
def test_sample_probabilities_closed_form(T):
    """The reference divides by T twice (x = logit / T, then exp((x - max) / T)):
    the kept probabilities are softmax(logit / T^2) over the top k in float64.
    One division instead of two would fail this for T != 1."""
    rng = np.random.default_rng(int(T * 10))
    lg = (rng.standard_normal(500) * 2).astype(np.float32)
    k = 40
    tok, order, probs, kept = oracle.sample_topk_topp(lg, T, k, 0.95, 0.3)
    x = lg.astype(np.float32) / np.float32(T)
    exp_order = np.lexsort((np.arange(lg.size), -x))[:k]           # larger first, ties by index
    assert np.array_equal(order, exp_order)
    z = lg[order].astype(np.float64) / (T * T)
    ref = np.exp(z - z.max())
    ref /= ref.sum()
    np.testing.assert_allclose(probs, ref, rtol=2e-5, atol=1e-9)
    cum = np.cumsum(ref)
    assert np.min(np.abs(cum - 0.95)) > 1e-5                        # the cut is not a near tie
    assert kept == int(np.argmax(cum > 0.95)) + 1


def test_sample_coin_walk_brute_force():
    """A draw at the middle of kept interval j picks order[j]; u = 0 picks the
    first; a draw just below 1 picks the last kept."""
    rng = np.random.default_rng(9)
    lg = (rng.standard_normal(300) * 1.5).astype(np.float32)
    tok, order, probs, kept = oracle.sample_topk_topp(lg, 1.0, 30, 0.9, 0.0)
    assert tok == order[0]
    cum = np.cumsum(probs.astype(np.float64))[:kept]
    lo = np.concatenate([[0.0], cum[:-1]])
    for j in range(kept):
        u = (lo[j] + cum[j]) / 2 / cum[-1]
        assert oracle.sample_topk_topp(lg, 1.0, 30, 0.9, u)[0] == order[j], j
    assert oracle.sample_topk_topp(lg, 1.0, 30, 0.9, 1 - 2 ** -24)[0] == order[kept - 1]


def test_sample_ties_keep_lowest_indices():
    lg = np.array([5, 3, 3, 3, 1], np.float32)
    tok, order, probs, kept = oracle.sample_topk_topp(lg, 1.0, 2, 1.0, 0.99)
    assert list(order) == [0, 1] and tok == 1
    lg = np.array([0, 2, 2, 1, 2], np.float32)
    assert list(oracle.sample_topk_topp(lg, 1.0, 3, 1.0, 0.5)[1]) == [1, 2, 4]


def test_sample_coin_is_splitmix64():
    """The first two SplitMix64 outputs of seed 0 are the published
    0xE220A8397B1DCDAF and 0x6E789E6AA1B965F4 (Vigna's splitmix64.c); the
    draw is their top 24 bits over 2^24.  Draws over many positions are
    uniform to within sampling error."""
    assert oracle.sample_coin(0, 0) == 0xE220A8 / 2 ** 24
    assert oracle.sample_coin(0, 1) == 0x6E789E / 2 ** 24
    u = np.array([oracle.sample_coin(12345, p) for p in range(20000)])
    assert u.min() >= 0 and u.max() < 1
    assert abs(u.mean() - 0.5) < 0.01
    hist = np.histogram(u, bins=10, range=(0, 1))[0]
    assert hist.min() > 1800 and hist.max() < 2200


# ------------------------------------------------------------ Qwen3 forward

def _qwen3_fixture():
    import json

    from tests import qwen3_weights as QW

    g = np.load(os.path.join(GOLD, "qwen3_tiny.npz"))
    cfg = json.loads(str(g["config"]))
    init = json.loads(str(g["init"]))
    bits = QW.weight_bits(cfg, int(g["seed"]), init["proj_std"], init["embed_std"],
                          tuple(init["norm_range"]), init["tied"])
    w = QW.to_f32(bits)
    w["inv_freq"] = oracle.inv_freq(cfg["head_dim"], cfg["rope_theta"])
    return cfg, w, g


def _qwen3_oracle_logits(cfg, w, g):
    ids, T = g["ids"], int(g["prompt"])
    ref = oracle.Qwen3Reference(cfg, w)
    rows = [ref.forward(ids[:T], 0)]
    for s in range(len(ids) - T):
        rows.append(ref.forward(ids[T + s:T + s + 1], T + s))
    return np.stack(rows)


# The oracle against the float64 forward with the same bf16 rounding points
# (tests/golden/make_qwen3_golden.py, itself checked against transformers'
# Qwen3).  The remaining differences are fp32-vs-fp64 sums flipping a bf16
# activation by one step now and then; on logits of std ~17 they measure
# max 0.20, mean 0.043 (the rounding points themselves move the logits by
# mean 0.067).  Each planted slip below moves them by mean 1 or more.
QWEN3_PIN_MAX = 0.5
QWEN3_PIN_MEAN = 0.1


def test_qwen3_reference_vs_float64_fixture():
    cfg, w, g = _qwen3_fixture()
    got = _qwen3_oracle_logits(cfg, w, g)
    d = np.abs(got.astype(np.float64) - g["logits_rounded"])
    assert d.max() <= QWEN3_PIN_MAX and d.mean() <= QWEN3_PIN_MEAN, (d.max(), d.mean())
    # Same greedy pick at every step, and the exact (unrounded) forward is
    # within the spread the rounding points themselves cause.
    assert np.array_equal(got.argmax(1), g["logits_rounded"].argmax(1))
    assert np.abs(got - g["logits_exact"]).max() < 1.0
    assert float(g["transformers_max_diff"]) < 1e-5 * np.abs(g["logits_exact"]).max()


def _interleaved_rope(qk, inv_freq, num_tokens, num_heads, d, pos0=0):
    """RoPE over adjacent pairs (2i, 2i+1): the GPT-J pairing, not Qwen3's."""
    x = np.asarray(qk, np.float32).reshape(num_tokens, num_heads, d // 2, 2).copy()
    t = (np.arange(num_tokens, dtype=np.float32) + np.float32(pos0))[:, None, None]
    a = t * np.asarray(inv_freq, np.float32)[None, None, :]
    c, s = np.cos(a), np.sin(a)
    x0, x1 = x[..., 0].copy(), x[..., 1].copy()
    x[..., 0], x[..., 1] = x0 * c - x1 * s, x1 * c + x0 * s
    return oracle.round_bf16(x.reshape(np.shape(qk)))


@pytest.mark.parametrize("mistake", ["rope_pairing", "norm_after_rope", "kv_head_map",
                                     "no_q_norm"])
def test_qwen3_fixture_catches_planted_mistakes(monkeypatch, mistake):
    """Plausible misreadings planted in the oracle (on the CPU) fail the pin."""
    cfg, w, g = _qwen3_fixture()
    if mistake == "rope_pairing":
        monkeypatch.setattr(oracle, "rope", _interleaved_rope)
    elif mistake == "norm_after_rope":
        # RoPE first, then the per-head norm: swap the two calls' effects.
        real_norm, real_rope = oracle.multi_rmsnorm, oracle.rope
        pending = {}

        def norm_later(x, wt, d, eps):
            pending["args"] = (wt, d, eps)
            return np.asarray(x, np.float32)

        def rope_then_norm(qk, inv, T, H, d, pos0=0):
            wt, dd, eps = pending.pop("args")
            return real_norm(real_rope(qk, inv, T, H, d, pos0), wt, dd, eps)

        monkeypatch.setattr(oracle, "multi_rmsnorm", norm_later)
        monkeypatch.setattr(oracle, "rope", rope_then_norm)
    elif mistake == "kv_head_map":
        # Query head h reading KV head h % Hkv instead of h // (Hq/Hkv).
        real_flash, real_dec = oracle.flash_reference, oracle.decode_attention
        hq, hkv = cfg["num_q_heads"], cfg["num_kv_heads"]
        perm = np.array([(h % hkv) * (hq // hkv) + h // hkv for h in range(hq)])

        def flash_mod(q, k, v, rows=None, nthreads=0):
            inv = np.argsort(perm)
            return real_flash(q[:, perm], k, v, rows, nthreads)[:, inv]

        def dec_mod(q, k, v, pos, msl):
            inv = np.argsort(perm)
            s, ob, o = real_dec(q[perm], k, v, pos, msl)
            return s[inv], ob[inv], o[inv]

        monkeypatch.setattr(oracle, "flash_reference", flash_mod)
        monkeypatch.setattr(oracle, "decode_attention", dec_mod)
    elif mistake == "no_q_norm":
        real_norm = oracle.multi_rmsnorm
        calls = {"n": 0}

        def skip_every_other(x, wt, d, eps):  # q is normalised first in each layer
            calls["n"] += 1
            return oracle.round_bf16(x) if calls["n"] % 2 == 1 else real_norm(x, wt, d, eps)

        monkeypatch.setattr(oracle, "multi_rmsnorm", skip_every_other)
    got = _qwen3_oracle_logits(cfg, w, g)
    d = np.abs(got.astype(np.float64) - g["logits_rounded"])
    print(f"{mistake}: max {d.max():.3g} mean {d.mean():.3g}")
    assert d.max() > QWEN3_PIN_MAX and d.mean() > 5 * QWEN3_PIN_MEAN, \
        f"{mistake}: max {d.max():.3g} mean {d.mean():.3g} passed the pin"
