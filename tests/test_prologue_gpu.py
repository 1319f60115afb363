"""Qwen3 pre-attention ops and the fused long prefill (config 4) vs the oracle.

Cases follow tests/test_precompute_freq_f32.cu:31-36 (1e-6),
tests/test_batch_multi_rmsnorm_bf16.cu:113-119 and
tests/test_multi_rmsnorm_bf16.cu, tests/test_rope_bf16.cu:34-54 (2e-2).
"""
import numpy as np
import pytest
import torch

import oracle
from tests import helpers as H
from toyinfer_amd import attn, synth

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("d,buf,theta", [(2, 4, 2.0), (258, 140, 1.0), (130, 80, 10000.0),
                                         (514, 300, 123.5), (128, 64, 1e6)])
def test_precompute_freq(dev, d, buf, theta):
    init = (4.0 - 0.21 * np.arange(buf)).astype(np.float32)
    out = H.to_dev_f32(init, dev)
    attn.precompute_freq_f32(out, d, theta)
    H.sync()
    exp = init.copy()
    exp[: d // 2] = oracle.inv_freq(d, theta)
    H.check_close(out.cpu().numpy(), exp, 1e-6, 1e-6, f"inv_freq D={d}")


@pytest.mark.parametrize("batch,heads,d,eps,ip,wp", [
    (2, 1, 64, 1e-5, 0.13, 0.09),   # tests/test_batch_multi_rmsnorm_bf16.cu:114-117
    (2, 4, 64, 1e-4, 0.09, 0.05),
    (5, 8, 128, 1e-6, 0.07, 0.03),
])
def test_batch_multi_rmsnorm(dev, batch, heads, d, eps, ip, wp):
    x, w = oracle.make_batch_rmsnorm_case(batch, heads, d, ip, wp)
    xb, wb = oracle.f32_to_bf16(x), oracle.f32_to_bf16(w)
    exp = oracle.multi_rmsnorm(oracle.bf16_to_f32(xb), oracle.bf16_to_f32(wb), d, eps)
    xd = H.to_dev_bf16(xb, dev)
    out = torch.empty_like(xd)
    attn.batch_multi_rmsnorm_bf16(xd, H.to_dev_bf16(wb, dev), out, eps, batch, heads, d)
    H.sync()
    got = H.bf16_bits_to_f32(H.from_dev_bf16(out))
    H.check_close(got, exp, 2e-2, 2e-2, "batch rmsnorm")
    # In place, as src/transformer.cpp:380-387 calls it.
    attn.batch_multi_rmsnorm_bf16(xd, H.to_dev_bf16(wb, dev), xd, eps, batch, heads, d)
    H.sync()
    assert np.array_equal(H.from_dev_bf16(xd), H.from_dev_bf16(out))


def test_multi_rmsnorm_single_token_leaves_tail(dev):
    """tests/multi_rmsnorm_test_common.h: rows past nums_head stay untouched."""
    x, w = oracle.make_rmsnorm_case(3, 128, 3 * 128 + 6, 0.05, 0.11)
    xb, wb = oracle.f32_to_bf16(x), oracle.f32_to_bf16(w)
    xq = oracle.bf16_to_f32(xb)
    exp = xq.copy()
    exp[: 3 * 128] = oracle.multi_rmsnorm(xq[: 3 * 128], oracle.bf16_to_f32(wb), 128, 1e-6)
    xd = H.to_dev_bf16(xb, dev)
    attn.multi_rmsnorm_bf16(xd, H.to_dev_bf16(wb, dev), xd, 1e-6, 3, 128)
    H.sync()
    H.check_close(H.bf16_bits_to_f32(H.from_dev_bf16(xd)), exp, 2e-2, 2e-2, "rmsnorm tail")
    assert np.array_equal(H.from_dev_bf16(xd)[3 * 128:], xb[3 * 128:])


@pytest.mark.parametrize("tokens,heads,d,phase,fscale", [
    (12, 3, 64, 0.03, 0.001),
    (38, 4, 128, 0.021, None),     # inv_freq = theta 10000 table
    (300, 8, 128, 0.017, "qwen"),  # theta 1e6, positions 0..299
])
def test_batch_rope(dev, tokens, heads, d, phase, fscale):
    qk, f = oracle.make_rope_case(tokens * heads, d, tokens * heads * d, phase,
                                  fscale if isinstance(fscale, float) else 0.0)
    if fscale is None:
        f = oracle.inv_freq(d, 10000.0)
    elif fscale == "qwen":
        f = oracle.inv_freq(d, 1e6)
    qkb = oracle.f32_to_bf16(qk)
    exp = oracle.rope(oracle.bf16_to_f32(qkb), f, tokens, heads, d)
    qd = H.to_dev_bf16(qkb, dev)
    attn.batch_rope_bf16(qd, H.to_dev_f32(f, dev), tokens, heads, d)
    H.sync()
    H.check_close(H.bf16_bits_to_f32(H.from_dev_bf16(qd)), exp, 2e-2, 2e-2, "rope")


@pytest.mark.parametrize("d,theta,npos", [(128, 1e6, 8192), (64, 1e4, 300)])
def test_rope_cos_sin_table(dev, d, theta, npos):
    f = oracle.inv_freq(d, theta)
    table = torch.empty((npos, d // 2, 2), dtype=torch.float32, device=dev)
    attn.rope_cos_sin_f32(table, H.to_dev_f32(f, dev), npos, d)
    H.sync()
    got = table.cpu().numpy()
    ang = np.arange(npos, dtype=np.float32)[:, None] * f[None, :]   # float32 products
    exp = np.stack([np.cos(ang.astype(np.float64)), np.sin(ang.astype(np.float64))], -1)
    # fp32 sincos of the fp32 angle: a few ulp of 1 at worst
    assert np.abs(got - exp).max() < 4e-7


def test_rope_position0_is_identity(dev):
    x = synth.normal_bf16(3, "x", (1, 4, 128))
    xd = H.to_dev_bf16(x, dev)
    attn.batch_rope_bf16(xd, H.to_dev_f32(oracle.inv_freq(128, 1e6), dev), 1, 4, 128)
    H.sync()
    assert np.array_equal(H.from_dev_bf16(xd), x)


def test_qk_norm_rope_fused_matches_two_pass(dev):
    t, h, d = 257, 8, 128
    x = synth.normal_bf16(4, "k", (t, h, d))
    g = synth.uniform_bf16(4, "gk", (d,), 0.9, 1.1)
    f = H.to_dev_f32(oracle.inv_freq(d, 1e6), dev)
    xd, gd = H.to_dev_bf16(x, dev), H.to_dev_bf16(g, dev)
    fused = torch.empty_like(xd)
    attn.qk_norm_rope_bf16(xd, gd, fused, f, 1e-6, t, h, d)
    two = torch.empty_like(xd)
    attn.batch_multi_rmsnorm_bf16(xd, gd, two, 1e-6, t, h, d)
    attn.batch_rope_bf16(two, f, t, h, d)
    H.sync()
    assert np.array_equal(H.from_dev_bf16(fused), H.from_dev_bf16(two))
    exp = oracle.qk_norm_rope(oracle.bf16_to_f32(x), oracle.bf16_to_f32(g),
                              oracle.inv_freq(d, 1e6), 1e-6)
    H.check_bar(H.bf16_bits_to_f32(H.from_dev_bf16(fused)), exp, "qk_norm_rope")


def fused_prefill(qb, kb, vb, gq, gk, eps, theta, dev):
    s, hq, d = qb.shape
    hkv = kb.shape[1]
    q, k, v = H.to_dev_bf16(qb, dev), H.to_dev_bf16(kb, dev), H.to_dev_bf16(vb, dev)
    o = torch.empty((s, hq, d), dtype=torch.bfloat16, device=dev)
    k_out = torch.empty_like(k)
    f = torch.empty(d // 2, dtype=torch.float32, device=dev)
    attn.precompute_freq_f32(f, d, theta)
    table = torch.empty((s, d // 2, 2), dtype=torch.float32, device=dev)
    attn.rope_cos_sin_f32(table, f, s, d)
    attn.prefill_qknorm_rope_attention_bf16(q, k, v, o, k_out, H.to_dev_bf16(gq, dev),
                                            H.to_dev_bf16(gk, dev), table, eps, hq, hkv, d, s)
    H.sync()
    return H.from_dev_bf16(o), H.from_dev_bf16(k_out), (q, k, v, f)


def config4_inputs(s, hq, hkv, d, seed=4):
    return (synth.normal_bf16(seed, "q", (s, hq, d)), synth.normal_bf16(seed, "k", (s, hkv, d)),
            synth.normal_bf16(seed, "v", (s, hkv, d)),
            synth.uniform_bf16(seed, "gamma_q", (d,), 0.9, 1.1),
            synth.uniform_bf16(seed, "gamma_k", (d,), 0.9, 1.1))


def oracle_fused(qb, kb, vb, gq, gk, eps, theta, rows=None):
    d = qb.shape[2]
    f = oracle.inv_freq(d, theta)
    qn = oracle.qk_norm_rope(oracle.bf16_to_f32(qb), oracle.bf16_to_f32(gq), f, eps)
    kn = oracle.qk_norm_rope(oracle.bf16_to_f32(kb), oracle.bf16_to_f32(gk), f, eps)
    return oracle.flash_reference(qn, kn, oracle.bf16_to_f32(vb), rows=rows), kn


@pytest.mark.parametrize("s,hq,hkv,d", [(1024, 32, 8, 128), (333, 8, 2, 64), (1, 4, 2, 128)])
def test_fused_prefill_full(dev, s, hq, hkv, d):
    print(f"[fused] S={s} {hq}/{hkv} D={d}", flush=True)
    qb, kb, vb, gq, gk = config4_inputs(s, hq, hkv, d)
    got, k_out, _ = fused_prefill(qb, kb, vb, gq, gk, 1e-6, 1e6, dev)
    exp, kn = oracle_fused(qb, kb, vb, gq, gk, 1e-6, 1e6)
    H.check_bar(H.bf16_bits_to_f32(k_out), kn, "K_out")
    H.check_bar(H.bf16_bits_to_f32(got), oracle.round_bf16(exp), "fused O")


def test_fused_equals_unfused_composition(dev):
    """Fused entry point == norm/rope kernels in place + plain prefill."""
    s, hq, hkv, d = 700, 16, 8, 128
    qb, kb, vb, gq, gk = config4_inputs(s, hq, hkv, d, seed=5)
    fused, k_out, (q, k, v, f) = fused_prefill(qb, kb, vb, gq, gk, 1e-6, 1e6, dev)
    attn.qk_norm_rope_bf16(q, H.to_dev_bf16(gq, dev), q, f, 1e-6, s, hq, d)
    attn.qk_norm_rope_bf16(k, H.to_dev_bf16(gk, dev), k, f, 1e-6, s, hkv, d)
    o = torch.empty((s, hq, d), dtype=torch.bfloat16, device=dev)
    attn.flash_attention_v1_bf16(q, k, v, o, hq, hkv, d, s)
    H.sync()
    assert np.array_equal(H.from_dev_bf16(k), k_out)
    a, b = H.bf16_bits_to_f32(fused), H.bf16_bits_to_f32(H.from_dev_bf16(o))
    H.check_bar(a, b, "fused vs unfused", max_abs=1e-2, mean_abs=2e-4)


def test_fused_prefill_head_pairs_ragged_rows(dev):
    """The fused entry at a length where the head-pair 128-row kernel is
    chosen (S = 4100, 32/8: 33 query tiles x 16 pairs, two rounds of the
    device) with a partial last query tile: first and last rows and every
    37th against the oracle."""
    s, hq, hkv, d = 4100, 32, 8, 128
    print("[fused] S=4100 32/8 head pairs, row subset", flush=True)
    qb, kb, vb, gq, gk = config4_inputs(s, hq, hkv, d, seed=7)
    got, k_out, _ = fused_prefill(qb, kb, vb, gq, gk, 1e-6, 1e6, dev)
    rows = sorted(set(range(40)) | set(range(s - 40, s)) | set(range(0, s, 37)))
    exp, kn = oracle_fused(qb, kb, vb, gq, gk, 1e-6, 1e6, rows=rows)
    H.check_bar(H.bf16_bits_to_f32(k_out), kn, "K_out")
    H.check_bar(H.bf16_bits_to_f32(got[rows]), oracle.round_bf16(exp[rows]), "fused O rows")


def test_config4_row_subset(dev):
    """Config 4 (S=8192, 32/8, D=128): rows 0-63, 8128-8191 and every 61st
    against the oracle (the full fp64 reference is minutes of CPU)."""
    s, hq, hkv, d = 8192, 32, 8, 128
    print("[fused] config4 S=8192 row subset", flush=True)
    qb, kb, vb, gq, gk = config4_inputs(s, hq, hkv, d)
    got, _, _ = fused_prefill(qb, kb, vb, gq, gk, 1e-6, 1e6, dev)
    rows = sorted(set(range(64)) | set(range(s - 64, s)) | set(range(0, s, 61)))
    exp, _ = oracle_fused(qb, kb, vb, gq, gk, 1e-6, 1e6, rows=rows)
    mx, mn = H.check_bar(H.bf16_bits_to_f32(got[rows]), oracle.round_bf16(exp[rows]), "config4")
    print(f"[fused] config4 rows={len(rows)} max-abs {mx:.3g} mean-abs {mn:.3g}", flush=True)
