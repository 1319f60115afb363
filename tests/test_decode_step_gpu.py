"""Decode-step pre-pass ops vs the oracle: rope_bf16 / rope_bf16_graph at one
position, write_kv_cache_bf16, and the fused norm + RoPE + cache-write pass
that replaces src/transformer.cpp:535-552.

RoPE and RMSNorm use the reference tests' bar (tests/test_rope_bf16.cu:34-54,
tests/test_multi_rmsnorm_bf16.cu: 2e-2 absolute and relative); cache writes
and V copies are bit-exact.
"""
import numpy as np
import pytest
import torch

import oracle
from tests import helpers as H
from toyinfer_amd import attn, synth

pytestmark = pytest.mark.gpu

SENTINEL = 0x7F11  # a bf16 bit pattern no computed value here takes


def inv_freq_dev(d, dev, theta=1e6):
    inv = oracle.inv_freq(d, theta)
    return inv, H.to_dev_f32(inv, dev)


def expected_rope(xb, inv, pos, heads, d):
    return oracle.rope(oracle.bf16_to_f32(xb), inv, 1, heads, d, pos0=pos)


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("pos", [0, 1, 777, 40959])
def test_rope_single_position(dev, d, pos):
    heads = 8
    print(f"[step] rope D={d} pos={pos}", flush=True)
    xb = synth.normal_bf16(21, "x", (heads, d))
    inv, invd = inv_freq_dev(d, dev)
    exp = expected_rope(xb, inv, pos, heads, d)
    a = H.to_dev_bf16(xb, dev)
    attn.rope_bf16(a, invd, pos, heads, d)
    b = H.to_dev_bf16(xb, dev)
    pos_d = torch.tensor([pos], dtype=torch.int32, device=dev)
    attn.rope_bf16_graph(b, invd, pos_d, heads, d)
    H.sync()
    ga, gb = H.from_dev_bf16(a), H.from_dev_bf16(b)
    H.check_close(H.bf16_bits_to_f32(ga), exp, 2e-2, 2e-2, f"rope_bf16 pos={pos}")
    assert np.array_equal(ga, gb), "host-pos and device-pos RoPE differ"
    if pos == 0:  # closed form: angle 0 leaves every value as it was
        assert np.array_equal(ga, xb)


@pytest.mark.parametrize("kv_dim,offset", [(1024, 0), (6, 0), (1024, 2)])
@pytest.mark.parametrize("pos", [0, 9])
def test_write_kv_cache(dev, kv_dim, offset, pos):
    """Row pos of the cache gets src bit for bit; every other element keeps
    its value (16-byte path, pair path for kv_dim % 8 != 0 or a cache base
    that is only 4-byte aligned)."""
    rows = 10
    src = synth.normal_bf16(22, "s", (kv_dim,))
    buf = torch.full((rows * kv_dim + offset,), SENTINEL, dtype=torch.int16, device=dev)
    cache = buf[offset:]
    pos_d = torch.tensor([pos], dtype=torch.int32, device=dev)
    attn.write_kv_cache_bf16(H.to_dev_bf16(src, dev), cache, pos_d, kv_dim)
    H.sync()
    got = buf.cpu().numpy().view(np.uint16)
    exp = np.full(rows * kv_dim + offset, SENTINEL, np.uint16)
    exp[offset + pos * kv_dim: offset + (pos + 1) * kv_dim] = src
    assert np.array_equal(got, exp)


def prologue_case(seed, hq, hkv, d):
    q = synth.normal_bf16(seed, "q", (hq, d))
    k = synth.normal_bf16(seed, "k", (hkv, d))
    v = synth.normal_bf16(seed, "v", (hkv, d))
    gq = synth.uniform_bf16(seed, "gq", (d,), 0.9, 1.1)
    gk = synth.uniform_bf16(seed, "gk", (d,), 0.9, 1.1)
    return q, k, v, gq, gk


def expected_prologue(q, k, gq, gk, inv, pos, hq, hkv, d, eps):
    qn = oracle.multi_rmsnorm(oracle.bf16_to_f32(q), oracle.bf16_to_f32(gq), d, eps)
    kn = oracle.multi_rmsnorm(oracle.bf16_to_f32(k), oracle.bf16_to_f32(gk), d, eps)
    return (oracle.rope(qn, inv, 1, hq, d, pos0=pos), oracle.rope(kn, inv, 1, hkv, d, pos0=pos))


def run_prologue(dev, q, k, v, gq, gk, invd, pos, msl, hq, hkv, d, eps, in_place):
    qd = H.to_dev_bf16(q, dev)
    qo = qd if in_place else torch.full((hq, d), 0.25, dtype=torch.bfloat16, device=dev)
    kc = torch.full((msl, hkv, d), SENTINEL, dtype=torch.int16, device=dev)
    vc = torch.full((msl, hkv, d), SENTINEL, dtype=torch.int16, device=dev)
    pos_d = torch.tensor([pos], dtype=torch.int32, device=dev)
    attn.decode_qkv_prologue_bf16(qd, H.to_dev_bf16(k, dev), H.to_dev_bf16(v, dev),
                                  H.to_dev_bf16(gq, dev), H.to_dev_bf16(gk, dev), invd, pos_d,
                                  msl, eps, qo, kc, vc, hq, hkv, d)
    H.sync()
    return (H.from_dev_bf16(qo), kc.cpu().numpy().view(np.uint16),
            vc.cpu().numpy().view(np.uint16))


@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (16, 8, 128), (8, 2, 64), (6, 3, 64)])
@pytest.mark.parametrize("pos,in_place", [(0, False), (13, True), (63, False)])
def test_decode_qkv_prologue(dev, hq, hkv, d, pos, in_place):
    msl, eps = 64, 1e-6
    print(f"[step] prologue {hq}/{hkv} D={d} pos={pos} in_place={in_place}", flush=True)
    q, k, v, gq, gk = prologue_case(23, hq, hkv, d)
    inv, invd = inv_freq_dev(d, dev)
    qo, kc, vc = run_prologue(dev, q, k, v, gq, gk, invd, pos, msl, hq, hkv, d, eps, in_place)
    qe, ke = expected_prologue(q, k, gq, gk, inv, pos, hq, hkv, d, eps)
    H.check_close(H.bf16_bits_to_f32(qo), qe, 2e-2, 2e-2, "q_out")
    H.check_close(H.bf16_bits_to_f32(kc[pos]), ke, 2e-2, 2e-2, "k cache row")
    assert np.array_equal(vc[pos], v), "v cache row"
    others = np.arange(msl) != pos
    assert (kc[others] == SENTINEL).all() and (vc[others] == SENTINEL).all(), \
        "rows other than pos changed"


def test_decode_qkv_prologue_clamps_position(dev):
    """A device position past the cache writes (and rotates for) row msl-1,
    the row the graph attention also clamps to."""
    hq, hkv, d, msl, eps = 8, 2, 128, 16, 1e-6
    q, k, v, gq, gk = prologue_case(24, hq, hkv, d)
    inv, invd = inv_freq_dev(d, dev)
    qo, kc, vc = run_prologue(dev, q, k, v, gq, gk, invd, 1000, msl, hq, hkv, d, eps, False)
    qe, ke = expected_prologue(q, k, gq, gk, inv, msl - 1, hq, hkv, d, eps)
    H.check_close(H.bf16_bits_to_f32(qo), qe, 2e-2, 2e-2, "q_out")
    H.check_close(H.bf16_bits_to_f32(kc[msl - 1]), ke, 2e-2, 2e-2, "k cache row")
    assert np.array_equal(vc[msl - 1], v)
    assert (kc[: msl - 1] == SENTINEL).all()


def test_fused_prologue_equals_reference_sequence(dev):
    """The fused pass and the six-launch sequence of src/transformer.cpp:535-552
    (the drop-in ops, same rounding points) give identical bits."""
    hq, hkv, d, msl, pos, eps = 32, 8, 128, 48, 29, 1e-6
    q, k, v, gq, gk = prologue_case(25, hq, hkv, d)
    _, invd = inv_freq_dev(d, dev)
    qo, kc, vc = run_prologue(dev, q, k, v, gq, gk, invd, pos, msl, hq, hkv, d, eps, True)
    qd, kd = H.to_dev_bf16(q, dev), H.to_dev_bf16(k, dev)
    kc2 = torch.full((msl, hkv, d), SENTINEL, dtype=torch.int16, device=dev)
    vc2 = torch.full((msl, hkv, d), SENTINEL, dtype=torch.int16, device=dev)
    pos_d = torch.tensor([pos], dtype=torch.int32, device=dev)
    attn.multi_rmsnorm_bf16(qd, H.to_dev_bf16(gq, dev), qd, eps, hq, d)
    attn.multi_rmsnorm_bf16(kd, H.to_dev_bf16(gk, dev), kd, eps, hkv, d)
    attn.rope_bf16_graph(qd, invd, pos_d, hq, d)
    attn.rope_bf16_graph(kd, invd, pos_d, hkv, d)
    attn.write_kv_cache_bf16(kd, kc2, pos_d, hkv * d)
    attn.write_kv_cache_bf16(H.to_dev_bf16(v, dev), vc2, pos_d, hkv * d)
    H.sync()
    assert np.array_equal(qo, H.from_dev_bf16(qd))
    assert np.array_equal(kc, kc2.cpu().numpy().view(np.uint16))
    assert np.array_equal(vc, vc2.cpu().numpy().view(np.uint16))


def test_fused_prologue_graph_replay(dev):
    """Captured once; each replay reads the new device position."""
    hq, hkv, d, msl, eps = 16, 8, 128, 40, 1e-6
    q, k, v, gq, gk = prologue_case(26, hq, hkv, d)
    inv, invd = inv_freq_dev(d, dev)
    qd, kd, vd = H.to_dev_bf16(q, dev), H.to_dev_bf16(k, dev), H.to_dev_bf16(v, dev)
    gqd, gkd = H.to_dev_bf16(gq, dev), H.to_dev_bf16(gk, dev)
    qo = torch.empty((hq, d), dtype=torch.bfloat16, device=dev)
    kc = torch.full((msl, hkv, d), SENTINEL, dtype=torch.int16, device=dev)
    vc = torch.full((msl, hkv, d), SENTINEL, dtype=torch.int16, device=dev)
    pos_d = torch.zeros(1, dtype=torch.int32, device=dev)
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()

    def op():
        attn.decode_qkv_prologue_bf16(qd, kd, vd, gqd, gkd, invd, pos_d, msl, eps, qo, kc, vc,
                                      hq, hkv, d, stream)
    with torch.cuda.stream(stream):
        op()
    H.sync()
    with torch.cuda.graph(graph, stream=stream):
        op()
    for pos in (0, 17, 39, 5):
        pos_d.fill_(pos)
        H.sync()
        graph.replay()
        H.sync()
        qe, ke = expected_prologue(q, k, gq, gk, inv, pos, hq, hkv, d, eps)
        H.check_close(H.bf16_bits_to_f32(H.from_dev_bf16(qo)), qe, 2e-2, 2e-2, f"q pos={pos}")
        kcn = kc.cpu().numpy().view(np.uint16)
        H.check_close(H.bf16_bits_to_f32(kcn[pos]), ke, 2e-2, 2e-2, f"k pos={pos}")
        assert np.array_equal(vc.cpu().numpy().view(np.uint16)[pos], v)
