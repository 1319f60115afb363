"""toyinfer_decode_attention_bf16_noalloc (the batched decode with its split
partials in the library's own device array) against the entry point with a
caller workspace: the same kernels and split count, so outputs must be
bit-identical; two calls in a row, the second on a smaller input, and a
device-length call after them.  Sizes beyond the array are rejected on the
host.
"""
import numpy as np
import pytest
import torch

import oracle
from tests import helpers as H
from toyinfer_amd import attn, synth

pytestmark = pytest.mark.gpu


def inputs(seed, b, cap, hq, hkv, d):
    return (synth.normal_bf16(seed, "q", (b, hq, d)),
            synth.normal_bf16(seed, "k", (b, cap, hkv, d)),
            synth.normal_bf16(seed, "v", (b, cap, hkv, d)))


def both(dev, b, L, hq, hkv, d, seed, lens=None):
    """(no-alloc output, workspace-entry output, host inputs) as bf16 bits."""
    qb, kb, vb = inputs(seed, b, L, hq, hkv, d)
    q, k, v = H.to_dev_bf16(qb, dev), H.to_dev_bf16(kb, dev), H.to_dev_bf16(vb, dev)
    lens_d = None if lens is None else torch.tensor(np.asarray(lens, np.int32), device=dev)
    splits = attn.decode_default_splits(b, hq, hkv, d, L)
    assert attn.decode_workspace_bytes(b, hq, d, splits) <= attn.DECODE_SCRATCH_BYTES
    o_na = torch.full((b, hq, d), 7.0, dtype=torch.bfloat16, device=dev)
    attn.decode_attention_bf16_noalloc(q, k, v, o_na, b, hq, hkv, d, lens_d, L, L * hkv * d, 0)
    H.sync()
    ws = attn.decode_workspace(b, hq, d, splits, dev)
    o_ws = torch.full((b, hq, d), -7.0, dtype=torch.bfloat16, device=dev)
    attn.decode_attention_bf16(q, k, v, o_ws, b, hq, hkv, d, lens_d, L, L * hkv * d, splits, ws)
    H.sync()
    return H.from_dev_bf16(o_na), H.from_dev_bf16(o_ws), (qb, kb, vb)


def test_noalloc_matches_workspace_entry_two_calls(dev):
    print("[no-alloc] B=8 L=4096 32/8 D=128, then B=2 L=1000 16/8 D=128", flush=True)
    a_na, a_ws, (qb, kb, vb) = both(dev, 8, 4096, 32, 8, 128, seed=301)
    assert np.array_equal(a_na, a_ws), "first call differs from the workspace entry point"
    exp = oracle.round_bf16(oracle.decode_batched(qb, kb, vb, [4096] * 8))
    H.check_bar(H.bf16_bits_to_f32(a_na), exp, "first call vs oracle")
    # Second call, smaller: the array still holds the first call's partials.
    b_na, b_ws, (qb, kb, vb) = both(dev, 2, 1000, 16, 8, 128, seed=302)
    assert np.array_equal(b_na, b_ws), "second (smaller) call differs from the workspace entry"
    exp = oracle.round_bf16(oracle.decode_batched(qb, kb, vb, [1000] * 2))
    H.check_bar(H.bf16_bits_to_f32(b_na), exp, "second call vs oracle")


def test_noalloc_device_lengths_and_head_dim_64(dev):
    print("[no-alloc] ragged device lengths, D=64", flush=True)
    lens = [1, 300, 517]
    a_na, a_ws, (qb, kb, vb) = both(dev, 3, 600, 12, 4, 64, seed=303, lens=lens)
    assert np.array_equal(a_na, a_ws)
    exp = oracle.round_bf16(oracle.decode_batched(qb, kb, vb, lens))
    H.check_bar(H.bf16_bits_to_f32(a_na), exp, "ragged D=64")


def test_noalloc_rejects_sizes_beyond_the_array(dev):
    t = torch.zeros(64, dtype=torch.bfloat16, device=dev)
    b, hq, hkv, d, L = 4096, 32, 8, 128, 4096
    assert attn.decode_workspace_bytes(b, hq, d, 1) > attn.DECODE_SCRATCH_BYTES
    with pytest.raises(attn.ToyInferError) as e:
        attn.decode_attention_bf16_noalloc(t, t, t, t, b, hq, hkv, d, None, L, L * hkv * d, 1)
    assert e.value.status == attn.ERR_WORKSPACE


def test_noalloc_captured_in_a_graph_replays_bit_identically(dev):
    """The callers this entry point is for capture it: a torch CUDAGraph holds
    one call (device lengths, so each replay reads the lengths then current);
    three replays, with eager work and synchronisations between them, each
    match the workspace entry point bit for bit.  The array's address is
    taken on the entry point's first call on the device, which the capture
    does not contain (the calls of the tests above, or the direct call here)."""
    print("[no-alloc] graph capture and replays, B=4 L=2048 32/8 D=128", flush=True)
    b, L, hq, hkv, d = 4, 2048, 32, 8, 128
    qb, kb, vb = inputs(305, b, L, hq, hkv, d)
    q, k, v = H.to_dev_bf16(qb, dev), H.to_dev_bf16(kb, dev), H.to_dev_bf16(vb, dev)
    lens_d = torch.tensor([L, L, L, L], dtype=torch.int32, device=dev)
    o_na = torch.zeros((b, hq, d), dtype=torch.bfloat16, device=dev)
    side = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(side):
        attn.decode_attention_bf16_noalloc(q, k, v, o_na, b, hq, hkv, d, lens_d, L, L * hkv * d,
                                           0, side)
    H.sync()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        attn.decode_attention_bf16_noalloc(q, k, v, o_na, b, hq, hkv, d, lens_d, L, L * hkv * d,
                                           0, side)
    H.sync()
    splits = attn.decode_default_splits(b, hq, hkv, d, L)
    ws = attn.decode_workspace(b, hq, d, splits, dev)
    o_ws = torch.empty_like(o_na)
    for r, lens in enumerate(([2048, 1, 700, 2048], [5, 2047, 64, 1000], [2048] * 4)):
        lens_d.copy_(torch.tensor(lens, dtype=torch.int32))
        o_na.fill_(3.0)
        H.sync()
        g.replay()
        H.sync()
        attn.decode_attention_bf16(q, k, v, o_ws, b, hq, hkv, d, lens_d, L, L * hkv * d, splits,
                                   ws)
        H.sync()
        got = H.from_dev_bf16(o_na)
        assert np.array_equal(got, H.from_dev_bf16(o_ws)), f"replay {r} differs"
        exp = oracle.round_bf16(oracle.decode_batched(qb, kb, vb, lens))
        H.check_bar(H.bf16_bits_to_f32(got), exp, f"replay {r} vs oracle")
