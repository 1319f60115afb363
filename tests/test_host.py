"""Host-side checks that need no GPU: the C ABI library loads and exports
every declared entry point, argument validation happens on the host with
the documented status codes, workspace sizing, the synthetic generator, and
bench.py's single-GPU contract."""
import ctypes
import json
import os
import re
import subprocess
import sys

import numpy as np
import pytest

from toyinfer_amd import attn, synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "toyinfer_attn.h")
L = attn.LIB
P = 0x10000  # a 256-byte aligned stand-in address; never dereferenced here
INVALID, UNSUPPORTED, WORKSPACE = (attn.ERR_INVALID_ARGUMENT, attn.ERR_UNSUPPORTED,
                                   attn.ERR_WORKSPACE)


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(toyinfer_\w+)\s*\(", text)))


def test_every_declared_function_is_exported_and_bound():
    names = declared_functions()
    assert len(names) >= 15
    out = subprocess.run(["nm", "-D", "--defined-only", attn.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (toyinfer_\w+)", out))
    assert set(names) <= exported, set(names) - exported
    assert set(names) == set(attn.SIGNATURES), set(names) ^ set(attn.SIGNATURES)


def test_layer_op_validation():
    """Decoder-layer ops reject bad arguments before any launch."""
    assert L.toyinfer_rmsnorm_bf16(P, P, P, None, 1e-6, 7, None) == INVALID     # odd size
    assert L.toyinfer_rmsnorm_bf16(P + 2, P, P, None, 1e-6, 8, None) == INVALID  # 4-byte alignment
    assert L.toyinfer_batch_rmsnorm_bf16(P, P, P, P + 2, 1e-6, 2, 8, None) == INVALID
    assert L.toyinfer_batch_rmsnorm_bf16(P, P, P, None, 1e-6, 0, 8, None) == INVALID
    assert L.toyinfer_residual_add_bf16(P, None, 8, None) == INVALID
    assert L.toyinfer_batch_residual_add_bf16(P, P, 3, 5, None) == INVALID    # odd total
    assert L.toyinfer_swiglu_bf16x2(P, P, P, 0, None) == INVALID
    assert L.toyinfer_batch_swiglu_bf16x2(P, P, P + 2, 2, 8, None) == INVALID
    g = L.toyinfer_gather_embedding_bf16
    assert g(P, P, P, 0, 8, 10, None) == INVALID
    assert g(P, P, P, 70000, 8, 10, None) == INVALID                          # > 65535 tokens
    assert g(P, P + 2, P, 1, 8, 10, None) == INVALID                          # ids 4-byte aligned
    assert g(P, P, P, 1, 8, 0, None) == INVALID                               # empty vocabulary
    assert L.toyinfer_argmax_f32(P, 0, P, None) == INVALID
    assert L.toyinfer_argmax_f32(P, 10, None, None) == INVALID
    import ctypes
    ws = attn.sample_workspace_bytes()
    assert ws >= 256 + 2 * 32 * 256 * 4
    smp = L.toyinfer_sample_topk_topp_f32
    assert smp(P, 1000, 0.6, 0, 0.95, P, P, P, ws, None) == INVALID   # top_k 0 (asserted in the reference)
    assert smp(P, 1000, -0.5, 20, 0.95, P, P, P, ws, None) == INVALID  # negative temperature
    assert smp(P, 1000, float("nan"), 20, 0.95, P, P, P, ws, None) == INVALID
    assert smp(P, 0, 0.6, 20, 0.95, P, P, P, ws, None) == INVALID
    assert smp(P, 1000, 0.6, 20, 0.95, None, P, P, ws, None) == INVALID  # coin required
    assert smp(P, 1000, 0.6, 20, 0.95, P, P, P + 64, ws, None) == INVALID  # workspace alignment
    assert smp(P, 1000, 0.6, 257, 0.95, P, P, P, ws, None) == UNSUPPORTED  # k above the maximum
    assert smp(P, 262145, 0.6, 20, 0.95, P, P, P, ws, None) == UNSUPPORTED
    assert smp(P, 1000, 0.6, 20, 0.95, P, P, P, ws - 4, None) == WORKSPACE
    seg = L.toyinfer_gemm_segments_bf16
    W = (ctypes.c_void_p * 3)(P, P, P)
    Y = (ctypes.c_void_p * 3)(P, P, P)
    R = (ctypes.c_uint32 * 3)(64, 64, 64)
    assert seg(P, 100, 256, 4, W, Y, R, 0, None) == INVALID                   # at most 3 segments
    assert seg(P, 100, 256, 0, W, Y, R, 0, None) == INVALID
    assert seg(P, 4, 256, 3, W, Y, R, 0, None) == UNSUPPORTED                 # GEMV-sized batch
    assert seg(P, 100, 96, 3, W, Y, R, 0, None) == UNSUPPORTED                # N % 64 != 0
    assert seg(P + 2, 100, 256, 3, W, Y, R, 0, None) == UNSUPPORTED           # unaligned input


def test_model_header_functions_exported_and_bound():
    """include/toyinfer_qwen3.h: every function exported and bound by
    toyinfer_amd/qwen3.py (importing it binds them; no GPU call)."""
    from toyinfer_amd import qwen3
    text = re.sub(r"/\*.*?\*/", "", open(os.path.join(ROOT, "include", "toyinfer_qwen3.h")).read(),
                  flags=re.S)
    names = set(re.findall(r"\b(toyinfer_\w+)\s*\(", text))
    assert len(names) == 15
    out = subprocess.run(["nm", "-D", "--defined-only", attn.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    assert names <= set(re.findall(r"\bT (toyinfer_\w+)", out))
    assert names == set(qwen3._SIGS)


def test_model_config_validation():
    """Configuration and pointer checks run before any allocation."""
    import ctypes

    from toyinfer_amd import qwen3
    good = dict(num_layers=2, hidden_size=256, num_q_heads=4, num_kv_heads=2, head_dim=64,
                intermediate_size=512, vocab_size=1000, max_seq_len=64, max_prefill_tokens=32,
                rms_norm_eps=1e-6, rope_theta=1e6)
    cfg = qwen3.Config(**good)
    assert L.toyinfer_qwen3_state_bytes(ctypes.byref(cfg)) > 2 * 2 * 64 * 128 * 2
    for bad in (dict(head_dim=96), dict(num_kv_heads=3), dict(max_prefill_tokens=64),
                dict(hidden_size=100), dict(rms_norm_eps=0.0), dict(num_layers=0)):
        c = qwen3.Config(**dict(good, **bad))
        assert L.toyinfer_qwen3_state_bytes(ctypes.byref(c)) == 0, bad
    layers = (qwen3.Layer * 2)()
    for i in range(2):
        for n in qwen3.LAYER_FIELDS:
            setattr(layers[i], n, P)
    h = ctypes.c_void_p()
    create = L.toyinfer_qwen3_create
    layers[1].down_proj = P + 8                            # weights need 16-byte alignment
    assert create(ctypes.byref(cfg), P, P, P, layers, ctypes.byref(h)) == INVALID
    assert create(ctypes.byref(cfg), None, P, P, layers, ctypes.byref(h)) == INVALID
    c = qwen3.Config(**dict(good, head_dim=96))
    assert create(ctypes.byref(c), P, P, P, layers, ctypes.byref(h)) == UNSUPPORTED
    assert L.toyinfer_qwen3_prefill(None, P, 4) == INVALID
    assert L.toyinfer_qwen3_decode(None, 1, 1) == INVALID
    assert L.toyinfer_qwen3_set_sampling(None, 0.6, 20, 0.95, 1) == INVALID


def test_abi_version_and_status_strings():
    assert L.toyinfer_abi_version() == 1
    assert attn.status_string(0) == "ok"
    for st in (INVALID, UNSUPPORTED, WORKSPACE, attn.ERR_HIP, attn.ERR_IO):
        assert attn.status_string(st) not in ("ok", "unknown status")


def flash(q=P, k=P, v=P, o=P, hq=16, hkv=8, d=128, s=100, algo=0):
    return L.toyinfer_flash_attention_algo_bf16(q, k, v, o, hq, hkv, d, s, algo, None)


def test_prefill_argument_validation():
    assert flash(hkv=3) == INVALID                 # Hq % Hkv != 0
    assert flash(hq=0) == INVALID
    assert flash(d=96) == UNSUPPORTED              # the reference instantiates 64 and 128 only
    assert flash(s=0) == INVALID
    assert flash(q=None) == INVALID
    assert flash(k=P + 2) == INVALID               # 16-byte alignment
    assert flash(algo=5) == INVALID
    assert flash(s=1 << 30) == UNSUPPORTED         # K/V rows beyond 32-bit byte offsets
    assert L.toyinfer_flash_attention_v1_bf16(P, P, P, P, 8, 3, 128, 4, None) == INVALID


def test_fused_prefill_argument_validation():
    f = L.toyinfer_prefill_qknorm_rope_attention_bf16
    assert f(P, P, P, P, P, P, P, None, 1e-6, 32, 8, 128, 64, None) == INVALID   # no rope table
    assert f(P, P, P, P, P, P, P, P + 8, 1e-6, 32, 8, 128, 64, None) == INVALID  # table alignment
    assert f(P, P, P, P, None, P, P, P, 1e-6, 32, 8, 128, 64, None) == INVALID   # no K_out
    assert f(P, P, P, P, P, P, P, P, 1e-6, 32, 8, 64 + 32, 64, None) == UNSUPPORTED


def test_decode_reference_contract_validation():
    f = L.toyinfer_attention_bf16
    assert f(P, P, P, P, P, P, 32, 8, 128, 40, 40, None) == INVALID     # pos >= max_seq_len
    assert f(P, P, P, P, P, P, 32, 8, 128, 0, 0, None) == INVALID       # empty cache
    assert f(P, P, P, None, P, P, 32, 8, 128, 3, 40, None) == INVALID   # no score buffer
    assert f(P, P, P, P, P, P, 32, 6, 128, 3, 40, None) == INVALID
    g = L.toyinfer_attention_bf16_graph
    assert g(P, P, P, P, P, P, 32, 8, 128, None, 40, None) == INVALID   # no device pos
    assert g(P, P, P, P, P, P, 32, 8, 128, P + 2, 40, None) == INVALID


def test_batched_decode_validation_and_workspace():
    f = L.toyinfer_decode_attention_bf16
    ws = L.toyinfer_decode_workspace_bytes(8, 32, 128, 12)
    heads = 8 * 32

    def a256(x):
        return (x + 255) // 256 * 256
    # (m, l) pairs, then o[D] partials
    assert ws == a256(heads * 12 * 2 * 4) + heads * 12 * 128 * 4
    args = dict(q=P, k=P, v=P, o=P, b=8, hq=32, hkv=8, d=128, lens=None, L=4096,
                stride=4096 * 8 * 128, splits=12, w=P, wb=ws)

    def call(**kw):
        a = dict(args, **kw)
        return f(a["q"], a["k"], a["v"], a["o"], a["b"], a["hq"], a["hkv"], a["d"], a["lens"],
                 a["L"], a["stride"], a["splits"], a["w"], a["wb"], None)

    assert call(wb=ws - 1) == WORKSPACE
    assert call(b=0) == INVALID
    assert call(L=0) == INVALID
    assert call(stride=4095 * 8 * 128) == INVALID   # sequences would overlap
    assert call(splits=1025) == INVALID
    assert call(w=P + 64) == INVALID                # workspace 256-byte alignment
    assert call(lens=P + 1) == INVALID
    assert call(d=80) == UNSUPPORTED


def test_default_split_counts_are_bounded():
    for b, hq, hkv, L_ in [(8, 32, 8, 4096), (1, 32, 8, 32768), (1, 16, 8, 100), (3, 6, 3, 1)]:
        s = L.toyinfer_decode_default_splits(b, hq, hkv, 128, L_)
        assert 1 <= s <= max(1, -(-L_ // 128)) and s <= 1024


def test_prologue_op_validation():
    assert L.toyinfer_precompute_freq_f32(P, 127, 1e6, None) == INVALID
    assert L.toyinfer_precompute_freq_f32(None, 128, 1e6, None) == INVALID
    assert L.toyinfer_rope_cos_sin_f32(P, P, 0, 128, None) == INVALID
    assert L.toyinfer_batch_rope_bf16(P, None, 4, 8, 128, None) == INVALID
    assert L.toyinfer_batch_multi_rmsnorm_bf16(P, None, P, 1e-6, 4, 8, 128, None) == INVALID
    assert L.toyinfer_batch_multi_rmsnorm_bf16(P, P, P, 1e-6, 0, 8, 128, None) == INVALID
    assert L.toyinfer_multi_rmsnorm_bf16(P, P, P, 1e-6, 8, 96, None) == UNSUPPORTED
    # rows move with 16-byte accesses
    assert L.toyinfer_batch_rope_bf16(P + 2, P, 4, 8, 128, None) == INVALID
    assert L.toyinfer_batch_multi_rmsnorm_bf16(P, P + 8, P, 1e-6, 4, 8, 128, None) == INVALID
    assert L.toyinfer_qk_norm_rope_bf16(P, P, P + 4, P, 1e-6, 4, 8, 128, None) == INVALID


def test_decode_step_op_validation():
    """Bad arguments of the decode-step pre-pass ops are rejected before any launch."""
    assert L.toyinfer_rope_bf16(None, P, 3, 8, 128, None) == INVALID
    assert L.toyinfer_rope_bf16(P + 2, P, 3, 8, 128, None) == INVALID      # rows move 16 B at a time
    assert L.toyinfer_rope_bf16(P, P, 3, 0, 128, None) == INVALID
    assert L.toyinfer_rope_bf16(P, P, 3, 8, 80, None) == UNSUPPORTED
    assert L.toyinfer_rope_bf16_graph(P, P, None, 8, 128, None) == INVALID  # no device pos
    assert L.toyinfer_rope_bf16_graph(P, None, P, 8, 128, None) == INVALID
    w = L.toyinfer_write_kv_cache_bf16
    assert w(P, P, P, 7, None) == INVALID          # odd kv_dim: the reference moves bf16 pairs
    assert w(P, P, P, 0, None) == INVALID
    assert w(P, P + 2, P, 8, None) == INVALID      # cache rows need 4-byte alignment
    assert w(P, P, None, 8, None) == INVALID
    f = L.toyinfer_decode_qkv_prologue_bf16
    args = [P] * 7 + [64, 1e-6] + [P] * 3 + [32, 8, 128, None]
    a = list(args); a[7] = 0
    assert f(*a) == INVALID                        # empty cache
    a = list(args); a[2] = None
    assert f(*a) == INVALID                        # no v
    a = list(args); a[10] = P + 8
    assert f(*a) == INVALID                        # misaligned k_cache
    a = list(args); a[14] = 80
    assert f(*a) == UNSUPPORTED


def test_projection_validation():
    """Bad arguments of the projection ops are rejected before any launch."""
    g, gf, b = (L.toyinfer_gemv_proj_bf16, L.toyinfer_gemv_proj_bf162float,
                L.toyinfer_batch_gemv_proj_bf16)
    assert g(None, P, P, 8, 8, None) == INVALID
    assert g(P, P, P, 0, 8, None) == INVALID
    assert g(P, P, P, 8, 0, None) == INVALID
    assert g(P, P, P, 8, (1 << 22) + 1, None) == INVALID   # 32-bit byte offsets
    assert g(P + 1, P, P, 8, 8, None) == INVALID           # bf16 needs 2-byte alignment
    assert gf(P, P, P + 2, 8, 8, None) == INVALID          # fp32 out needs 4
    assert gf(P, None, P, 8, 8, None) == INVALID
    assert b(P, P, P, 0, 8, 8, None) == INVALID
    assert b(P, P, None, 3, 8, 8, None) == INVALID


def test_python_wrapper_raises_on_bad_status():
    class Fake:
        def __init__(self, addr):
            self.addr = addr

        def data_ptr(self):
            return self.addr

    with pytest.raises(attn.ToyInferError) as e:
        attn.flash_attention_v1_bf16(Fake(P), Fake(P), Fake(P), Fake(P), 4, 3, 128, 8, stream=0)
    assert e.value.status == INVALID


# ------------------------------------------------------ synthetic inputs

def test_generator_c_matches_numpy_specification():
    for seed, name, n in [(1, "q", 100003), (2026, "k", 4097), (7, "v", 1), (2 ** 63 + 9, "x", 2)]:
        assert np.array_equal(synth.normal_bf16(seed, name, (n,), use_c=True),
                              synth.normal_bf16(seed, name, (n,), use_c=False))
        assert np.array_equal(synth.uniform_bf16(seed, name, (n,), 0.9, 1.1, use_c=True),
                              synth.uniform_bf16(seed, name, (n,), 0.9, 1.1, use_c=False))
        b = synth.normal_bf16(seed, name, (n,))
        assert np.array_equal(synth.scale_bf16(b, 0.02, use_c=True),
                              synth.scale_bf16(b, 0.02, use_c=False))


def test_generator_pinned_values_and_statistics():
    assert synth.normal_bf16(2026, "q", (8,)).tolist() == [16346, 16293, 49012, 49049, 49147,
                                                            16008, 16289, 48714]
    assert synth.uniform_bf16(2026, "gamma_q", (4,), 0.9, 1.1).tolist() == [16268, 16257,
                                                                            16267, 16267]
    z = synth.bf16_bits_to_f32(synth.normal_bf16(3, "stats", (1 << 20,))).astype(np.float64)
    assert abs(z.mean()) < 5e-3 and abs(z.std() - 1) < 5e-3
    assert abs((np.abs(z) > 1.96).mean() - 0.05) < 2e-3
    u = synth.bf16_bits_to_f32(synth.uniform_bf16(3, "u", (1 << 16,), 0.9, 1.1))
    assert u.min() >= 0.9 - 1e-2 and u.max() <= 1.1 + 1e-2


def test_generator_ln_and_sincos_accuracy():
    u = np.linspace(1e-12, 1.0, 200001)
    assert np.abs(synth._ln(u) - np.log(u)).max() < 1e-14
    w = np.linspace(0, 1, 200001, endpoint=False)
    s, c = synth._sincos_2pi(w)
    assert np.abs(s - np.sin(2 * np.pi * w)).max() < 1e-14
    assert np.abs(c - np.cos(2 * np.pi * w)).max() < 1e-14


# --------------------------------------------------------------- bench.py

def test_bench_refuses_more_than_one_gpu():
    res = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                         capture_output=True, text=True, timeout=300)
    assert res.returncode != 0
    msg = json.loads(res.stdout.strip().splitlines()[-1])
    assert "one GPU" in msg["error"]


# ------------------------------------------------------- drop-in C++ header

CALL_SITES = r"""
#include "kernel_warpper.h"
using toyinfer::bf16;
void prefill(const bf16* q, const bf16* k, const bf16* v, bf16* o, uint32_t hd, hipStream_t s) {
    // the instantiations src/prefill.cu:433-452 provides
    toyinfer::flash_attention_v1_bf16<32, 2, 64>(q, k, v, o, 16, 8, hd, 100);
    toyinfer::flash_attention_v1_bf16<32, 4, 64>(q, k, v, o, 16, 8, hd, 100);
    toyinfer::flash_attention_v1_bf16<32, 4, 128>(q, k, v, o, 16, 8, hd, 100, s);
    toyinfer::flash_attention_v1_bf16<64, 4, 128>(q, k, v, o, 16, 8, hd, 100, s);
}
void decode(const bf16* q, const bf16* k, const bf16* v, float* sc, float* ob, bf16* o,
            const uint32_t* pos_d, hipStream_t s) {
    toyinfer::attention_bf16<256, 32>(q, k, v, sc, ob, o, 32, 8, 128, 5, 40);
    toyinfer::attention_bf16_graph<256, 32>(q, k, v, sc, ob, o, 32, 8, 128, pos_d, 40, s);
}
void prologue(bf16* x, const bf16* w, float* f, hipStream_t s) {
    toyinfer::precompute_freq_f32(f, 128, 1e6f);
    toyinfer::batch_multi_rmsnorm_bf16(x, w, x, 1e-6f, 7, 8, 128, s);
    toyinfer::multi_rmsnorm_bf16(x, w, x, 1e-6f, 8, 128);
    toyinfer::batch_rope_bf16(x, f, 7, 8, 128, s);
}
"""


def compile_snippet(tmp_path, text):
    src = tmp_path / "snippet.cpp"
    src.write_text(text)
    return subprocess.run(["/opt/rocm/llvm/bin/clang++", "-std=c++17", "-fsyntax-only", "-Wall",
                           "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
                           "-I" + os.path.join(ROOT, "include"), str(src)],
                          capture_output=True, text=True, timeout=120)


def test_dropin_header_compiles_reference_call_sites(tmp_path):
    res = compile_snippet(tmp_path, CALL_SITES)
    assert res.returncode == 0, res.stderr


@pytest.mark.parametrize("bad", ["toyinfer::flash_attention_v1_bf16<32, 4, 96>(q, q, q, o, 1, 1, 96, 1);",
                                 "toyinfer::flash_attention_v1_bf16<48, 4, 128>(q, q, q, o, 1, 1, 128, 1);",
                                 "toyinfer::attention_bf16<100, 32>(q, q, q, f, f, o, 1, 1, 128, 0, 1);"])
def test_dropin_header_rejects_illegal_instantiations(tmp_path, bad):
    text = ('#include "kernel_warpper.h"\nusing toyinfer::bf16;\n'
            "void f_(const bf16* q, bf16* o, float* f) { " + bad + " }\n")
    res = compile_snippet(tmp_path, text)
    assert res.returncode != 0 and "static assertion failed" in res.stderr
