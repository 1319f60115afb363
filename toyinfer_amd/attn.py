"""Python host side of the MI355X attention path, over the C ABI.

Mirrors the reference's launch-wrapper API (include/kernel_warpper.h) with
the same names, argument meaning and order; device buffers are torch tensors
on a ROCm device (PyTorch is only the allocator and stream provider here).
Every call goes through ``toyinfer_amd/lib/libtoyinfer_attn.so``; there is no
CPU fallback: if the library is missing, loading this module fails loudly.

Errors: the C ABI returns a status; a non-zero status raises
``ToyInferError`` (the reference instead prints and calls exit(EXIT_FAILURE),
src/kernel_common.cuh:11-20; the C++ drop-in header keeps that behaviour).
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libtoyinfer_attn.so")

OK = 0
ERR_INVALID_ARGUMENT = 1
ERR_UNSUPPORTED = 2
ERR_WORKSPACE = 3
ERR_HIP = 4
ERR_IO = 5

# Every entry point of include/toyinfer_attn.h, with its ctypes signature.
_vp, _u32, _u64, _f32, _i32, _sz = (ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64,
                                    ctypes.c_float, ctypes.c_int, ctypes.c_size_t)
SIGNATURES = {
    "toyinfer_status_string": (ctypes.c_char_p, [_i32]),
    "toyinfer_last_hip_error": (_i32, []),
    "toyinfer_abi_version": (_u32, []),
    "toyinfer_flash_attention_v1_bf16": (_i32, [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _vp]),
    "toyinfer_flash_attention_algo_bf16": (_i32, [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _i32,
                                                  _vp]),
    "toyinfer_prefill_qknorm_rope_attention_bf16": (
        _i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _f32, _u32, _u32, _u32, _u32, _vp]),
    "toyinfer_attention_bf16": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32,
                                       _u32, _vp]),
    "toyinfer_attention_bf16_graph": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _vp,
                                             _u32, _vp]),
    "toyinfer_attention_bf16_graph_lean": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32,
                                                  _vp, _u32, _vp]),
    "toyinfer_decode_attention_bf16": (_i32, [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _vp,
                                              _u32, _u64, _u32, _vp, _sz, _vp]),
    "toyinfer_decode_attention_bf16_noalloc": (_i32, [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32,
                                                      _vp, _u32, _u64, _u32, _vp]),
    "toyinfer_decode_default_splits": (_u32, [_u32, _u32, _u32, _u32, _u32]),
    "toyinfer_decode_workspace_bytes": (_sz, [_u32, _u32, _u32, _u32]),
    "toyinfer_precompute_freq_f32": (_i32, [_vp, _i32, _f32, _vp]),
    "toyinfer_rope_cos_sin_f32": (_i32, [_vp, _vp, _u32, _u32, _vp]),
    "toyinfer_multi_rmsnorm_bf16": (_i32, [_vp, _vp, _vp, _f32, _u32, _u32, _vp]),
    "toyinfer_batch_multi_rmsnorm_bf16": (_i32, [_vp, _vp, _vp, _f32, _u32, _u32, _u32, _vp]),
    "toyinfer_batch_rope_bf16": (_i32, [_vp, _vp, _u32, _u32, _u32, _vp]),
    "toyinfer_qk_norm_rope_bf16": (_i32, [_vp, _vp, _vp, _vp, _f32, _u32, _u32, _u32, _vp]),
    "toyinfer_rope_bf16": (_i32, [_vp, _vp, _u32, _u32, _u32, _vp]),
    "toyinfer_rope_bf16_graph": (_i32, [_vp, _vp, _vp, _u32, _u32, _vp]),
    "toyinfer_write_kv_cache_bf16": (_i32, [_vp, _vp, _vp, _u32, _vp]),
    "toyinfer_gemv_proj_bf16": (_i32, [_vp, _vp, _vp, _u32, _u32, _vp]),
    "toyinfer_gemv_proj_bf162float": (_i32, [_vp, _vp, _vp, _u32, _u32, _vp]),
    "toyinfer_batch_gemv_proj_bf16": (_i32, [_vp, _vp, _vp, _u32, _u32, _u32, _vp]),
    "toyinfer_gemm_segments_bf16": (_i32, [_vp, _u32, _u32, _u32, _vp, _vp, _vp, _i32, _vp]),
    "toyinfer_gemm_swiglu_bf16": (_i32, [_vp, _u32, _u32, _vp, _vp, _u32, _vp, _vp]),
    "toyinfer_rmsnorm_bf16": (_i32, [_vp, _vp, _vp, _vp, _f32, _u32, _vp]),
    "toyinfer_batch_rmsnorm_bf16": (_i32, [_vp, _vp, _vp, _vp, _f32, _u32, _u32, _vp]),
    "toyinfer_residual_add_bf16": (_i32, [_vp, _vp, _u32, _vp]),
    "toyinfer_batch_residual_add_bf16": (_i32, [_vp, _vp, _u32, _u32, _vp]),
    "toyinfer_swiglu_bf16x2": (_i32, [_vp, _vp, _vp, _u32, _vp]),
    "toyinfer_batch_swiglu_bf16x2": (_i32, [_vp, _vp, _vp, _u32, _u32, _vp]),
    "toyinfer_gather_embedding_bf16": (_i32, [_vp, _vp, _vp, _u32, _u32, _u32, _vp]),
    "toyinfer_argmax_f32": (_i32, [_vp, _u32, _vp, _vp]),
    "toyinfer_sample_workspace_bytes": (_sz, []),
    "toyinfer_sample_topk_topp_f32": (_i32, [_vp, _u32, _f32, _u32, _f32, _vp, _vp, _vp, _sz,
                                             _vp]),
    "toyinfer_decode_qkv_prologue_bf16": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _u32, _f32,
                                                 _vp, _vp, _vp, _u32, _u32, _u32, _vp]),
}


class ToyInferError(RuntimeError):
    def __init__(self, fn: str, status: int, hip_error: int = 0):
        self.status = status
        self.hip_error = hip_error
        msg = f"{fn}: {status_string(status)} (status {status})"
        if status == ERR_HIP:
            msg += f", hipError {hip_error}"
        super().__init__(msg)


def _load() -> ctypes.CDLL:
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} not found: build the HIP library first "
            "(python -m toyinfer_amd.build, or __graft_entry__.build())")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


LIB = _load()


def status_string(status: int) -> str:
    return LIB.toyinfer_status_string(status).decode()


def _check(fn: str, status: int) -> None:
    if status != OK:
        raise ToyInferError(fn, status, LIB.toyinfer_last_hip_error() if status == ERR_HIP else 0)


# ------------------------------------------------------------ tensor glue

def _ptr(t) -> Optional[int]:
    """Device address of a torch tensor (None passes a null pointer)."""
    if t is None:
        return None
    return int(t.data_ptr())


def _stream(stream) -> Optional[int]:
    """hipStream_t handle: an int, a torch.cuda.Stream, or None for torch's
    current stream on the current device."""
    if isinstance(stream, int):
        return stream
    import torch

    if stream is None:
        stream = torch.cuda.current_stream()
    return int(stream.cuda_stream)


# ---------------------------------------------------------------- prefill

def flash_attention_v1_bf16(Qs, Ks, Vs, Os, num_q_heads: int, num_kv_heads: int, heads_dim: int,
                            seq_len: int, stream=None) -> None:
    """Causal GQA prefill (include/kernel_warpper.h:128-135).
    Qs [S][Hq][D], Ks/Vs [S][Hkv][D], Os [S][Hq][D]: bf16 device tensors."""
    _check("flash_attention_v1_bf16",
           LIB.toyinfer_flash_attention_v1_bf16(_ptr(Qs), _ptr(Ks), _ptr(Vs), _ptr(Os),
                                                num_q_heads, num_kv_heads, heads_dim, seq_len,
                                                _stream(stream)))


ALGO_AUTO, ALGO_SPLIT_KEYS, ALGO_ROW_TILES, ALGO_SPLIT_PAIRS, ALGO_ROW_PAIRS = 0, 1, 2, 3, 4


def flash_attention_algo_bf16(Qs, Ks, Vs, Os, num_q_heads: int, num_kv_heads: int,
                              heads_dim: int, seq_len: int, algo: int, stream=None) -> None:
    """Prefill with an explicit kernel choice (0 auto, 1 split keys, 2 row tiles,
    3 split keys with GQA head pairs, 4 row tiles with GQA head pairs)."""
    _check("flash_attention_algo_bf16",
           LIB.toyinfer_flash_attention_algo_bf16(_ptr(Qs), _ptr(Ks), _ptr(Vs), _ptr(Os),
                                                  num_q_heads, num_kv_heads, heads_dim, seq_len,
                                                  algo, _stream(stream)))


def prefill_qknorm_rope_attention_bf16(Q_raw, K_raw, Vs, Os, K_out, q_gamma, k_gamma,
                                       rope_cos_sin, rms_norm_eps: float, num_q_heads: int,
                                       num_kv_heads: int, heads_dim: int, seq_len: int,
                                       stream=None) -> None:
    """QK-RMSNorm + RoPE fused in front of causal GQA prefill; rope_cos_sin is
    the fp32 [>= S][D/2][2] table from rope_cos_sin_f32."""
    _check("prefill_qknorm_rope_attention_bf16",
           LIB.toyinfer_prefill_qknorm_rope_attention_bf16(
               _ptr(Q_raw), _ptr(K_raw), _ptr(Vs), _ptr(Os), _ptr(K_out), _ptr(q_gamma),
               _ptr(k_gamma), _ptr(rope_cos_sin), rms_norm_eps, num_q_heads, num_kv_heads,
               heads_dim, seq_len, _stream(stream)))


# ----------------------------------------------------------------- decode

def attention_bf16(Q, Ks, Vs, score, O_buffer, O, num_q_heads: int, num_kv_heads: int,
                   heads_dim: int, pos: int, max_seq_len: int, stream=None) -> None:
    """Single-sequence decode, reference contract (include/kernel_warpper.h:98-105)."""
    _check("attention_bf16",
           LIB.toyinfer_attention_bf16(_ptr(Q), _ptr(Ks), _ptr(Vs), _ptr(score), _ptr(O_buffer),
                                       _ptr(O), num_q_heads, num_kv_heads, heads_dim, pos,
                                       max_seq_len, _stream(stream)))


def attention_bf16_graph(Q, Ks, Vs, score, O_buffer, O, num_q_heads: int, num_kv_heads: int,
                         heads_dim: int, pos_d, max_seq_len: int, stream=None) -> None:
    """Decode with pos read on the device (include/kernel_warpper.h:107-114)."""
    _check("attention_bf16_graph",
           LIB.toyinfer_attention_bf16_graph(_ptr(Q), _ptr(Ks), _ptr(Vs), _ptr(score),
                                             _ptr(O_buffer), _ptr(O), num_q_heads, num_kv_heads,
                                             heads_dim, _ptr(pos_d), max_seq_len,
                                             _stream(stream)))


def attention_bf16_graph_lean(Q, Ks, Vs, score, O_buffer, O, num_q_heads: int,
                              num_kv_heads: int, heads_dim: int, pos_d, max_seq_len: int,
                              stream=None) -> None:
    """The engine's decode call with score as scratch: O and O_buffer only."""
    _check("attention_bf16_graph_lean",
           LIB.toyinfer_attention_bf16_graph_lean(_ptr(Q), _ptr(Ks), _ptr(Vs), _ptr(score),
                                                  _ptr(O_buffer), _ptr(O), num_q_heads,
                                                  num_kv_heads, heads_dim, _ptr(pos_d),
                                                  max_seq_len, _stream(stream)))


def decode_default_splits(batch: int, num_q_heads: int, num_kv_heads: int, heads_dim: int,
                          seq_len: int) -> int:
    return int(LIB.toyinfer_decode_default_splits(batch, num_q_heads, num_kv_heads, heads_dim,
                                                  seq_len))


def decode_workspace_bytes(batch: int, num_q_heads: int, heads_dim: int, num_splits: int) -> int:
    return int(LIB.toyinfer_decode_workspace_bytes(batch, num_q_heads, heads_dim, num_splits))


def decode_workspace(batch: int, num_q_heads: int, heads_dim: int, num_splits: int, device):
    """An uninitialised uint8 workspace tensor sized for these shapes."""
    import torch

    return torch.empty(decode_workspace_bytes(batch, num_q_heads, heads_dim, num_splits),
                       dtype=torch.uint8, device=device)


def decode_attention_bf16(q, k_cache, v_cache, o, batch: int, num_q_heads: int,
                          num_kv_heads: int, heads_dim: int, seq_lens_d, seq_len: int,
                          kv_batch_stride: int, num_splits: int, workspace,
                          stream=None) -> None:
    """Batched split-K decode; workspace is a device tensor (any dtype) of at least
    decode_workspace_bytes(...) bytes (see decode_workspace)."""
    ws_bytes = workspace.numel() * workspace.element_size()
    _check("decode_attention_bf16",
           LIB.toyinfer_decode_attention_bf16(_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(o), batch,
                                              num_q_heads, num_kv_heads, heads_dim,
                                              _ptr(seq_lens_d), seq_len, kv_batch_stride,
                                              num_splits, _ptr(workspace), ws_bytes,
                                              _stream(stream)))


DECODE_SCRATCH_BYTES = 8 << 20  # TOYINFER_DECODE_SCRATCH_BYTES


def decode_attention_bf16_noalloc(q, k_cache, v_cache, o, batch: int, num_q_heads: int,
                                  num_kv_heads: int, heads_dim: int, seq_lens_d, seq_len: int,
                                  kv_batch_stride: int, num_splits: int, stream=None) -> None:
    """decode_attention_bf16 with the split partials in the library's own
    per-GPU device array (no workspace argument, nothing allocated)."""
    _check("decode_attention_bf16_noalloc",
           LIB.toyinfer_decode_attention_bf16_noalloc(_ptr(q), _ptr(k_cache), _ptr(v_cache),
                                                      _ptr(o), batch, num_q_heads, num_kv_heads,
                                                      heads_dim, _ptr(seq_lens_d), seq_len,
                                                      kv_batch_stride, num_splits,
                                                      _stream(stream)))


# ------------------------------------------------------------ prologue ops

def precompute_freq_f32(inv_freq, head_dim: int, theta: float, stream=None) -> None:
    _check("precompute_freq_f32",
           LIB.toyinfer_precompute_freq_f32(_ptr(inv_freq), head_dim, theta, _stream(stream)))


def rope_cos_sin_f32(table, inv_freq, num_positions: int, head_dim: int, stream=None) -> None:
    """table [num_positions][D/2][2] fp32 = (cos, sin)(t * inv_freq[i])."""
    _check("rope_cos_sin_f32",
           LIB.toyinfer_rope_cos_sin_f32(_ptr(table), _ptr(inv_freq), num_positions, head_dim,
                                         _stream(stream)))


def multi_rmsnorm_bf16(input, weight, output, rms_norm_eps: float, nums_head: int,
                       head_dim: int, stream=None) -> None:
    _check("multi_rmsnorm_bf16",
           LIB.toyinfer_multi_rmsnorm_bf16(_ptr(input), _ptr(weight), _ptr(output), rms_norm_eps,
                                           nums_head, head_dim, _stream(stream)))


def batch_multi_rmsnorm_bf16(input, weight, output, rms_norm_eps: float, num_tokens: int,
                             nums_head: int, head_dim: int, stream=None) -> None:
    _check("batch_multi_rmsnorm_bf16",
           LIB.toyinfer_batch_multi_rmsnorm_bf16(_ptr(input), _ptr(weight), _ptr(output),
                                                 rms_norm_eps, num_tokens, nums_head, head_dim,
                                                 _stream(stream)))


def batch_rope_bf16(qk, inv_freq, num_tokens: int, nums_head: int, head_dim: int,
                    stream=None) -> None:
    _check("batch_rope_bf16",
           LIB.toyinfer_batch_rope_bf16(_ptr(qk), _ptr(inv_freq), num_tokens, nums_head, head_dim,
                                        _stream(stream)))


def qk_norm_rope_bf16(input, weight, output, inv_freq, rms_norm_eps: float, num_tokens: int,
                      nums_head: int, head_dim: int, stream=None) -> None:
    _check("qk_norm_rope_bf16",
           LIB.toyinfer_qk_norm_rope_bf16(_ptr(input), _ptr(weight), _ptr(output), _ptr(inv_freq),
                                          rms_norm_eps, num_tokens, nums_head, head_dim,
                                          _stream(stream)))


def rope_bf16(qk, inv_freq, pos: int, nums_head: int, head_dim: int, stream=None) -> None:
    _check("rope_bf16",
           LIB.toyinfer_rope_bf16(_ptr(qk), _ptr(inv_freq), pos, nums_head, head_dim,
                                  _stream(stream)))


def rope_bf16_graph(qk, inv_freq, pos_d, nums_head: int, head_dim: int, stream=None) -> None:
    _check("rope_bf16_graph",
           LIB.toyinfer_rope_bf16_graph(_ptr(qk), _ptr(inv_freq), _ptr(pos_d), nums_head, head_dim,
                                        _stream(stream)))


def write_kv_cache_bf16(src, cache, pos_d, kv_dim: int, stream=None) -> None:
    _check("write_kv_cache_bf16",
           LIB.toyinfer_write_kv_cache_bf16(_ptr(src), _ptr(cache), _ptr(pos_d), kv_dim,
                                            _stream(stream)))


def decode_qkv_prologue_bf16(q, k, v, q_norm_weight, k_norm_weight, inv_freq, pos_d,
                             max_seq_len: int, rms_norm_eps: float, q_out, k_cache, v_cache,
                             num_q_heads: int, num_kv_heads: int, head_dim: int,
                             stream=None) -> None:
    """Fused decode-step pre-pass: q_norm+RoPE of q into q_out, k_norm+RoPE of k
    into row *pos_d of k_cache, v into row *pos_d of v_cache (one launch)."""
    _check("decode_qkv_prologue_bf16",
           LIB.toyinfer_decode_qkv_prologue_bf16(
               _ptr(q), _ptr(k), _ptr(v), _ptr(q_norm_weight), _ptr(k_norm_weight),
               _ptr(inv_freq), _ptr(pos_d), max_seq_len, rms_norm_eps, _ptr(q_out),
               _ptr(k_cache), _ptr(v_cache), num_q_heads, num_kv_heads, head_dim,
               _stream(stream)))


# ------------------------------------------------------------ projections

def gemv_proj_bf16(W, hidden_states, y, M: int, N: int, stream=None) -> None:
    """y[m] = sum_n W[m][n] hidden_states[n] (bf16 out): include/kernel_warpper.h:53-57."""
    _check("gemv_proj_bf16",
           LIB.toyinfer_gemv_proj_bf16(_ptr(W), _ptr(hidden_states), _ptr(y), M, N,
                                       _stream(stream)))


def gemv_proj_bf162float(W, hidden_states, y, M: int, N: int, stream=None) -> None:
    """The same with fp32 out (lm-head): include/kernel_warpper.h:66-70."""
    _check("gemv_proj_bf162float",
           LIB.toyinfer_gemv_proj_bf162float(_ptr(W), _ptr(hidden_states), _ptr(y), M, N,
                                             _stream(stream)))


def batch_gemv_proj_bf16(W, hidden_states, y, num_tokens: int, M: int, N: int,
                         stream=None) -> None:
    """y[t][m] = sum_n W[m][n] hidden_states[t][n]: include/kernel_warpper.h:59-64."""
    _check("batch_gemv_proj_bf16",
           LIB.toyinfer_batch_gemv_proj_bf16(_ptr(W), _ptr(hidden_states), _ptr(y),
                                             num_tokens, M, N, _stream(stream)))


def gemm_segments_bf16(hidden_states, num_tokens: int, N: int, Ws, ys, rows, residual=False,
                       stream=None) -> None:
    """Stacked projections of one input (extension): ys[s] = x * Ws[s]^T [+ ys[s]]."""
    n = len(Ws)
    w_arr = (ctypes.c_void_p * n)(*[_ptr(w) for w in Ws])
    y_arr = (ctypes.c_void_p * n)(*[_ptr(y) for y in ys])
    r_arr = (ctypes.c_uint32 * n)(*rows)
    _check("gemm_segments_bf16",
           LIB.toyinfer_gemm_segments_bf16(_ptr(hidden_states), num_tokens, N, n, w_arr, y_arr,
                                           r_arr, int(bool(residual)), _stream(stream)))


def gemm_swiglu_bf16(hidden_states, num_tokens: int, N: int, W_gate, W_up, M: int, out,
                     stream=None) -> None:
    """Gate/up projections with SwiGLU in the epilogue (extension):
    out = bf16(bf16(up) * silu(bf16(gate)))."""
    _check("gemm_swiglu_bf16",
           LIB.toyinfer_gemm_swiglu_bf16(_ptr(hidden_states), num_tokens, N, _ptr(W_gate),
                                         _ptr(W_up), M, _ptr(out), _stream(stream)))


# ------------------------------------------------- rest of a decoder layer

def rmsnorm_bf16(input, weight, output, sum, eps: float, size: int, stream=None) -> None:
    """include/kernel_warpper.h:25-29; sum may be None."""
    _check("rmsnorm_bf16", LIB.toyinfer_rmsnorm_bf16(_ptr(input), _ptr(weight), _ptr(output),
                                                     _ptr(sum), eps, size, _stream(stream)))


def batch_rmsnorm_bf16(input, weight, output, sum, eps: float, num_tokens: int, size: int,
                       stream=None) -> None:
    """include/kernel_warpper.h:31-36; sum may be None."""
    _check("batch_rmsnorm_bf16",
           LIB.toyinfer_batch_rmsnorm_bf16(_ptr(input), _ptr(weight), _ptr(output), _ptr(sum),
                                           eps, num_tokens, size, _stream(stream)))


def residual_add_bf16(residual, hidden_state, size: int, stream=None) -> None:
    _check("residual_add_bf16",
           LIB.toyinfer_residual_add_bf16(_ptr(residual), _ptr(hidden_state), size,
                                          _stream(stream)))


def batch_residual_add_bf16(residual, hidden_state, num_tokens: int, size: int,
                            stream=None) -> None:
    _check("batch_residual_add_bf16",
           LIB.toyinfer_batch_residual_add_bf16(_ptr(residual), _ptr(hidden_state), num_tokens,
                                                size, _stream(stream)))


def swiglu_bf16x2(gate, up, intermedia, size: int, stream=None) -> None:
    _check("swiglu_bf16x2", LIB.toyinfer_swiglu_bf16x2(_ptr(gate), _ptr(up), _ptr(intermedia),
                                                       size, _stream(stream)))


def batch_swiglu_bf16x2(gate, up, intermedia, num_tokens: int, size: int, stream=None) -> None:
    _check("batch_swiglu_bf16x2",
           LIB.toyinfer_batch_swiglu_bf16x2(_ptr(gate), _ptr(up), _ptr(intermedia), num_tokens,
                                            size, _stream(stream)))


def gather_embedding_bf16(table, token_ids, hidden_states, num_tokens: int, hidden_size: int,
                          vocab_size: int = 0xFFFFFFFF, stream=None) -> None:
    _check("gather_embedding_bf16",
           LIB.toyinfer_gather_embedding_bf16(_ptr(table), _ptr(token_ids), _ptr(hidden_states),
                                              num_tokens, hidden_size, vocab_size,
                                              _stream(stream)))


def argmax_f32(logits, n: int, out_index, stream=None) -> None:
    _check("argmax_f32", LIB.toyinfer_argmax_f32(_ptr(logits), n, _ptr(out_index),
                                                 _stream(stream)))


def sample_workspace_bytes() -> int:
    return int(LIB.toyinfer_sample_workspace_bytes())


def sample_topk_topp_f32(logits, vocab: int, temperature: float, top_k: int, top_p: float,
                         coin, out_token, workspace, stream=None) -> None:
    """Device top-k/top-p pick (src/sampler.cpp:18-67); coin is a device
    float in [0, 1); workspace zero-filled before its first use."""
    _check("sample_topk_topp_f32",
           LIB.toyinfer_sample_topk_topp_f32(_ptr(logits), vocab, temperature, top_k, top_p,
                                             _ptr(coin), _ptr(out_token), _ptr(workspace),
                                             workspace.numel() * workspace.element_size(),
                                             _stream(stream)))

