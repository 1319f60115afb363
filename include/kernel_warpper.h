// Drop-in launch-wrapper header for the attention hot path.
//
// Same file name, namespace and template signatures as the reference's
// include/kernel_warpper.h for the functions on the attention path, so the
// reference's call sites (src/transformer.cpp:20-39 prefill dispatch,
// :380-391 QK-norm/RoPE, :569-573 decode, and the kernel tests) compile
// unchanged apart from the stream type (hipStream_t).  Each wrapper forwards
// to the C ABI in toyinfer_attn.h (libtoyinfer_attn.so, gfx950 kernels) and,
// like the reference's CUDA_CHECK (src/kernel_common.cuh:11-20), prints the
// error and exits the process on a non-zero status.  The template
// parameters Bc/Br/NUM_THREADS/TILE_SEQ are the reference's CUDA tile
// shapes; here they are checked for legality and otherwise ignored (the
// kernels pick their own gfx950 tiling).  HEAD_DIM must equal heads_dim.
//
// Compile callers with ROCm's clang (hipcc or amdclang++); bf16 is HIP's
// 2-byte IEEE bfloat16, layout-compatible with the reference's bf16.
// Link: -L<lib dir> -ltoyinfer_attn -lamdhip64.
#pragma once

#include <hip/hip_bf16.h>
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <cstdlib>
#include <iostream>

#include "toyinfer_attn.h"

namespace toyinfer {
using bf16 = __hip_bfloat16;    // include/kernel_warpper.h:9
using bf162 = __hip_bfloat162;  // include/kernel_warpper.h:10

static_assert(sizeof(bf16) == 2 && sizeof(bf162) == 4, "bf16 must be a 2-byte type");

namespace detail {
inline void check(int status, const char* what, const char* file, int line) {
    if (status == TOYINFER_OK) return;
    std::cerr << "toyinfer error: " << toyinfer_status_string(status) << " (" << status
              << ") in " << what << " at " << file << ':' << line;
    if (status == TOYINFER_ERR_HIP) {
        const int e = toyinfer_last_hip_error();
        std::cerr << ": " << hipGetErrorString(static_cast<hipError_t>(e)) << " (" << e << ")";
    }
    std::cerr << std::endl;
    std::exit(EXIT_FAILURE);
}
}  // namespace detail

#define TOYINFER_CHECK(call, name) ::toyinfer::detail::check((call), name, __FILE__, __LINE__)

// ---------------------------------------------------------------- prefill

// include/kernel_warpper.h:128-135, src/prefill.cu:381-395.  Causal GQA
// attention over positions 0..seq_len-1: Qs/Os [S][Hq][D], Ks/Vs [S][Hkv][D].
template <const uint32_t Bc, const uint32_t Br, const uint32_t HEAD_DIM>
void flash_attention_v1_bf16(const bf16* __restrict__ Qs, const bf16* __restrict__ Ks,
                             const bf16* __restrict__ Vs, bf16* __restrict__ Os,
                             const uint32_t num_q_heads, const uint32_t num_kv_heads,
                             const uint32_t heads_dim, const uint32_t seq_len,
                             hipStream_t stream_d = nullptr) {
    static_assert(HEAD_DIM == 64 || HEAD_DIM == 128, "HEAD_DIM must be 64 or 128");
    static_assert(Bc > 0 && Br > 0 && HEAD_DIM % Bc == 0, "HEAD_DIM % Bc must be 0");
    if (heads_dim != HEAD_DIM)
        detail::check(TOYINFER_ERR_INVALID_ARGUMENT, "flash_attention_v1_bf16 (heads_dim != HEAD_DIM)",
                      __FILE__, __LINE__);
    TOYINFER_CHECK(toyinfer_flash_attention_v1_bf16(Qs, Ks, Vs, Os, num_q_heads, num_kv_heads,
                                                    heads_dim, seq_len, stream_d),
                   "flash_attention_v1_bf16");
}

// ----------------------------------------------------------------- decode

// include/kernel_warpper.h:98-105, src/decode.cu:665-701.  One sequence:
// Q [Hq][D], Ks/Vs [max_seq_len][Hkv][D] attending to rows 0..pos.  On
// return score [Hq][max_seq_len] holds the softmax probabilities (zeros past
// pos), O_buffer [Hq][D] the fp32 output and O its bf16 rounding.
template <const uint32_t NUM_THREADS, const uint32_t TILE_SEQ>
void attention_bf16(const bf16* __restrict__ Q, const bf16* __restrict__ Ks,
                    const bf16* __restrict__ Vs, float* __restrict__ score,
                    float* __restrict__ O_buffer, bf16* __restrict__ O,
                    const uint32_t num_q_heads, const uint32_t num_kv_heads,
                    const uint32_t heads_dim, const uint32_t pos, const uint32_t max_seq_len,
                    hipStream_t stream_d = nullptr) {
    static_assert(NUM_THREADS > 0 && NUM_THREADS <= 1024 && NUM_THREADS % 32 == 0 && TILE_SEQ > 0,
                  "illegal launch shape");
    TOYINFER_CHECK(toyinfer_attention_bf16(Q, Ks, Vs, score, O_buffer, O, num_q_heads, num_kv_heads,
                                           heads_dim, pos, max_seq_len, stream_d),
                   "attention_bf16");
}

// include/kernel_warpper.h:107-114, src/decode.cu:703-744: the same with pos
// read on the device from *pos_d, so one captured graph serves every step.
template <const uint32_t NUM_THREADS, const uint32_t TILE_SEQ>
void attention_bf16_graph(const bf16* __restrict__ Q, const bf16* __restrict__ Ks,
                          const bf16* __restrict__ Vs, float* __restrict__ score,
                          float* __restrict__ O_buffer, bf16* __restrict__ O,
                          const uint32_t num_q_heads, const uint32_t num_kv_heads,
                          const uint32_t heads_dim, const uint32_t* __restrict__ pos_d,
                          const uint32_t max_seq_len, hipStream_t stream_d = nullptr) {
    static_assert(NUM_THREADS > 0 && NUM_THREADS <= 1024 && NUM_THREADS % 32 == 0 && TILE_SEQ > 0,
                  "illegal launch shape");
    TOYINFER_CHECK(toyinfer_attention_bf16_graph(Q, Ks, Vs, score, O_buffer, O, num_q_heads,
                                                 num_kv_heads, heads_dim, pos_d, max_seq_len,
                                                 stream_d),
                   "attention_bf16_graph");
}

// Extension: the engine's decode call site (src/transformer.cpp:569-573) with
// `score` used as scratch (no probabilities written) and O_buffer / O as the
// contract defines them; a drop-in replacement there, since the engine reads
// neither score nor O_buffer afterwards.
template <const uint32_t NUM_THREADS, const uint32_t TILE_SEQ>
void attention_bf16_graph_lean(const bf16* __restrict__ Q, const bf16* __restrict__ Ks,
                               const bf16* __restrict__ Vs, float* __restrict__ score,
                               float* __restrict__ O_buffer, bf16* __restrict__ O,
                               const uint32_t num_q_heads, const uint32_t num_kv_heads,
                               const uint32_t heads_dim, const uint32_t* __restrict__ pos_d,
                               const uint32_t max_seq_len, hipStream_t stream_d = nullptr) {
    static_assert(NUM_THREADS > 0 && NUM_THREADS <= 1024 && NUM_THREADS % 32 == 0 && TILE_SEQ > 0,
                  "illegal launch shape");
    TOYINFER_CHECK(toyinfer_attention_bf16_graph_lean(Q, Ks, Vs, score, O_buffer, O, num_q_heads,
                                                      num_kv_heads, heads_dim, pos_d,
                                                      max_seq_len, stream_d),
                   "attention_bf16_graph_lean");
}

// ------------------------------------------- QK-norm, RoPE and inv_freq

// include/kernel_warpper.h:23, src/decode.cu:43-50 (legacy default stream).
inline void precompute_freq_f32(float* inv_freq, int n, float base) {
    TOYINFER_CHECK(toyinfer_precompute_freq_f32(inv_freq, n, base, nullptr), "precompute_freq_f32");
}

// include/kernel_warpper.h:39-42; input may alias output.
inline void multi_rmsnorm_bf16(const bf16* input, const bf16* __restrict__ weight, bf16* output,
                               const float rms_norm_eps, const uint32_t nums_head,
                               const uint32_t head_dim, hipStream_t stream_d = nullptr) {
    TOYINFER_CHECK(toyinfer_multi_rmsnorm_bf16(input, weight, output, rms_norm_eps, nums_head,
                                               head_dim, stream_d),
                   "multi_rmsnorm_bf16");
}

// include/kernel_warpper.h:45-50; input may alias output.
inline void batch_multi_rmsnorm_bf16(const bf16* input, const bf16* __restrict__ weight,
                                     bf16* output, const float rms_norm_eps,
                                     const uint32_t num_tokens, const uint32_t nums_head,
                                     const uint32_t head_dim, hipStream_t stream_d = nullptr) {
    TOYINFER_CHECK(toyinfer_batch_multi_rmsnorm_bf16(input, weight, output, rms_norm_eps,
                                                     num_tokens, nums_head, head_dim, stream_d),
                   "batch_multi_rmsnorm_bf16");
}

// include/kernel_warpper.h:88-90: in place, token t at position t.
inline void batch_rope_bf16(bf16* qk_ptr, const float* __restrict__ inv_freq,
                            const uint32_t num_tokens, const uint32_t nums_head,
                            const uint32_t head_dim, hipStream_t stream_d = nullptr) {
    TOYINFER_CHECK(toyinfer_batch_rope_bf16(qk_ptr, inv_freq, num_tokens, nums_head, head_dim,
                                            stream_d),
                   "batch_rope_bf16");
}

// include/kernel_warpper.h:79-81: in place, every head at position pos.
inline void rope_bf16(bf16* qk_ptr, const float* __restrict__ inv_freq, uint32_t pos,
                      const uint32_t nums_head, const uint32_t head_dim,
                      hipStream_t stream_d = nullptr) {
    TOYINFER_CHECK(toyinfer_rope_bf16(qk_ptr, inv_freq, pos, nums_head, head_dim, stream_d),
                   "rope_bf16");
}

// include/kernel_warpper.h:83-86: the position is read from pos_d when the
// kernel runs (graph replays see each new position).
inline void rope_bf16_graph(bf16* qk_ptr, const float* __restrict__ inv_freq,
                            const uint32_t* __restrict__ pos_d, const uint32_t nums_head,
                            const uint32_t head_dim, hipStream_t stream_d = nullptr) {
    TOYINFER_CHECK(toyinfer_rope_bf16_graph(qk_ptr, inv_freq, pos_d, nums_head, head_dim,
                                            stream_d),
                   "rope_bf16_graph");
}

// include/kernel_warpper.h:92-96: kv_dim values to cache row *pos_d.
// NUM_THREADS does not change the kernel.
template <const uint32_t NUM_THREADS>
void write_kv_cache_bf16(const bf16* __restrict__ src, bf16* __restrict__ cache,
                         const uint32_t* __restrict__ pos_d, const uint32_t kv_dim,
                         hipStream_t stream_d = nullptr) {
    static_assert(NUM_THREADS > 0 && NUM_THREADS <= 1024, "illegal launch shape");
    TOYINFER_CHECK(toyinfer_write_kv_cache_bf16(src, cache, pos_d, kv_dim, stream_d),
                   "write_kv_cache_bf16");
}

// include/kernel_warpper.h:53-57: y = W * hidden_states, bf16 out.
// NUM_THREADS does not change the kernel.
template <const uint32_t NUM_THREADS>
void gemv_proj_bf16(const bf16* __restrict__ W, const bf16* __restrict__ hidden_states,
                    bf16* __restrict__ y, const uint32_t M, const uint32_t N,
                    hipStream_t stream_d = nullptr) {
    static_assert(NUM_THREADS > 0 && NUM_THREADS <= 1024, "illegal launch shape");
    TOYINFER_CHECK(toyinfer_gemv_proj_bf16(W, hidden_states, y, M, N, stream_d),
                   "gemv_proj_bf16");
}

// include/kernel_warpper.h:59-64: num_tokens rows of hidden_states.
template <const uint32_t NUM_THREADS>
void batch_gemv_proj_bf16(const bf16* __restrict__ W, const bf16* __restrict__ hidden_states,
                          bf16* __restrict__ y, const uint32_t num_tokens, const uint32_t M,
                          const uint32_t N, hipStream_t stream_d = nullptr) {
    static_assert(NUM_THREADS > 0 && NUM_THREADS <= 1024, "illegal launch shape");
    TOYINFER_CHECK(toyinfer_batch_gemv_proj_bf16(W, hidden_states, y, num_tokens, M, N, stream_d),
                   "batch_gemv_proj_bf16");
}

// include/kernel_warpper.h:66-70: fp32 out (the lm-head).
template <const uint32_t NUM_THREADS>
void gemv_proj_bf162float(const bf16* __restrict__ W, const bf16* __restrict__ hidden_states,
                          float* __restrict__ y, const uint32_t M, const uint32_t N,
                          hipStream_t stream_d = nullptr) {
    static_assert(NUM_THREADS > 0 && NUM_THREADS <= 1024, "illegal launch shape");
    TOYINFER_CHECK(toyinfer_gemv_proj_bf162float(W, hidden_states, y, M, N, stream_d),
                   "gemv_proj_bf162float");
}

// include/kernel_warpper.h:12-15 and :17-21: hidden_state += residual (bf16).
template <const uint32_t NUM_THREADS>
void residual_add_bf16(const bf16* __restrict__ residual, bf16* __restrict__ hidden_state,
                       const uint32_t size, hipStream_t stream_d = nullptr) {
    static_assert(NUM_THREADS > 0 && NUM_THREADS <= 1024, "illegal launch shape");
    TOYINFER_CHECK(toyinfer_residual_add_bf16(residual, hidden_state, size, stream_d),
                   "residual_add_bf16");
}
template <const uint32_t NUM_THREADS>
void batch_residual_add_bf16(const bf16* __restrict__ residual, bf16* __restrict__ hidden_state,
                             const uint32_t num_tokens, const uint32_t size,
                             hipStream_t stream_d = nullptr) {
    static_assert(NUM_THREADS > 0 && NUM_THREADS <= 1024, "illegal launch shape");
    TOYINFER_CHECK(toyinfer_batch_residual_add_bf16(residual, hidden_state, num_tokens, size,
                                                    stream_d),
                   "batch_residual_add_bf16");
}

// include/kernel_warpper.h:25-29 and :31-36: full-row RMSNorm; *sum (per
// row) receives the sum of squares, as in the reference.
template <const uint32_t NUM_THREADS>
void rmsnorm_bf16(const bf16* __restrict__ input, const bf16* __restrict__ weight, bf16* output,
                  float* sum, const float rms_norm_eps, const uint32_t size,
                  hipStream_t stream_d = nullptr) {
    static_assert(NUM_THREADS > 0 && NUM_THREADS <= 1024, "illegal launch shape");
    TOYINFER_CHECK(toyinfer_rmsnorm_bf16(input, weight, output, sum, rms_norm_eps, size, stream_d),
                   "rmsnorm_bf16");
}
template <const uint32_t NUM_THREADS>
void batch_rmsnorm_bf16(const bf16* __restrict__ input, const bf16* __restrict__ weight,
                        bf16* output, float* sum, const float rms_norm_eps,
                        const uint32_t num_tokens, const uint32_t size,
                        hipStream_t stream_d = nullptr) {
    static_assert(NUM_THREADS > 0 && NUM_THREADS <= 1024, "illegal launch shape");
    TOYINFER_CHECK(toyinfer_batch_rmsnorm_bf16(input, weight, output, sum, rms_norm_eps,
                                               num_tokens, size, stream_d),
                   "batch_rmsnorm_bf16");
}

// include/kernel_warpper.h:71-77: rows of the table by device token ids
// (ids are not range-checked, as in the reference).
template <const uint32_t NUM_THREADS>
void gather_embedding_bf16(const bf16* __restrict__ embedding_table,
                           const uint32_t* __restrict__ token_ids,
                           bf16* __restrict__ hidden_states, const uint32_t num_tokens,
                           const uint32_t hidden_size, hipStream_t stream_d = nullptr) {
    static_assert(NUM_THREADS > 0 && NUM_THREADS <= 1024, "illegal launch shape");
    TOYINFER_CHECK(toyinfer_gather_embedding_bf16(embedding_table, token_ids, hidden_states,
                                                  num_tokens, hidden_size, 0xffffffffu, stream_d),
                   "gather_embedding_bf16");
}

// include/kernel_warpper.h:116-126: intermedia = bf16(up * silu(gate)).
template <const uint32_t NUM_THREADS>
void swiglu_bf16x2(const bf16* __restrict__ gate, const bf16* __restrict__ up,
                   bf16* __restrict__ intermedia, const uint32_t size,
                   hipStream_t stream_d = nullptr) {
    static_assert(NUM_THREADS > 0 && NUM_THREADS <= 1024, "illegal launch shape");
    TOYINFER_CHECK(toyinfer_swiglu_bf16x2(gate, up, intermedia, size, stream_d), "swiglu_bf16x2");
}
template <const uint32_t NUM_THREADS>
void batch_swiglu_bf16x2(const bf16* __restrict__ gate, const bf16* __restrict__ up,
                         bf16* __restrict__ intermedia, const uint32_t num_tokens,
                         const uint32_t size, hipStream_t stream_d = nullptr) {
    static_assert(NUM_THREADS > 0 && NUM_THREADS <= 1024, "illegal launch shape");
    TOYINFER_CHECK(toyinfer_batch_swiglu_bf16x2(gate, up, intermedia, num_tokens, size, stream_d),
                   "batch_swiglu_bf16x2");
}

// ------------------------------------------------------------- extensions
// Entry points with no counterpart in the reference: batched split-K decode,
// the prefill with QK-RMSNorm + RoPE fused in front, and the decode step's
// norm/RoPE/cache-write pre-pass in one launch.

// src/transformer.cpp:535-552 (multi_rmsnorm_bf16 x2, rope_bf16_graph x2,
// write_kv_cache_bf16 x2) in one launch; pos = min(*pos_d, max_seq_len - 1).
inline void decode_qkv_prologue_bf16(const bf16* q, const bf16* k, const bf16* v,
                                     const bf16* q_norm_weight, const bf16* k_norm_weight,
                                     const float* inv_freq, const uint32_t* pos_d,
                                     uint32_t max_seq_len, float rms_norm_eps, bf16* q_out,
                                     bf16* k_cache, bf16* v_cache, uint32_t num_q_heads,
                                     uint32_t num_kv_heads, uint32_t head_dim,
                                     hipStream_t stream_d = nullptr) {
    TOYINFER_CHECK(toyinfer_decode_qkv_prologue_bf16(
                       q, k, v, q_norm_weight, k_norm_weight, inv_freq, pos_d, max_seq_len,
                       rms_norm_eps, q_out, k_cache, v_cache, num_q_heads, num_kv_heads, head_dim,
                       stream_d),
                   "decode_qkv_prologue_bf16");
}

// Rotary (cos, sin) table [num_positions][D/2][2], built once per model.
inline void rope_cos_sin_f32(float* table, const float* inv_freq, uint32_t num_positions,
                             uint32_t head_dim, hipStream_t stream_d = nullptr) {
    TOYINFER_CHECK(toyinfer_rope_cos_sin_f32(table, inv_freq, num_positions, head_dim, stream_d),
                   "rope_cos_sin_f32");
}

// batch_multi_rmsnorm_bf16 followed by batch_rope_bf16 in one pass.
inline void qk_norm_rope_bf16(const bf16* input, const bf16* weight, bf16* output,
                              const float* inv_freq, float rms_norm_eps, uint32_t num_tokens,
                              uint32_t nums_head, uint32_t head_dim,
                              hipStream_t stream_d = nullptr) {
    TOYINFER_CHECK(toyinfer_qk_norm_rope_bf16(input, weight, output, inv_freq, rms_norm_eps,
                                              num_tokens, nums_head, head_dim, stream_d),
                   "qk_norm_rope_bf16");
}

// Per-head RMSNorm + RoPE on Q and K (one pass over K, fused into the
// attention kernel for Q), then causal attention; K_out receives the
// normalised, rotated K (the KV-cache value).  Inputs are not modified.
inline void prefill_qknorm_rope_attention_bf16(
    const bf16* Q_raw, const bf16* K_raw, const bf16* Vs, bf16* Os, bf16* K_out,
    const bf16* q_gamma, const bf16* k_gamma, const float* rope_cos_sin, float eps,
    uint32_t num_q_heads, uint32_t num_kv_heads, uint32_t heads_dim, uint32_t seq_len,
    hipStream_t stream_d = nullptr) {
    TOYINFER_CHECK(toyinfer_prefill_qknorm_rope_attention_bf16(
                       Q_raw, K_raw, Vs, Os, K_out, q_gamma, k_gamma, rope_cos_sin, eps,
                       num_q_heads, num_kv_heads, heads_dim, seq_len, stream_d),
                   "prefill_qknorm_rope_attention_bf16");
}

// Batched decode: q/o [B][Hq][D], sequence b's cache at k/v + b*kv_batch_stride
// elements ([max_len][Hkv][D]), length seq_lens_d[b] (device) or seq_len for
// all when seq_lens_d is null.  workspace: decode_workspace_bytes(...) bytes
// (no initialisation needed).  Calls sharing a workspace must not overlap.
inline void decode_attention_bf16(const bf16* q, const bf16* k_cache, const bf16* v_cache, bf16* o,
                                  uint32_t batch, uint32_t num_q_heads, uint32_t num_kv_heads,
                                  uint32_t heads_dim, const uint32_t* seq_lens_d, uint32_t seq_len,
                                  uint64_t kv_batch_stride, uint32_t num_splits, void* workspace,
                                  size_t workspace_bytes, hipStream_t stream_d = nullptr) {
    TOYINFER_CHECK(toyinfer_decode_attention_bf16(q, k_cache, v_cache, o, batch, num_q_heads,
                                                  num_kv_heads, heads_dim, seq_lens_d, seq_len,
                                                  kv_batch_stride, num_splits, workspace,
                                                  workspace_bytes, stream_d),
                   "decode_attention_bf16");
}

inline uint32_t decode_default_splits(uint32_t batch, uint32_t num_q_heads, uint32_t num_kv_heads,
                                      uint32_t heads_dim, uint32_t seq_len) {
    return toyinfer_decode_default_splits(batch, num_q_heads, num_kv_heads, heads_dim, seq_len);
}

inline size_t decode_workspace_bytes(uint32_t batch, uint32_t num_q_heads, uint32_t heads_dim,
                                     uint32_t num_splits) {
    return toyinfer_decode_workspace_bytes(batch, num_q_heads, heads_dim, num_splits);
}

}  // namespace toyinfer
