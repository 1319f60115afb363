/*
 * C ABI of the MI355X (gfx950) attention path for ToyInfer.
 *
 * Plain pointers, sizes and an opaque stream (a hipStream_t, NULL = the
 * legacy default stream, as in the reference).  Every entry point validates
 * its arguments on the host before touching the GPU and returns a status
 * code; none of them allocates, frees or synchronises, so all are safe to
 * enqueue while a stream is being captured into a HIP graph.  bf16 tensors
 * are 2-byte IEEE bfloat16 values (layout of __nv_bfloat16 / __hip_bfloat16).
 *
 * Citations name the reference launcher each function replaces
 * (paths are into the wiketool/ToyInfer tree).
 */
#ifndef TOYINFER_ATTN_H_
#define TOYINFER_ATTN_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TOYINFER_ABI_VERSION 1u

/* Status codes. */
#define TOYINFER_OK 0
#define TOYINFER_ERR_INVALID_ARGUMENT 1 /* shape, pointer or alignment precondition failed */
#define TOYINFER_ERR_UNSUPPORTED 2      /* valid in principle, not implemented (e.g. head_dim) */
#define TOYINFER_ERR_WORKSPACE 3        /* caller workspace too small */
#define TOYINFER_ERR_HIP 4              /* a HIP call failed; see toyinfer_last_hip_error() */
#define TOYINFER_ERR_IO 5               /* a model file is missing, unreadable or malformed */

const char* toyinfer_status_string(int status);
/* hipError_t of the most recent TOYINFER_ERR_HIP returned on this thread. */
int toyinfer_last_hip_error(void);
uint32_t toyinfer_abi_version(void);

/* ---------------------------------------------------------------- prefill */

/* Causal GQA prefill attention.  Replaces toyinfer::flash_attention_v1_bf16
 * <Bc, Br, HEAD_DIM> (include/kernel_warpper.h:128-135; src/prefill.cu:381-395).
 * Qs [S][Hq][D], Ks/Vs [S][Hkv][D], Os [S][Hq][D], bf16, token-major,
 * positions 0..S-1.  D in {64, 128}; Hq % Hkv == 0; S >= 1.
 * Pointers 16-byte aligned.  Writes Os[0..S) only. */
int toyinfer_flash_attention_v1_bf16(const void* Qs, const void* Ks, const void* Vs, void* Os,
                                     uint32_t num_q_heads, uint32_t num_kv_heads,
                                     uint32_t heads_dim, uint32_t seq_len, void* stream);

/* Same, with the kernel chosen explicitly (extension, for tuning and tests):
 * algo 0 = pick by shape (what toyinfer_flash_attention_v1_bf16 does),
 * 1 = 32-row workgroups whose waves split the keys (short sequences),
 * 2 = 128-row workgroups of one head (long sequences),
 * 3 = as 1 with both query heads of a GQA pair in one workgroup sharing
 *     each K/V tile (as 1 when Hq/Hkv is odd),
 * 4 = as 2 with both query heads of a GQA pair in one workgroup (as 2 when
 *     Hq/Hkv is odd).  Algo 0 picks among them by shape. */
int toyinfer_flash_attention_algo_bf16(const void* Qs, const void* Ks, const void* Vs, void* Os,
                                       uint32_t num_q_heads, uint32_t num_kv_heads,
                                       uint32_t heads_dim, uint32_t seq_len, int algo,
                                       void* stream);

/* Prefill with Qwen3's pre-attention ops fused in front: per-head RMSNorm of
 * Q and K (eps, gamma [D]) -> bf16 -> RoPE at position = token index -> bf16,
 * then causal GQA attention.  Equivalent to batch_multi_rmsnorm_bf16 +
 * batch_rope_bf16 on Q and K followed by flash_attention_v1_bf16, as
 * src/transformer.cpp:380-404 sequences them.  The rotation angles come from
 * rope_cos_sin [>= S][D/2][2] (fp32 (cos, sin), 16-byte aligned), built once
 * per model with toyinfer_rope_cos_sin_f32.  Q_raw is read only (normalised
 * and rotated on load); the normalised and rotated K is written to K_out
 * [S][Hkv][D] (may alias K_raw; typically the layer's KV-cache slot), then
 * used as the attention's K.  All tensor pointers 16-byte aligned. */
int toyinfer_prefill_qknorm_rope_attention_bf16(
    const void* Q_raw, const void* K_raw, const void* Vs, void* Os, void* K_out,
    const void* q_gamma, const void* k_gamma, const float* rope_cos_sin, float rms_norm_eps,
    uint32_t num_q_heads, uint32_t num_kv_heads, uint32_t heads_dim, uint32_t seq_len,
    void* stream);

/* ----------------------------------------------------------------- decode */

/* Single-token decode attention over one sequence's KV cache, reference
 * contract.  Replaces toyinfer::attention_bf16<NUM_THREADS, TILE_SEQ>
 * (include/kernel_warpper.h:98-105; src/decode.cu:665-701).
 * Q [Hq][D]; Ks/Vs [max_seq_len][Hkv][D] (rows 0..pos used); D in {64, 128}.
 * Outputs as the reference leaves them: score [Hq][max_seq_len] = softmax
 * probabilities for t <= pos and 0 for t > pos; O_buffer [Hq][D] = fp32
 * output; O [Hq][D] = bf16(O_buffer).  score and O_buffer also serve as the
 * split-K workspace, so no other memory is used. */
int toyinfer_attention_bf16(const void* Q, const void* Ks, const void* Vs, float* score,
                            float* O_buffer, void* O, uint32_t num_q_heads,
                            uint32_t num_kv_heads, uint32_t heads_dim, uint32_t pos,
                            uint32_t max_seq_len, void* stream);

/* Same, with pos read on the device from *pos_d when the kernels run, so the
 * call can be captured once into a graph and replayed for every position.
 * Replaces toyinfer::attention_bf16_graph<NUM_THREADS, TILE_SEQ>
 * (include/kernel_warpper.h:107-114; src/decode.cu:703-744).  A device pos
 * >= max_seq_len is clamped to max_seq_len - 1. */
int toyinfer_attention_bf16_graph(const void* Q, const void* Ks, const void* Vs, float* score,
                                  float* O_buffer, void* O, uint32_t num_q_heads,
                                  uint32_t num_kv_heads, uint32_t heads_dim,
                                  const uint32_t* pos_d, uint32_t max_seq_len, void* stream);

/* The engine's decode call (src/transformer.cpp:569-573) without the parts of
 * the contract the engine never reads (extension, same arguments as
 * toyinfer_attention_bf16_graph, pos read from pos_d on the device): O =
 * bf16 attention output and O_buffer = the same in fp32, as the contract
 * defines them; score is scratch (it holds the split partials, not the
 * probabilities) and may hold anything afterwards.  Only kernels are
 * launched, so a captured graph replays it at each new position.  For a
 * caller that reads score (the reference's tests), keep
 * toyinfer_attention_bf16_graph. */
int toyinfer_attention_bf16_graph_lean(const void* Q, const void* Ks, const void* Vs,
                                       float* score, float* O_buffer, void* O,
                                       uint32_t num_q_heads, uint32_t num_kv_heads,
                                       uint32_t heads_dim, const uint32_t* pos_d,
                                       uint32_t max_seq_len, void* stream);

/* Batched split-K decode attention (extension; the reference runs one
 * sequence per attention_bf16 call).  Only O is produced.
 * q [B][Hq][D]; sequence b's cache rows at k_cache/v_cache + b*kv_batch_stride
 * elements, row t of KV head h at + (t*Hkv + h)*D; o [B][Hq][D].
 * Lengths: seq_lens_d (device, [B], each in 1..seq_len) or, if NULL, every
 * sequence has length seq_len.  num_splits = 0 picks a default (at most
 * 1024 splits are accepted); the workspace must hold
 * toyinfer_decode_workspace_bytes(B, Hq, D, splits) bytes (256-byte
 * aligned) for the split count used; its contents need no initialisation.
 * Calls that share a workspace must not overlap. */
int toyinfer_decode_attention_bf16(const void* q, const void* k_cache, const void* v_cache,
                                   void* o, uint32_t batch, uint32_t num_q_heads,
                                   uint32_t num_kv_heads, uint32_t heads_dim,
                                   const uint32_t* seq_lens_d, uint32_t seq_len,
                                   uint64_t kv_batch_stride, uint32_t num_splits,
                                   void* workspace, size_t workspace_bytes, void* stream);
/* Split count num_splits = 0 resolves to for these shapes. */
uint32_t toyinfer_decode_default_splits(uint32_t batch, uint32_t num_q_heads,
                                        uint32_t num_kv_heads, uint32_t heads_dim,
                                        uint32_t seq_len);
size_t toyinfer_decode_workspace_bytes(uint32_t batch, uint32_t num_q_heads, uint32_t heads_dim,
                                       uint32_t num_splits);

/* toyinfer_decode_attention_bf16 without a workspace argument: the split
 * partials live in a device array inside this library (one copy per GPU,
 * TOYINFER_DECODE_SCRATCH_BYTES, held until the process ends), so the call
 * allocates nothing.  No counterpart in the reference: it is for callers that
 * cannot allocate device memory (code under graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  Same arguments, checks, kernels
 * and results as toyinfer_decode_attention_bf16 with the same split count;
 * TOYINFER_ERR_WORKSPACE when toyinfer_decode_workspace_bytes(batch,
 * num_q_heads, heads_dim, splits) exceeds TOYINFER_DECODE_SCRATCH_BYTES.
 * Every call on one GPU uses that GPU's array: calls that overlap on one GPU
 * (other streams, other threads) race and must be ordered by the caller.
 * The array's address is looked up on the first call on each device (the
 * device current at the call). */
#define TOYINFER_DECODE_SCRATCH_BYTES (8u << 20)
int toyinfer_decode_attention_bf16_noalloc(const void* q, const void* k_cache,
                                           const void* v_cache, void* o, uint32_t batch,
                                           uint32_t num_q_heads, uint32_t num_kv_heads,
                                           uint32_t heads_dim, const uint32_t* seq_lens_d,
                                           uint32_t seq_len, uint64_t kv_batch_stride,
                                           uint32_t num_splits, void* stream);

/* --------------------------------------------- Qwen3 pre-attention ops
 * bf16 tensors and gamma are 16-byte aligned (rows are moved with 16-byte
 * accesses); inv_freq 4-byte aligned. */

/* inv_freq[i] = 1 / powf(theta, 2i/D), i < D/2.  Replaces
 * toyinfer::precompute_freq_f32 (include/kernel_warpper.h:23; src/decode.cu:35-50). */
int toyinfer_precompute_freq_f32(float* inv_freq, int head_dim, float theta, void* stream);

/* Rotary table (extension): table[t][i] = (cosf, sinf)((float)t * inv_freq[i])
 * for t < num_positions, i < D/2, fp32 pairs; the same values batch_rope_bf16
 * computes per element, built once per model (like precompute_freq_f32). */
int toyinfer_rope_cos_sin_f32(float* table, const float* inv_freq, uint32_t num_positions,
                              uint32_t head_dim, void* stream);

/* Per-head RMSNorm, y = bf16(x / sqrt(mean(x^2) + eps) * w), rows of D.
 * input may equal output.  Replaces toyinfer::multi_rmsnorm_bf16
 * (include/kernel_warpper.h:39-42; src/decode.cu:144-199). */
int toyinfer_multi_rmsnorm_bf16(const void* input, const void* weight, void* output,
                                float rms_norm_eps, uint32_t nums_head, uint32_t head_dim,
                                void* stream);
/* Replaces toyinfer::batch_multi_rmsnorm_bf16 (include/kernel_warpper.h:45-50;
 * src/prefill.cu:114-122): the same over num_tokens * nums_head rows. */
int toyinfer_batch_multi_rmsnorm_bf16(const void* input, const void* weight, void* output,
                                      float rms_norm_eps, uint32_t num_tokens,
                                      uint32_t nums_head, uint32_t head_dim, void* stream);

/* Rotate-half RoPE in place, angle = token * inv_freq[i] for token
 * 0..num_tokens-1, pairs (i, i + D/2), outputs rounded to bf16.  Replaces
 * toyinfer::batch_rope_bf16 (include/kernel_warpper.h:88-90; src/prefill.cu:185-218). */
int toyinfer_batch_rope_bf16(void* qk, const float* inv_freq, uint32_t num_tokens,
                             uint32_t nums_head, uint32_t head_dim, void* stream);

/* Fused per-head RMSNorm -> bf16 -> RoPE(position = token) -> bf16 in one
 * pass (extension: batch_multi_rmsnorm_bf16 then batch_rope_bf16 in one
 * kernel).  input may equal output. */
int toyinfer_qk_norm_rope_bf16(const void* input, const void* weight, void* output,
                               const float* inv_freq, float rms_norm_eps, uint32_t num_tokens,
                               uint32_t nums_head, uint32_t head_dim, void* stream);

/* ------------------------------------------- decode-step pre-pass ops
 * One decoded token: q [Hq][D], k and v [Hkv][D]; caches [positions][Hkv][D]
 * (one layer's K or V cache base, as the reference passes them).  All bf16
 * tensors 16-byte aligned; pos_d and inv_freq 4-byte aligned. */

/* Rotate-half RoPE in place at position pos for all nums_head rows,
 * angle = (float)pos * inv_freq[i].  Replaces toyinfer::rope_bf16
 * (include/kernel_warpper.h:79-81; src/decode.cu:301-324, 353-361). */
int toyinfer_rope_bf16(void* qk, const float* inv_freq, uint32_t pos, uint32_t nums_head,
                       uint32_t head_dim, void* stream);
/* The same with the position read from device memory (*pos_d) when the
 * kernel runs, so a captured graph replays at each new position.  Replaces
 * toyinfer::rope_bf16_graph (include/kernel_warpper.h:83-86;
 * src/decode.cu:326-351, 363-372). */
int toyinfer_rope_bf16_graph(void* qk, const float* inv_freq, const uint32_t* pos_d,
                             uint32_t nums_head, uint32_t head_dim, void* stream);
/* cache[*pos_d * kv_dim + i] = src[i], i < kv_dim (even).  *pos_d must be a
 * row the cache holds, as in the reference.  Replaces
 * toyinfer::write_kv_cache_bf16<NUM_THREADS> (include/kernel_warpper.h:92-96;
 * src/decode.cu:374-397). */
int toyinfer_write_kv_cache_bf16(const void* src, void* cache, const uint32_t* pos_d,
                                 uint32_t kv_dim, void* stream);
/* Fused decode-step pre-pass (extension): in one launch, per-head RMSNorm
 * -> bf16 -> RoPE(pos) -> bf16 of q into q_out (q_out may equal q) and of k
 * into row pos of k_cache, and v copied into row pos of v_cache, with
 * pos = min(*pos_d, max_seq_len - 1) read on the device.  Replaces the six
 * launches of src/transformer.cpp:535-552 (multi_rmsnorm_bf16 x2,
 * rope_bf16_graph x2, write_kv_cache_bf16 x2) with the same rounding points. */
int toyinfer_decode_qkv_prologue_bf16(const void* q, const void* k, const void* v,
                                      const void* q_norm_weight, const void* k_norm_weight,
                                      const float* inv_freq, const uint32_t* pos_d,
                                      uint32_t max_seq_len, float rms_norm_eps, void* q_out,
                                      void* k_cache, void* v_cache, uint32_t num_q_heads,
                                      uint32_t num_kv_heads, uint32_t head_dim, void* stream);

/* ---- Projections (the attention path's producers and consumer) ----
 * W is [M][N] bf16 row-major, x is [num_tokens][N] bf16, y[t][m] =
 * sum_n W[m][n] * x[t][n] accumulated in fp32 and rounded once.  Only
 * y[0 .. num_tokens * M) is written.  M, N, num_tokens >= 1, N <= 2^22;
 * pointers aligned to their element size (16-byte alignment and
 * N % 8 == 0 select the vector path). */

/* Decode projection, bf16 out.  Replaces toyinfer::gemv_proj_bf16<NUM_THREADS>
 * (include/kernel_warpper.h:53-57; src/decode.cu:201-248). */
int toyinfer_gemv_proj_bf16(const void* W, const void* hidden_states, void* y, uint32_t M,
                            uint32_t N, void* stream);
/* Decode projection, fp32 out (the lm-head).  Replaces
 * toyinfer::gemv_proj_bf162float<NUM_THREADS> (include/kernel_warpper.h:66-70;
 * src/decode.cu:250-298). */
int toyinfer_gemv_proj_bf162float(const void* W, const void* hidden_states, float* y,
                                  uint32_t M, uint32_t N, void* stream);
/* Prefill projection over num_tokens rows, bf16 out: an MFMA GEMM when
 * num_tokens > 4, N % 64 == 0 and W and hidden_states are 16-byte aligned,
 * else the GEMV over groups of 4 tokens.  Replaces
 * toyinfer::batch_gemv_proj_bf16<NUM_THREADS> (include/kernel_warpper.h:59-64;
 * src/prefill.cu:124-174). */
int toyinfer_batch_gemv_proj_bf16(const void* W, const void* hidden_states, void* y,
                                  uint32_t num_tokens, uint32_t M, uint32_t N, void* stream);
/* Extension: up to three projections of the same hidden_states in one MFMA
 * GEMM launch (the stacked q/k/v or gate/up of a layer): y[s] [num_tokens]
 * [rows[s]] = hidden_states * W[s]^T; with residual != 0, y[s] = bf16(y[s] +
 * bf16(product)) (a projection followed by the residual add).  Needs
 * num_tokens > 4, N % 64 == 0 and 16-byte aligned hidden_states and W[s];
 * each element equals what toyinfer_batch_gemv_proj_bf16 gives for it. */
int toyinfer_gemm_segments_bf16(const void* hidden_states, uint32_t num_tokens, uint32_t N,
                                uint32_t num_segments, const void* const* W, void* const* y,
                                const uint32_t* rows, int residual, void* stream);
/* Extension: the gate and up projections of one layer with SwiGLU in the
 * GEMM epilogue: out[t][m] = bf16(bf16(up) * silu(bf16(gate))), gate =
 * hidden_states * W_gate^T, up = hidden_states * W_up^T ([M][N] each), i.e.
 * two toyinfer_batch_gemv_proj_bf16 calls followed by
 * toyinfer_batch_swiglu_bf16x2 (the sequence at src/transformer.cpp:434-444,
 * include/kernel_warpper.h:59-64 and :121-126) in one launch, bit for bit.
 * Needs num_tokens > 4, N % 64 == 0 and 16-byte aligned operands. */
int toyinfer_gemm_swiglu_bf16(const void* hidden_states, uint32_t num_tokens, uint32_t N,
                              const void* W_gate, const void* W_up, uint32_t M, void* out,
                              void* stream);

/* ---- The rest of a Qwen3 decoder layer (for the model harness) ----
 * bf16 tensors need 4-byte alignment (16 bytes and sizes % 8 == 0 take the
 * vector path); sizes are even, as the reference's bf16x2 kernels assume. */

/* output = bf16(input * rsqrt(sum/size + eps) * weight) over one row of
 * `size`; *sum = the row's sum of squares (fp32).  Replaces
 * toyinfer::rmsnorm_bf16<NUM_THREADS> (include/kernel_warpper.h:25-29;
 * src/decode.cu:67-142), one launch instead of memset + two kernels. */
int toyinfer_rmsnorm_bf16(const void* input, const void* weight, void* output, float* sum,
                          float rms_norm_eps, uint32_t size, void* stream);
/* The same per row of num_tokens rows; sum[t] per row.  Replaces
 * toyinfer::batch_rmsnorm_bf16<NUM_THREADS> (include/kernel_warpper.h:31-36;
 * src/prefill.cu:42-112). */
int toyinfer_batch_rmsnorm_bf16(const void* input, const void* weight, void* output, float* sum,
                                float rms_norm_eps, uint32_t num_tokens, uint32_t size,
                                void* stream);
/* hidden_state = bf16(hidden_state + residual).  Replaces
 * toyinfer::residual_add_bf16<NUM_THREADS> (include/kernel_warpper.h:12-15;
 * src/decode.cu:7-33). */
int toyinfer_residual_add_bf16(const void* residual, void* hidden_state, uint32_t size,
                               void* stream);
/* Over num_tokens * size values.  Replaces toyinfer::batch_residual_add_bf16
 * (include/kernel_warpper.h:17-21; src/prefill.cu:176-183). */
int toyinfer_batch_residual_add_bf16(const void* residual, void* hidden_state,
                                     uint32_t num_tokens, uint32_t size, void* stream);
/* intermedia = bf16(up * gate / (1 + exp(-gate))).  Replaces
 * toyinfer::swiglu_bf16x2<NUM_THREADS> (include/kernel_warpper.h:116-119;
 * src/decode.cu:746-775). */
int toyinfer_swiglu_bf16x2(const void* gate, const void* up, void* intermedia, uint32_t size,
                           void* stream);
/* Over num_tokens * size values.  Replaces toyinfer::batch_swiglu_bf16x2
 * (include/kernel_warpper.h:121-126; src/prefill.cu:397-405). */
int toyinfer_batch_swiglu_bf16x2(const void* gate, const void* up, void* intermedia,
                                 uint32_t num_tokens, uint32_t size, void* stream);
/* hidden_states[t] = embedding_table[token_ids[t]] (token_ids in device
 * memory); ids >= vocab_size give zero rows (vocab_size = 0xFFFFFFFF: no
 * check, as the reference).  Replaces toyinfer::gather_embedding_bf16
 * (include/kernel_warpper.h:71-77; src/prefill.cu:6-36). */
int toyinfer_gather_embedding_bf16(const void* embedding_table, const uint32_t* token_ids,
                                   void* hidden_states, uint32_t num_tokens,
                                   uint32_t hidden_size, uint32_t vocab_size, void* stream);
/* *out_index = the first index of the maximum of logits[0..n) under strict
 * '>' from -FLT_MAX (UINT32_MAX if none), on the device.  Extension: the
 * reference's greedy sampler does this on the host (src/sampler.cpp:71-82). */
int toyinfer_argmax_f32(const float* logits, uint32_t n, uint32_t* out_index, void* stream);

/* Device-side top-k / top-p sampling.  Replaces toyinfer::Sampler::sample
 * (include/sampler.h:10-16; src/sampler.cpp:18-67), which the reference runs
 * on the host over logits copied back each step (src/engine.cpp:183-190):
 * here logits[0..vocab) stay in device memory and *out_token is written on
 * the device.  Same rules: |temperature| < 1e-3 or top_k == 1 gives the first
 * index of the maximum (as toyinfer_argmax_f32); otherwise x = logit /
 * temperature, the top min(top_k, vocab) values of x, p = exp((x - max) /
 * temperature) normalised, sorted descending, cut after the first running
 * sum above top_p, and the first kept token whose running sum exceeds
 * *coin times the kept sum.  *coin (device memory, in [0, 1)) is the
 * uniform draw the reference takes from its time-seeded mt19937.  Ties at
 * the k-th value keep the lowest indices.  The workspace
 * (toyinfer_sample_workspace_bytes(), 256-byte aligned) must be zero before
 * its first use; every call leaves it so.  Calls sharing a workspace must be
 * stream-ordered.  Limits: vocab <= TOYINFER_SAMPLE_MAX_VOCAB, top_k <=
 * TOYINFER_SAMPLE_MAX_K unless greedy (TOYINFER_ERR_UNSUPPORTED beyond);
 * top_k == 0 (an assertion in the reference) and a negative or NaN
 * temperature give TOYINFER_ERR_INVALID_ARGUMENT. */
#define TOYINFER_SAMPLE_MAX_K 256u
#define TOYINFER_SAMPLE_MAX_VOCAB 262144u
size_t toyinfer_sample_workspace_bytes(void);
int toyinfer_sample_topk_topp_f32(const float* logits, uint32_t vocab, float temperature,
                                  uint32_t top_k, float top_p, const float* coin,
                                  uint32_t* out_token, void* workspace, size_t workspace_bytes,
                                  void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TOYINFER_ATTN_H_ */
