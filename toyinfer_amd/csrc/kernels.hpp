// Host-side launch interface between the C ABI (capi.hip) and the kernels.
// Launchers assume their arguments were validated by the caller.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace tiattn {

// ------------------------------------------------------------------ decode
//
// Split-K decode writes one partial (m, l, o[D]) per (sequence, q-head,
// split).  Where partials live is described by base pointers and strides so
// the same kernels serve the batched workspace layout and the reference
// contract's score/O_buffer/O buffers.
struct DecodePartials {
    float* ml;              // (m, l) pairs: ml + bh*ml_head + s*2
    float* o;               // o[D]:        o + bh*o_head + s*o_split
    int64_t ml_head;        // floats between consecutive (seq, q-head)
    int64_t o_head;
    int64_t o_split;
};

// Partials carved from a decode workspace of `heads` (sequence, q-head)
// pairs: the (m, l) pairs first, the o rows from the next 256-byte boundary.
inline DecodePartials decode_partials_in(void* workspace, size_t heads, uint32_t splits,
                                         uint32_t d) {
    char* ws = static_cast<char*>(workspace);
    const size_t ml_bytes = (heads * splits * 2 * sizeof(float) + 255) / 256 * 256;
    DecodePartials part{};
    part.ml = reinterpret_cast<float*>(ws);
    part.ml_head = 2 * (int64_t)splits;
    part.o = reinterpret_cast<float*>(ws + ml_bytes);
    part.o_head = (int64_t)splits * d;
    part.o_split = d;
    return part;
}

enum LenMode : int {
    kLenHost = 0,        // every sequence has length len_host
    kLenDevice = 1,      // lengths in len_dev[B]
    kLenDevicePos = 2,   // one device position: length = *len_dev + 1 (clamped to len_cap)
};

struct DecodeProblem {
    const uint16_t* q;   // [B][Hq][D]
    const uint16_t* k;
    const uint16_t* v;
    int64_t kv_stride;   // elements between sequences
    uint32_t batch, hq, hkv, d;
    int len_mode;
    const uint32_t* len_dev;
    uint32_t len_host;   // kLenHost: the length; otherwise unused
    uint32_t len_cap;    // upper bound for device lengths (grid sizing, clamping)
    uint32_t splits;
    // Prologue pass only: 0, or 128 when splits * 128 >= len_cap, so that
    // split s owns cache rows [128 s, 128 s + 128) whatever the length and
    // loads them before the device length arrives.
    uint32_t slice_rows;
};

// Split pass: grid (splits, Hkv * head groups, B).
hipError_t launch_decode_split(const DecodeProblem& p, const DecodePartials& part,
                               hipStream_t stream);
// The reference contract's split pass (B = 1, two or more splits, partials in
// the score rows: part.ml = score, ml_head = o_head = len_cap = msl): where
// the rows past the length have room, it also stores the raw scores and
// moves the partials behind them; launch_decode_finalize_compat follows it.
hipError_t launch_decode_split_compat(const DecodeProblem& p, const DecodePartials& part,
                                      hipStream_t stream);

// The engine's decode step (one sequence, the token at position L - 1 with
// L from len_dev) folds its pre-attention row work into the split pass:
// p.q holds the raw q projection, each workgroup applies q RMSNorm + RoPE to
// its heads, and the workgroup whose slice ends at L normalises and rotates
// the raw k row, writes k and v to cache row L - 1 and uses them in place of
// that row.  Results equal the prologue kernel followed by the split pass.
struct DecodePrologue {
    const uint16_t* q_w;    // q RMSNorm weight [D]
    const uint16_t* k_raw;  // the token's raw k projection [Hkv][D]
    const uint16_t* k_w;    // k RMSNorm weight [D]
    const uint16_t* v_raw;  // [Hkv][D]
    const float2* rope;     // the token position's rotary row [D/2] (cos, sin)
    uint16_t* k_cache;      // p.k and p.v, writable
    uint16_t* v_cache;
    float eps;
};
hipError_t launch_decode_split_prologue(const DecodeProblem& p, const DecodePartials& part,
                                        const DecodePrologue& pro, hipStream_t stream);
// Combine partials into o [B][Hq][D] bf16 (and o_f32 in fp32 when given);
// aligned8: every partial row starts 8-byte aligned.
hipError_t launch_decode_combine(const DecodeProblem& p, const DecodePartials& part, uint16_t* o,
                                 hipStream_t stream, float* o_f32 = nullptr,
                                 bool aligned8 = true);
// Reference-contract finaliser (B == 1): combine partials, write O_buffer
// (fp32), O (bf16) and score [Hq][msl] (probabilities, zeros past pos).
hipError_t launch_decode_finalize_compat(const DecodeProblem& p, const DecodePartials& part,
                                         float* score, uint32_t msl, float* o_buffer,
                                         uint16_t* o, hipStream_t stream);

uint32_t decode_default_splits(uint32_t batch, uint32_t hq, uint32_t hkv, uint32_t d,
                               uint32_t seq_len);
// Workgroups per KV head: up to 16 query heads share one workgroup.
uint32_t decode_head_groups(uint32_t group);
// Largest split count the combine kernels accept.
uint32_t decode_max_splits();

// ----------------------------------------------------------------- prefill
struct PrefillProblem {
    const uint16_t* q;   // [S][Hq][D] (raw when fused_q)
    const uint16_t* k;   // [S][Hkv][D] (already normalised/rotated when fused)
    const uint16_t* v;
    uint16_t* o;
    uint32_t s, hq, hkv, d;
    bool fused_q;
    const uint16_t* q_gamma;  // [D] (fused_q)
    const float* rope;        // [S][D/2] (cos, sin) pairs (fused_q)
    float eps;
    int variant;              // 0: pick by shape, 1: split over keys, 2: 128-row tiles,
                              // 3: split over keys, GQA head pairs per workgroup (1 for odd groups),
                              // 4: 128-row tiles, GQA head pairs per workgroup (2 for odd groups)
};
hipError_t launch_prefill(const PrefillProblem& p, hipStream_t stream);
// Whether launch_prefill takes the split-over-keys kernel for this problem.
bool prefill_uses_split(const PrefillProblem& p);

// ------------------------------------------------------ prologue kernels
hipError_t launch_precompute_freq(float* inv_freq, int d, float theta, hipStream_t stream);
// mode bit 1: RMSNorm with weight; bit 2: RoPE at position = row / nums_head.
enum RowOpMode : int { kRowNorm = 1, kRowRope = 2 };
// RoPE angles come from `table` ([tokens][D/2] (cos, sin)) when non-null,
// else from sincosf(token * inv_freq[i]).
hipError_t launch_row_norm_rope(const uint16_t* in, uint16_t* out, const uint16_t* weight,
                                const float* inv_freq, const float* table, float eps,
                                uint32_t num_tokens, uint32_t nums_head, uint32_t d, int mode,
                                hipStream_t stream);
// Per-head RMSNorm + RoPE (rotary table rows) of Q [T][hq][D] and K
// [T][hkv][D] in one launch: q -> q_out (may alias), k -> k_out (may alias).
hipError_t launch_qk_norm_rope_rows(const uint16_t* q, uint16_t* q_out, const uint16_t* q_weight,
                                    const uint16_t* k, uint16_t* k_out, const uint16_t* k_weight,
                                    const float* table, float eps, uint32_t num_tokens,
                                    uint32_t hq, uint32_t hkv, uint32_t d, hipStream_t stream);
hipError_t launch_rope_table(float* table, const float* inv_freq, uint32_t num_pos, uint32_t d,
                             hipStream_t stream);
// One decoded token's rows at a single position (device pos_d, else
// pos_host; clamped below pos_cap): query heads transformed in place or to
// q_out, key heads transformed into row pos of k_cache, value heads copied
// into row pos of v_cache.  hq or hkv may be 0.
struct TokenRowsArgs {
    const uint16_t* q = nullptr;
    uint16_t* q_out = nullptr;
    const uint16_t* q_weight = nullptr;
    const uint16_t* k = nullptr;
    uint16_t* k_cache = nullptr;
    const uint16_t* k_weight = nullptr;
    const uint16_t* v = nullptr;
    uint16_t* v_cache = nullptr;
    const float* inv_freq = nullptr;
    const uint32_t* pos_d = nullptr;
    uint32_t pos_host = 0, pos_cap = 1;
    float eps = 0.0f;
    uint32_t hq = 0, hkv = 0;
    int q_mode = 0, k_mode = 0;
};
hipError_t launch_token_rows(const TokenRowsArgs& a, uint32_t d, hipStream_t stream);
// kv_dim (even) values from src to cache + (*pos_d) * kv_dim.
hipError_t launch_kv_row_copy(const uint16_t* src, uint16_t* cache, const uint32_t* pos_d,
                              uint32_t kv_dim, hipStream_t stream);

// ------------------------------------------------------------ projections
// y[t][m] = sum_n W[m][n] x[t][n]; W [M][N], x [T][N], y [T][M], fp32
// accumulation.  Batches above kGemvMaxTokens tokens with N % 64 == 0 and
// 16-byte aligned W and x run on the MFMA GEMM, the rest on the GEMV.
constexpr uint32_t kGemvMaxTokens = 4;
constexpr uint32_t kProjMaxN = 1u << 22;  // keeps every byte offset in 32 bits
hipError_t launch_gemv_bf16(const uint16_t* W, const uint16_t* x, uint16_t* y, uint32_t M,
                            uint32_t N, hipStream_t stream);
hipError_t launch_gemv_f32(const uint16_t* W, const uint16_t* x, float* y, uint32_t M, uint32_t N,
                           hipStream_t stream);
hipError_t launch_batch_proj_bf16(const uint16_t* W, const uint16_t* x, uint16_t* y, uint32_t T,
                                  uint32_t M, uint32_t N, hipStream_t stream);
bool proj_uses_gemm(uint32_t T, uint32_t N, const void* W, const void* x);
// MFMA GEMM over up to three weight segments sharing the input x [T][N]:
// y[s][t][m] = sum_n w[s][m][n] x[t][n], y[s] being [T][rows[s]]; with
// `residual`, y[s][t][m] = bf16(y[s][t][m] + bf16(sum)).  Requires T > 0,
// N % 64 == 0 and 16-byte aligned x and weights (proj_uses_gemm).
struct GemmArgs {
    const uint16_t* x = nullptr;
    uint32_t T = 0, N = 0;
    int nseg = 1;
    const uint16_t* w[3] = {nullptr, nullptr, nullptr};
    uint16_t* y[3] = {nullptr, nullptr, nullptr};
    uint32_t rows[3] = {0, 0, 0};
    bool residual = false;
    // SwiGLU epilogue: nseg = 2, w[0] gate and w[1] up (rows[0] == rows[1]),
    // y[0][t][m] = bf16(bf16(up) * silu(bf16(gate))).
    bool swiglu = false;
};
hipError_t launch_gemm(const GemmArgs& g, hipStream_t stream);

// ------------------------------------------------- fused decode projections
// One token: y = W * f(x) with f = RMSNorm(x; norm_w, eps) when norm_w is set,
// over up to three stacked weight segments (rows[s] x n each), and an
// epilogue: kDgPlain y[s][m] = bf16(acc); kDgResidual y[s][m] =
// bf16(y[s][m] + bf16(acc)); kDgSwiglu (one segment, w[0] gate, w[1] up)
// y[0][m] = bf16(bf16(up) * silu(bf16(gate))).
// n % 8 == 0, n <= kDecodeGemvMaxN, 16-byte aligned x, norm_w and weights.
enum DecodeGemvEpi : int { kDgPlain = 0, kDgResidual = 1, kDgSwiglu = 2 };
constexpr uint32_t kDecodeGemvMaxN = 16384;
struct DecodeGemvArgs {
    const uint16_t* x = nullptr;
    const uint16_t* norm_w = nullptr;
    float eps = 0.0f;
    uint32_t n = 0;
    int nseg = 1;
    const uint16_t* w[3] = {nullptr, nullptr, nullptr};
    uint16_t* y[3] = {nullptr, nullptr, nullptr};
    uint32_t rows[3] = {0, 0, 0};
    int epi = kDgPlain;
};
hipError_t launch_decode_gemv(const DecodeGemvArgs& a, hipStream_t stream);
// Argmax over many workgroups with a last-arriving finaliser (same result and
// out/pos_d behaviour as launch_argmax); key and ticket (device, zero before
// the first launch) are left zero after every launch.
hipError_t launch_argmax_wide(const float* logits, uint32_t n, uint32_t* out, uint32_t* pos_d,
                              uint32_t out_cap, uint64_t* key, uint32_t* ticket,
                              hipStream_t stream);

// Top-k / top-p sampling (sampler.hip).  `workspace` holds
// sample_workspace_bytes(), zero before the first launch (each launch leaves
// it so).  coin: device pointer to u in [0, 1), or null to hash (seed, *pos).
// pos: null writes out[0]; else out[*pos + 1] (if below out_cap), *pos += 1.
constexpr uint32_t kSampleMaxK = 256, kSampleMaxVocab = 262144;
struct SampleArgs {
    const float* logits = nullptr;
    uint32_t n = 0;
    float temperature = 0.0f;
    uint32_t k = 1;
    float top_p = 1.0f;
    bool greedy = true;  // |temperature| < 1e-3 or top_k == 1: first index of the maximum
    const float* coin = nullptr;
    uint64_t seed = 0;
    uint32_t* out = nullptr;
    uint32_t* pos = nullptr;
    uint32_t out_cap = 0;
    void* workspace = nullptr;
};
size_t sample_workspace_bytes();
// Checks the parameters as the reference's sampler reads them and fills n, k,
// temperature, top_p and greedy; returns a TOYINFER_* status.
int sample_config(uint32_t vocab, float temperature, uint32_t top_k, float top_p, SampleArgs& a);
hipError_t launch_sample(const SampleArgs& a, hipStream_t stream);

// ------------------------------------------------------------ model ops
// rows x size RMSNorm (size even); sum_out[row] = sum of squares (nullable).
hipError_t launch_rmsnorm_rows(const uint16_t* x, const uint16_t* w, uint16_t* y, float* sum_out,
                               float eps, uint32_t rows, uint32_t size, hipStream_t stream);
// hidden = bf16(hidden + residual) over n (even) values.
hipError_t launch_residual_add(const uint16_t* residual, uint16_t* hidden, size_t n,
                               hipStream_t stream);
// out = bf16(up * silu(gate)) over n (even) values.
hipError_t launch_swiglu(const uint16_t* gate, const uint16_t* up, uint16_t* out, size_t n,
                         hipStream_t stream);
// out[t] = table[ids[t]] for rows of `size` (even) values; ids >= vocab give zeros.
hipError_t launch_gather_rows(const uint16_t* table, const uint32_t* ids, uint16_t* out,
                              uint32_t tokens, uint32_t size, uint32_t vocab, hipStream_t stream);
// First maximum of logits[0..n) -> out[0]; with pos_d, -> out[*pos_d + 1]
// (if below out_cap) and *pos_d += 1.
hipError_t launch_argmax(const float* logits, uint32_t n, uint32_t* out, uint32_t* pos_d,
                         uint32_t out_cap, hipStream_t stream);
// *p = value, as a one-lane kernel (stream-ordered, capturable).
hipError_t launch_set_u32(uint32_t* p, uint32_t value, hipStream_t stream);
// hidden = table[ids[p]], seq_len_d[0] = p + 1, p = min(*pos_d, cap - 1);
// with rope_row: rope_row[0..rope_floats) = rope_table row p.
hipError_t launch_decode_step_setup(const uint16_t* table, const uint32_t* ids,
                                    const uint32_t* pos_d, uint16_t* hidden, uint32_t* seq_len_d,
                                    uint32_t size, uint32_t vocab, uint32_t cap,
                                    hipStream_t stream, const float* rope_table = nullptr,
                                    float* rope_row = nullptr, uint32_t rope_floats = 0);

}  // namespace tiattn
