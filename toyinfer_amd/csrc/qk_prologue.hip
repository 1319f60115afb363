// Qwen3 pre-attention ops on gfx950: per-head RMSNorm, rotate-half RoPE and
// the inverse-frequency table.
//
// One row (token, head) of D values is handled by D/16 lanes; lane c owns the
// eight RoPE pairs (8c + k, 8c + k + D/2) and moves them with 16-byte loads
// and stores, so the rotation needs no data exchange and the sum of squares
// is an xor-shuffle reduction over D/16 lanes.  Norm and RoPE
// can run separately (the reference's batch_multi_rmsnorm_bf16 and
// batch_rope_bf16, src/decode.cu:144-199, src/prefill.cu:185-218) or fused
// in one pass with the intermediate rounded to bf16 exactly where the
// two-kernel sequence rounds it (src/transformer.cpp:380-391).
//
// Arithmetic follows the host references of the reference's tests
// (tests/multi_rmsnorm_test_common.h:56-76, tests/rope_test_common.h:48-65):
// inv = 1/sqrtf(sum/D + eps), y = (x*inv)*w, angle = (float)pos * inv_freq,
// accurate sincosf (or the same values from a precomputed rotary table),
// products and sums separately rounded.
#include <math.h>

#include "common.hpp"
#include "kernels.hpp"
#include "norm_rope.hpp"

namespace tiattn {
namespace {

__global__ void precompute_freq_kernel(float* inv_freq, int d, float theta) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < d / 2) inv_freq[i] = 1.0f / powf(theta, (float)(2 * i) / (float)d);
}

// Rotary table: table[t][i] = (cos, sin)((float)t * inv_freq[i]), the exact
// values the per-element RoPE computes, produced once per model.
__global__ void rope_table_kernel(float2* table, const float* __restrict__ inv_freq,
                                  uint32_t num_pos, int half) {
    const uint64_t e = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= (uint64_t)num_pos * half) return;
    const uint32_t t = (uint32_t)(e / half), i = (uint32_t)(e % half);
    float sn, cs;
    sincosf((float)t * inv_freq[i], &sn, &cs);
    table[e] = make_float2(cs, sn);
}

// Rows (token, head) of a token-major [tokens][nums_head][D] tensor; RoPE
// position = row / nums_head.
template <int D>
__global__ __launch_bounds__(256) void row_norm_rope_kernel(const uint16_t* in, uint16_t* out,
                                                            const uint16_t* __restrict__ weight,
                                                            const float* __restrict__ inv_freq,
                                                            const float2* __restrict__ table,
                                                            float eps, uint32_t rows,
                                                            uint32_t nums_head, int mode) {
    constexpr int LPR = D / 16;
    constexpr int RPB = 256 / LPR;  // rows per block
    const uint32_t row = blockIdx.x * RPB + threadIdx.x / LPR;
    if (row >= rows) return;  // the LPR lanes of a row exit together
    const int64_t off = (int64_t)row * D;
    norm_rope_row<D>(in + off, out + off, weight, inv_freq, table, eps, row / nums_head,
                     threadIdx.x % LPR, mode);
}

// Rows [0, T*hq) are Q's (q -> q_out), rows [T*hq, T*(hq + hkv)) K's
// (k -> k_out); each row normalised with its tensor's weight and rotated at
// position = its token index.
struct QkRows {
    const uint16_t* q;
    uint16_t* q_out;
    const uint16_t* q_weight;
    const uint16_t* k;
    uint16_t* k_out;
    const uint16_t* k_weight;
    const float2* table;
    float eps;
    uint32_t q_rows, rows, hq, hkv;
};

template <int D>
__global__ __launch_bounds__(256) void qk_rows_norm_rope_kernel(QkRows a) {
    constexpr int LPR = D / 16;
    constexpr int RPB = 256 / LPR;
    const uint32_t row = blockIdx.x * RPB + threadIdx.x / LPR;
    if (row >= a.rows) return;  // the LPR lanes of a row exit together
    const bool is_q = row < a.q_rows;
    const uint32_t r = is_q ? row : row - a.q_rows;
    const int64_t off = (int64_t)r * D;
    norm_rope_row<D>((is_q ? a.q : a.k) + off, (is_q ? a.q_out : a.k_out) + off,
                     is_q ? a.q_weight : a.k_weight, nullptr, a.table, a.eps,
                     r / (is_q ? a.hq : a.hkv), threadIdx.x % LPR, kRowNorm | kRowRope);
}

// One decoded token at position pos = min(*pos_d or pos_host, pos_cap - 1):
// rows [0, hq) are its query heads (q -> q_out, q_mode), rows
// [hq, hq + hkv) its key heads (k -> row pos of k_cache, k_mode), rows
// [hq + hkv, hq + 2*hkv) its value heads (v -> row pos of v_cache, copied).
// Caches are [positions][hkv][D].
struct TokenRows {
    const uint16_t* q;
    uint16_t* q_out;
    const uint16_t* q_weight;
    const uint16_t* k;
    uint16_t* k_cache;
    const uint16_t* k_weight;
    const uint16_t* v;
    uint16_t* v_cache;
    const float* inv_freq;
    const uint32_t* pos_d;
    uint32_t pos_host, pos_cap;
    float eps;
    uint32_t hq, hkv;
    int q_mode, k_mode;
};

template <int D>
__global__ __launch_bounds__(256) void token_rows_kernel(TokenRows a) {
    constexpr int LPR = D / 16;
    constexpr int RPB = 256 / LPR;
    const uint32_t row = blockIdx.x * RPB + threadIdx.x / LPR;
    if (row >= a.hq + 2 * a.hkv) return;
    uint32_t pos = a.pos_d ? *a.pos_d : a.pos_host;
    pos = min(pos, a.pos_cap - 1);
    const int c = threadIdx.x % LPR;
    if (row < a.hq) {
        norm_rope_row<D>(a.q + (int64_t)row * D, a.q_out + (int64_t)row * D, a.q_weight, a.inv_freq,
                         nullptr, a.eps, pos, c, a.q_mode);
    } else if (row < a.hq + a.hkv) {
        const uint32_t j = row - a.hq;
        norm_rope_row<D>(a.k + (int64_t)j * D, a.k_cache + ((int64_t)pos * a.hkv + j) * D,
                         a.k_weight, a.inv_freq, nullptr, a.eps, pos, c, a.k_mode);
    } else {
        const uint32_t j = row - a.hq - a.hkv;
        norm_rope_row<D>(a.v + (int64_t)j * D, a.v_cache + ((int64_t)pos * a.hkv + j) * D, nullptr,
                         nullptr, nullptr, 0.0f, pos, c, 0);
    }
}

// Reference write_kv_cache_bf16 (src/decode.cu:374-397): kv_dim values to
// cache + pos * kv_dim, bf16 pairs (kv_dim even), 16 bytes per lane where
// both ends are 16-byte aligned.
__global__ __launch_bounds__(256) void kv_row_copy_kernel(const uint16_t* __restrict__ src,
                                                          uint16_t* __restrict__ cache,
                                                          const uint32_t* __restrict__ pos_d,
                                                          uint32_t kv_dim, int vec16) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    uint16_t* dst = cache + (int64_t)(*pos_d) * kv_dim;
    if (vec16) {
        if (8 * i < kv_dim)
            *reinterpret_cast<uint4*>(dst + 8 * i) = *reinterpret_cast<const uint4*>(src + 8 * i);
    } else if (2 * i < kv_dim) {
        *reinterpret_cast<uint32_t*>(dst + 2 * i) = *reinterpret_cast<const uint32_t*>(src + 2 * i);
    }
}

}  // namespace

hipError_t launch_precompute_freq(float* inv_freq, int d, float theta, hipStream_t stream) {
    const int n = d / 2;
    hipLaunchKernelGGL(precompute_freq_kernel, dim3((n + 63) / 64), dim3(64), 0, stream, inv_freq,
                       d, theta);
    return hipGetLastError();
}

hipError_t launch_rope_table(float* table, const float* inv_freq, uint32_t num_pos, uint32_t d,
                             hipStream_t stream) {
    const uint64_t n = (uint64_t)num_pos * (d / 2);
    hipLaunchKernelGGL(rope_table_kernel, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, stream,
                       reinterpret_cast<float2*>(table), inv_freq, num_pos, (int)(d / 2));
    return hipGetLastError();
}

hipError_t launch_token_rows(const TokenRowsArgs& a, uint32_t d, hipStream_t stream) {
    TokenRows k{};
    k.q = a.q; k.q_out = a.q_out; k.q_weight = a.q_weight;
    k.k = a.k; k.k_cache = a.k_cache; k.k_weight = a.k_weight;
    k.v = a.v; k.v_cache = a.v_cache;
    k.inv_freq = a.inv_freq; k.pos_d = a.pos_d; k.pos_host = a.pos_host; k.pos_cap = a.pos_cap;
    k.eps = a.eps; k.hq = a.hq; k.hkv = a.hkv; k.q_mode = a.q_mode; k.k_mode = a.k_mode;
    const uint32_t rows = a.hq + 2 * a.hkv;
    const uint32_t rows_per_block = 256 / (d / 16);
    const dim3 grid((rows + rows_per_block - 1) / rows_per_block);
    if (d == 64)
        hipLaunchKernelGGL(token_rows_kernel<64>, grid, dim3(256), 0, stream, k);
    else
        hipLaunchKernelGGL(token_rows_kernel<128>, grid, dim3(256), 0, stream, k);
    return hipGetLastError();
}

hipError_t launch_kv_row_copy(const uint16_t* src, uint16_t* cache, const uint32_t* pos_d,
                              uint32_t kv_dim, hipStream_t stream) {
    const bool vec16 = kv_dim % 8 == 0 && reinterpret_cast<uintptr_t>(src) % 16 == 0 &&
                       reinterpret_cast<uintptr_t>(cache) % 16 == 0;
    const uint32_t lanes = vec16 ? kv_dim / 8 : kv_dim / 2;
    hipLaunchKernelGGL(kv_row_copy_kernel, dim3((lanes + 255) / 256), dim3(256), 0, stream, src,
                       cache, pos_d, kv_dim, vec16 ? 1 : 0);
    return hipGetLastError();
}

hipError_t launch_qk_norm_rope_rows(const uint16_t* q, uint16_t* q_out, const uint16_t* q_weight,
                                    const uint16_t* k, uint16_t* k_out, const uint16_t* k_weight,
                                    const float* table, float eps, uint32_t num_tokens,
                                    uint32_t hq, uint32_t hkv, uint32_t d, hipStream_t stream) {
    QkRows a;
    a.q = q;
    a.q_out = q_out;
    a.q_weight = q_weight;
    a.k = k;
    a.k_out = k_out;
    a.k_weight = k_weight;
    a.table = reinterpret_cast<const float2*>(table);
    a.eps = eps;
    a.hq = hq;
    a.hkv = hkv;
    a.q_rows = num_tokens * hq;
    a.rows = num_tokens * (hq + hkv);
    const uint32_t rows_per_block = 256 / (d / 16);
    const dim3 grid((a.rows + rows_per_block - 1) / rows_per_block);
    if (d == 64)
        hipLaunchKernelGGL(qk_rows_norm_rope_kernel<64>, grid, dim3(256), 0, stream, a);
    else
        hipLaunchKernelGGL(qk_rows_norm_rope_kernel<128>, grid, dim3(256), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_row_norm_rope(const uint16_t* in, uint16_t* out, const uint16_t* weight,
                                const float* inv_freq, const float* table, float eps,
                                uint32_t num_tokens, uint32_t nums_head, uint32_t d, int mode,
                                hipStream_t stream) {
    const uint32_t rows = num_tokens * nums_head;
    const uint32_t rows_per_block = 256 / (d / 16);
    const dim3 grid((rows + rows_per_block - 1) / rows_per_block);
    const float2* t2 = reinterpret_cast<const float2*>(table);
    if (d == 64)
        hipLaunchKernelGGL(row_norm_rope_kernel<64>, grid, dim3(256), 0, stream, in, out, weight,
                           inv_freq, t2, eps, rows, nums_head, mode);
    else
        hipLaunchKernelGGL(row_norm_rope_kernel<128>, grid, dim3(256), 0, stream, in, out, weight,
                           inv_freq, t2, eps, rows, nums_head, mode);
    return hipGetLastError();
}

}  // namespace tiattn
