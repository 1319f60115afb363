// Qwen3 pre-attention ops on gfx950: per-head RMSNorm, rotate-half RoPE and
// the inverse-frequency table.
//
// One row (token, head) of D values is handled by D/2 lanes; lane i owns the
// RoPE pair (i, i + D/2), so the rotation needs no data exchange and the
// sum of squares is one xor-shuffle reduction over D/2 lanes.  Norm and RoPE
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

template <int D>
__global__ __launch_bounds__(256) void row_norm_rope_kernel(const uint16_t* in, uint16_t* out,
                                                            const uint16_t* __restrict__ weight,
                                                            const float* __restrict__ inv_freq,
                                                            const float2* __restrict__ table,
                                                            float eps, uint32_t rows,
                                                            uint32_t nums_head, int mode) {
#pragma clang fp contract(off)
    constexpr int LPR = D / 2;  // lanes per row
    const uint32_t row = blockIdx.x * (256 / LPR) + threadIdx.x / LPR;
    const int i = threadIdx.x % LPR;
    if (row >= rows) return;  // whole rows exit together
    const int64_t off = (int64_t)row * D;
    float re = bf16_to_f32(in[off + i]);
    float im = bf16_to_f32(in[off + i + LPR]);
    if (mode & kRowNorm) {
        float ss = re * re + im * im;
#pragma unroll
        for (int m = LPR / 2; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, 64);
        const float inv = 1.0f / sqrtf(ss / (float)D + eps);
        re = bf16_lo(pack_bf16x2(re * inv * bf16_to_f32(weight[i]), 0.0f));
        im = bf16_lo(pack_bf16x2(im * inv * bf16_to_f32(weight[i + LPR]), 0.0f));
    }
    if (mode & kRowRope) {
        const uint32_t t = row / nums_head;
        float sn, cs;
        if (table) {
            const float2 c2 = table[(uint64_t)t * LPR + i];
            cs = c2.x;
            sn = c2.y;
        } else {
            sincosf((float)t * inv_freq[i], &sn, &cs);
        }
        const float a = cs * re - sn * im;
        const float b = cs * im + sn * re;
        re = a;
        im = b;
    }
    out[off + i] = f32_to_bf16(re);
    out[off + i + LPR] = f32_to_bf16(im);
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

hipError_t launch_row_norm_rope(const uint16_t* in, uint16_t* out, const uint16_t* weight,
                                const float* inv_freq, const float* table, float eps,
                                uint32_t num_tokens, uint32_t nums_head, uint32_t d, int mode,
                                hipStream_t stream) {
    const uint32_t rows = num_tokens * nums_head;
    const uint32_t rows_per_block = 256 / (d / 2);
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
