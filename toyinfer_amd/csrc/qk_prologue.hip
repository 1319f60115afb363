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
    constexpr int HALF = D / 2;
    constexpr int LPR = HALF / 8;     // lanes per row; a lane owns the 8 pairs (8c + k, 8c + k + D/2)
    constexpr int RPB = 256 / LPR;    // rows per block
    const uint32_t row = blockIdx.x * RPB + threadIdx.x / LPR;
    const int c = threadIdx.x % LPR;
    if (row >= rows) return;  // the LPR lanes of a row exit together
    const int64_t off = (int64_t)row * D + 8 * c;
    // Every load goes out before the first use.
    const uint4 xr = ldg16(in + off), xi = ldg16(in + off + HALF);
    uint4 wr = make_uint4(0, 0, 0, 0), wi = wr;
    if (mode & kRowNorm) {
        wr = ldg16(weight + 8 * c);
        wi = ldg16(weight + 8 * c + HALF);
    }
    float4 cs[4];
    const uint32_t t = row / nums_head;
    if ((mode & kRowRope) && table) {
        const float4* tp = reinterpret_cast<const float4*>(table + (uint64_t)t * HALF + 8 * c);
#pragma unroll
        for (int k = 0; k < 4; ++k) cs[k] = tp[k];
    }
    float re[8], im[8];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t a = word_of(xr, k), b = word_of(xi, k);
        re[2 * k] = bf16_lo(a);
        re[2 * k + 1] = bf16_hi(a);
        im[2 * k] = bf16_lo(b);
        im[2 * k + 1] = bf16_hi(b);
    }
    if (mode & kRowNorm) {
        float ss = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; ++k) ss += re[k] * re[k];
#pragma unroll
        for (int k = 0; k < 8; ++k) ss += im[k] * im[k];
#pragma unroll
        for (int m = LPR / 2; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, LPR);
        const float inv = 1.0f / sqrtf(ss / (float)D + eps);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t a = word_of(wr, k), b = word_of(wi, k);
            re[2 * k] = bf16_lo(pack_bf16x2(re[2 * k] * inv * bf16_lo(a), 0.0f));
            re[2 * k + 1] = bf16_lo(pack_bf16x2(re[2 * k + 1] * inv * bf16_hi(a), 0.0f));
            im[2 * k] = bf16_lo(pack_bf16x2(im[2 * k] * inv * bf16_lo(b), 0.0f));
            im[2 * k + 1] = bf16_lo(pack_bf16x2(im[2 * k + 1] * inv * bf16_hi(b), 0.0f));
        }
    }
    if (mode & kRowRope) {
        float cv[8], sv[8];
        if (table) {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                cv[2 * k] = cs[k].x;
                sv[2 * k] = cs[k].y;
                cv[2 * k + 1] = cs[k].z;
                sv[2 * k + 1] = cs[k].w;
            }
        } else {
#pragma unroll
            for (int k = 0; k < 8; ++k) sincosf((float)t * inv_freq[8 * c + k], &sv[k], &cv[k]);
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const float a = cv[k] * re[k] - sv[k] * im[k];
            const float b = cv[k] * im[k] + sv[k] * re[k];
            re[k] = a;
            im[k] = b;
        }
    }
    uint4 orr, oi;
    orr.x = pack_bf16x2(re[0], re[1]);
    orr.y = pack_bf16x2(re[2], re[3]);
    orr.z = pack_bf16x2(re[4], re[5]);
    orr.w = pack_bf16x2(re[6], re[7]);
    oi.x = pack_bf16x2(im[0], im[1]);
    oi.y = pack_bf16x2(im[2], im[3]);
    oi.z = pack_bf16x2(im[4], im[5]);
    oi.w = pack_bf16x2(im[6], im[7]);
    *reinterpret_cast<uint4*>(out + off) = orr;
    *reinterpret_cast<uint4*>(out + off + HALF) = oi;
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
