// Per-head RMSNorm + rotate-half RoPE of one D-element row, shared by the
// pre-attention kernels and the engine's fused decode attention.
//
// One row is handled by LPR = D/16 lanes; lane c owns the eight RoPE pairs
// (8c + k, 8c + k + D/2), k < 8, so the rotation needs no data exchange and
// the sum of squares is an xor-shuffle reduction over the LPR lanes.  The
// work is split into a load phase (every global load of the row) and a
// compute phase, so that a caller can put other loads in flight between the
// two.
//
// Arithmetic follows the host references of the reference's tests
// (tests/multi_rmsnorm_test_common.h:56-76, tests/rope_test_common.h:48-65):
// inv = 1/sqrtf(sum/D + eps), y = (x*inv)*w rounded to bf16, angle =
// (float)pos * inv_freq, accurate sincosf (or the same values from a
// precomputed rotary table), products and sums separately rounded, the
// result rounded to bf16 (src/transformer.cpp:380-391 rounds the norm
// output before RoPE; so does this).
#pragma once

#include <math.h>

#include "common.hpp"
#include "kernels.hpp"

namespace tiattn {
namespace {

struct NormRopeIn {
    uint4 xr, xi;    // values 8c..8c+7 and D/2+8c..D/2+8c+7 of the row
    uint4 wr, wi;    // the norm weights at the same indices (kRowNorm)
    float4 tab[4];   // (cos, sin) pairs from a rotary table row
    float freq[8];   // inv_freq[8c .. 8c+7] (RoPE without a table)
};

// Load phase.  mode bit kRowNorm: RMSNorm with `weight`; bit kRowRope: RoPE
// at position t (angles from `table` row t when non-null, else from
// inv_freq); mode 0: a bit copy.
template <int D>
__device__ __forceinline__ NormRopeIn norm_rope_load(const uint16_t* in,
                                                     const uint16_t* __restrict__ weight,
                                                     const float* __restrict__ inv_freq,
                                                     const float2* __restrict__ table, uint32_t t,
                                                     int c, int mode) {
    constexpr int HALF = D / 2;
    NormRopeIn r;
    r.xr = ldg16(in + 8 * c);
    r.xi = ldg16(in + 8 * c + HALF);
    r.wr = r.wi = make_uint4(0, 0, 0, 0);
    if (mode & kRowNorm) {
        r.wr = ldg16(weight + 8 * c);
        r.wi = ldg16(weight + 8 * c + HALF);
    }
    if (mode & kRowRope) {
        if (table) {
            const float4* tp = reinterpret_cast<const float4*>(table + (uint64_t)t * HALF + 8 * c);
#pragma unroll
            for (int k = 0; k < 4; ++k) r.tab[k] = tp[k];
        } else {
#pragma unroll
            for (int k = 0; k < 8; ++k) r.freq[k] = inv_freq[8 * c + k];
        }
    }
    return r;
}

// Compute phase: the row's two output halves (lane c's 16-byte chunks at
// 8c and D/2 + 8c).  All LPR lanes of the row must call it together.
template <int D>
__device__ __forceinline__ void norm_rope_compute(const NormRopeIn& r, bool has_table, float eps,
                                                  uint32_t t, int mode, uint4* out_r,
                                                  uint4* out_i) {
#pragma clang fp contract(off)
    constexpr int LPR = D / 16;
    if (mode == 0) {
        *out_r = r.xr;
        *out_i = r.xi;
        return;
    }
    float re[8], im[8];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t a = word_of(r.xr, k), b = word_of(r.xi, k);
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
            const uint32_t a = word_of(r.wr, k), b = word_of(r.wi, k);
            re[2 * k] = bf16_lo(pack_bf16x2(re[2 * k] * inv * bf16_lo(a), 0.0f));
            re[2 * k + 1] = bf16_lo(pack_bf16x2(re[2 * k + 1] * inv * bf16_hi(a), 0.0f));
            im[2 * k] = bf16_lo(pack_bf16x2(im[2 * k] * inv * bf16_lo(b), 0.0f));
            im[2 * k + 1] = bf16_lo(pack_bf16x2(im[2 * k + 1] * inv * bf16_hi(b), 0.0f));
        }
    }
    if (mode & kRowRope) {
        float cv[8], sv[8];
        if (has_table) {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                cv[2 * k] = r.tab[k].x;
                sv[2 * k] = r.tab[k].y;
                cv[2 * k + 1] = r.tab[k].z;
                sv[2 * k + 1] = r.tab[k].w;
            }
        } else {
#pragma unroll
            for (int k = 0; k < 8; ++k) sincosf((float)t * r.freq[k], &sv[k], &cv[k]);
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const float a = cv[k] * re[k] - sv[k] * im[k];
            const float b = cv[k] * im[k] + sv[k] * re[k];
            re[k] = a;
            im[k] = b;
        }
    }
    out_r->x = pack_bf16x2(re[0], re[1]);
    out_r->y = pack_bf16x2(re[2], re[3]);
    out_r->z = pack_bf16x2(re[4], re[5]);
    out_r->w = pack_bf16x2(re[6], re[7]);
    out_i->x = pack_bf16x2(im[0], im[1]);
    out_i->y = pack_bf16x2(im[2], im[3]);
    out_i->z = pack_bf16x2(im[4], im[5]);
    out_i->w = pack_bf16x2(im[6], im[7]);
}

// Both phases, the result stored to `out` (which may alias `in`).
template <int D>
__device__ __forceinline__ void norm_rope_row(const uint16_t* in, uint16_t* out,
                                              const uint16_t* __restrict__ weight,
                                              const float* __restrict__ inv_freq,
                                              const float2* __restrict__ table, float eps,
                                              uint32_t t, int c, int mode) {
    const NormRopeIn r = norm_rope_load<D>(in, weight, inv_freq, table, t, c, mode);
    uint4 a, b;
    norm_rope_compute<D>(r, table != nullptr, eps, t, mode, &a, &b);
    *reinterpret_cast<uint4*>(out + 8 * c) = a;
    *reinterpret_cast<uint4*>(out + 8 * c + D / 2) = b;
}

}  // namespace
}  // namespace tiattn
