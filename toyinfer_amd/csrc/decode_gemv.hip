// One-token projections of the decode step with their neighbours fused in,
// so that a decoder layer is a handful of launches:
//   RMSNorm -> q/k/v projections        (one launch, three weight segments)
//   o projection -> residual add        (epilogue)
//   RMSNorm -> gate/up -> SwiGLU        (one launch, paired rows)
//   down projection -> residual add     (epilogue)
// Rounding points are the unfused sequence's: the normalised input is
// rounded to bf16 before the products, every projection output is rounded to
// bf16 before the residual add or SwiGLU, which round again.
//
// A workgroup (256 lanes) stages the input vector in LDS (normalised there
// when asked: fp32 sum of squares, rsqrt(sum/N + eps), bf16(x * inv * w)),
// then owns RB output rows (2 RB for gate/up) and streams 16-byte chunks of
// them as the plain GEMV does, reading the input chunks from LDS.  Rows past
// a segment's end read zeros through the buffer range and are not stored.
#include "common.hpp"
#include "kernels.hpp"

namespace tiattn {
namespace {

constexpr int kDgThreads = 256;
constexpr uint32_t kDgOob = 0xF0000000u;

__device__ __forceinline__ float dg_block_sum(float x, float* s_red) {
    x = wave_sum(x);
    if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = x;
    __syncthreads();
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < kDgThreads / 64; ++w) s += s_red[w];
    return s;
}

__device__ __forceinline__ float dot8(uint4 w, uint4 x, float acc) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
        acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, word_of(w, i)),
                                              __builtin_bit_cast(bf16x2_t, word_of(x, i)), acc,
                                              false);
    return acc;
}

__device__ __forceinline__ float bf16_round(float v) { return bf16_to_f32(f32_to_bf16(v)); }

template <int RB, bool NORM, int EPI>
__global__ __launch_bounds__(kDgThreads) void decode_gemv_kernel(DecodeGemvArgs a) {
    constexpr int NR = EPI == kDgSwiglu ? 2 * RB : RB;
    extern __shared__ __align__(16) uint16_t s_x[];  // n values (dynamic: 2 n bytes)
    __shared__ float s_red[kDgThreads / 64];
    __shared__ float s_acc[kDgThreads / 64][NR];
    const uint32_t N = a.n, nchunk = N / 8;

    // Which segment and rows this workgroup owns.
    // (each segment spans whole groups of RB rows).
    uint32_t r0 = blockIdx.x * RB;
    int seg = 0;
    while (seg + 1 < a.nseg && r0 >= (a.rows[seg] + RB - 1) / RB * RB) {
        r0 -= (a.rows[seg] + RB - 1) / RB * RB;
        ++seg;
    }
    const uint32_t nrows = min((uint32_t)RB, a.rows[seg] - r0);
    const uint32_t row_bytes = 2 * N;

    // The weight rows do not depend on the input: the first trip's chunks
    // are requested before the input is staged (and normalised).
    __amdgpu_buffer_rsrc_t rw[EPI == kDgSwiglu ? 2 : 1];
    rw[0] = make_rsrc(a.w[seg] + (size_t)r0 * N, nrows * row_bytes);
    if constexpr (EPI == kDgSwiglu) rw[1] = make_rsrc(a.w[1] + (size_t)r0 * N, nrows * row_bytes);
    uint4 wv[2][NR];
    auto load_trip = [&](uint32_t off0, uint32_t off1) __attribute__((always_inline)) {
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            wv[0][r] = buf_load16(rw[r / RB], (r % RB) * row_bytes + off0);
            wv[1][r] = buf_load16(rw[r / RB], (r % RB) * row_bytes + off1);
        }
    };
    {
        const uint32_t c = threadIdx.x, c2 = c + kDgThreads;
        load_trip(c < nchunk ? c * 16 : kDgOob, c2 < nchunk ? c2 * 16 : kDgOob);
    }

    // Stage the input (normalised if asked) in LDS.
    if constexpr (NORM) {
        float ss = 0.0f;
        for (uint32_t c = threadIdx.x; c < nchunk; c += kDgThreads) {
            const uint4 v = ldg16(a.x + 8 * c);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t wd = word_of(v, i);
                ss = fmaf(bf16_lo(wd), bf16_lo(wd), ss);
                ss = fmaf(bf16_hi(wd), bf16_hi(wd), ss);
            }
        }
        const float inv = rsqrtf(fmaf(dg_block_sum(ss, s_red), 1.0f / (float)N, a.eps));
        for (uint32_t c = threadIdx.x; c < nchunk; c += kDgThreads) {
            const uint4 v = ldg16(a.x + 8 * c), g = ldg16(a.norm_w + 8 * c);
            uint4 o;
            uint32_t* ow = reinterpret_cast<uint32_t*>(&o);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t p = word_of(v, i), q = word_of(g, i);
                ow[i] = pack_bf16x2(bf16_lo(p) * inv * bf16_lo(q), bf16_hi(p) * inv * bf16_hi(q));
            }
            *reinterpret_cast<uint4*>(s_x + 8 * c) = o;
        }
    } else {
        for (uint32_t c = threadIdx.x; c < nchunk; c += kDgThreads)
            *reinterpret_cast<uint4*>(s_x + 8 * c) = ldg16(a.x + 8 * c);
    }
    __syncthreads();

    float acc[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) acc[r] = 0.0f;
    for (uint32_t c = threadIdx.x; c < nchunk; c += 2 * kDgThreads) {
        const uint32_t c2 = c + kDgThreads;
        const uint4 x0 = *reinterpret_cast<const uint4*>(s_x + 8 * c);
        const uint4 x1 = c2 < nchunk ? *reinterpret_cast<const uint4*>(s_x + 8 * c2) : uint4{0, 0, 0, 0};
#pragma unroll
        for (int r = 0; r < NR; ++r) acc[r] = dot8(wv[1][r], x1, dot8(wv[0][r], x0, acc[r]));
        // The next trip's rows.
        const uint32_t n0 = c + 2 * kDgThreads, n1 = n0 + kDgThreads;
        if (n0 < nchunk) load_trip(n0 * 16, n1 < nchunk ? n1 * 16 : kDgOob);
    }

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        const float s = wave_sum(acc[r]);
        if (lane == 0) s_acc[wave][r] = s;
    }
    __syncthreads();
    if (threadIdx.x < RB && threadIdx.x < nrows) {
        const int r = threadIdx.x;
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < kDgThreads / 64; ++w) v += s_acc[w][r];
        const uint32_t m = r0 + r;
        if constexpr (EPI == kDgPlain) {
            a.y[seg][m] = f32_to_bf16(v);
        } else if constexpr (EPI == kDgResidual) {
            a.y[seg][m] = f32_to_bf16(bf16_to_f32(a.y[seg][m]) + bf16_round(v));
        } else {
            float u = 0.0f;
#pragma unroll
            for (int w = 0; w < kDgThreads / 64; ++w) u += s_acc[w][RB + r];
            const float g = bf16_round(v), up = bf16_round(u);
            a.y[0][m] = f32_to_bf16(up * (g * (1.0f / (1.0f + expf(-g)))));
        }
    }
}

template <int RB, bool NORM, int EPI>
hipError_t dg_launch(const DecodeGemvArgs& a, uint32_t total_groups, hipStream_t stream) {
    decode_gemv_kernel<RB, NORM, EPI><<<total_groups, kDgThreads, 2 * a.n, stream>>>(a);
    return hipGetLastError();
}

template <bool NORM, int EPI>
hipError_t dg_rows(const DecodeGemvArgs& a, hipStream_t stream) {
    uint32_t total = 0;
    for (int s = 0; s < a.nseg; ++s) total += a.rows[s];
    // Rows per workgroup: about two workgroups per CU at least.
    const int rb = total >= 4096 ? 8 : total >= 2048 ? 4 : 2;
    auto groups = [&](uint32_t r) {
        uint32_t g = 0;
        for (int s = 0; s < a.nseg; ++s) g += (a.rows[s] + r - 1) / r;
        return g;
    };
    if (rb == 8) return dg_launch<8, NORM, EPI>(a, groups(8), stream);
    if (rb == 4) return dg_launch<4, NORM, EPI>(a, groups(4), stream);
    return dg_launch<2, NORM, EPI>(a, groups(2), stream);
}

// Two-stage-in-one argmax: each workgroup reduces a slice to a 64-bit key
// (orderable value bits above the complemented index, so the larger value
// and then the smaller index win) and folds it into *key with an atomic max;
// the last workgroup to arrive (ticket) writes the index, advances the
// position as the one-workgroup argmax does, and rearms key and ticket for
// the next launch.
constexpr int kAmBlocks = 256, kAmThreads = 256;

__device__ __forceinline__ uint64_t am_key(float v, uint32_t i) {
    // Values not above -FLT_MAX (and NaN) never win: key 0.
    if (!(v > -3.402823466e38f)) return 0;
    const uint32_t b = __float_as_uint(v);
    const uint32_t ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((uint64_t)ord << 32) | (uint64_t)(0xffffffffu - i);
}

__global__ __launch_bounds__(kAmThreads) void argmax_wide_kernel(const float* __restrict__ logits,
                                                                 uint32_t n, uint32_t* out,
                                                                 uint32_t* pos_d, uint32_t out_cap,
                                                                 uint64_t* key, uint32_t* ticket) {
    __shared__ uint64_t s_k[kAmThreads / 64];
    __shared__ bool s_last;
    uint64_t best = 0;
    for (uint32_t i = blockIdx.x * kAmThreads + threadIdx.x; i < n; i += kAmBlocks * kAmThreads) {
        const uint64_t k = am_key(logits[i], i);
        best = k > best ? k : best;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const uint64_t o = __shfl_xor(best, off);
        best = o > best ? o : best;
    }
    if ((threadIdx.x & 63) == 0) s_k[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < kAmThreads / 64; ++w) best = s_k[w] > best ? s_k[w] : best;
        __hip_atomic_fetch_max(key, best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __threadfence();
        s_last = atomicAdd(ticket, 1u) == kAmBlocks - 1;
    }
    __syncthreads();
    if (s_last && threadIdx.x == 0) {
        __threadfence();
        const uint64_t k = __hip_atomic_exchange(key, (uint64_t)0, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
        *ticket = 0;
        const uint32_t idx = k ? 0xffffffffu - (uint32_t)(k & 0xffffffffu) : 0xffffffffu;
        if (pos_d) {
            const uint32_t p = *pos_d;
            if (p + 1 < out_cap) out[p + 1] = idx;
            *pos_d = p + 1;
        } else {
            out[0] = idx;
        }
    }
}

}  // namespace

hipError_t launch_decode_gemv(const DecodeGemvArgs& a, hipStream_t stream) {
    const bool norm = a.norm_w != nullptr;
    switch (a.epi) {
        case kDgPlain: return norm ? dg_rows<true, kDgPlain>(a, stream) : dg_rows<false, kDgPlain>(a, stream);
        case kDgResidual:
            return norm ? dg_rows<true, kDgResidual>(a, stream) : dg_rows<false, kDgResidual>(a, stream);
        default: return norm ? dg_rows<true, kDgSwiglu>(a, stream) : dg_rows<false, kDgSwiglu>(a, stream);
    }
}

hipError_t launch_argmax_wide(const float* logits, uint32_t n, uint32_t* out, uint32_t* pos_d,
                              uint32_t out_cap, uint64_t* key, uint32_t* ticket,
                              hipStream_t stream) {
    argmax_wide_kernel<<<kAmBlocks, kAmThreads, 0, stream>>>(logits, n, out, pos_d, out_cap, key,
                                                             ticket);
    return hipGetLastError();
}

}  // namespace tiattn
