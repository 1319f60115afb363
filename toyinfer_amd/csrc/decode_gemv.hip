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
    const uint32_t spans[3] = {(a.rows[0] + RB - 1) / RB * RB, (a.rows[1] + RB - 1) / RB * RB,
                               (a.rows[2] + RB - 1) / RB * RB};
    const int seg = segment_of(spans, a.nseg, r0);
    const uint32_t seg_rows = pick3(a.rows, seg);
    const uint16_t* const seg_w = pick3(a.w, seg);
    uint16_t* const seg_y = pick3(a.y, seg);
    const uint32_t nrows = min((uint32_t)RB, seg_rows - r0);
    const uint32_t row_bytes = 2 * N;

    // The weight rows do not depend on the input: the first trip's chunks
    // are requested before the input is staged (and normalised).
    __amdgpu_buffer_rsrc_t rw[EPI == kDgSwiglu ? 2 : 1];
    rw[0] = make_rsrc(seg_w + (size_t)r0 * N, nrows * row_bytes);
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

    // Stage the input (normalised if asked) in LDS.  With up to four chunks
    // per lane (N <= 8192) the input and norm weights are read from global
    // memory once, the raw chunks parked in LDS for the normalising pass.
    if (NORM && nchunk <= 4 * kDgThreads) {
        constexpr int MC = 4;
        uint4 gv[MC];
        float ss = 0.0f;
#pragma unroll
        for (int k = 0; k < MC; ++k) {
            const uint32_t c = threadIdx.x + k * kDgThreads;
            if (c < nchunk) {
                const uint4 v = ldg16(a.x + 8 * c);
                gv[k] = ldg16(a.norm_w + 8 * c);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t wd = word_of(v, i);
                    ss = fmaf(bf16_lo(wd), bf16_lo(wd), ss);
                    ss = fmaf(bf16_hi(wd), bf16_hi(wd), ss);
                }
                *reinterpret_cast<uint4*>(s_x + 8 * c) = v;
            }
        }
        const float inv = rsqrtf(fmaf(dg_block_sum(ss, s_red), 1.0f / (float)N, a.eps));
#pragma unroll
        for (int k = 0; k < MC; ++k) {
            const uint32_t c = threadIdx.x + k * kDgThreads;
            if (c < nchunk) {
                const uint4 v = *reinterpret_cast<const uint4*>(s_x + 8 * c), g = gv[k];
                uint4 o;
                uint32_t* ow = reinterpret_cast<uint32_t*>(&o);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t p = word_of(v, i), q = word_of(g, i);
                    ow[i] = pack_bf16x2(bf16_lo(p) * inv * bf16_lo(q), bf16_hi(p) * inv * bf16_hi(q));
                }
                *reinterpret_cast<uint4*>(s_x + 8 * c) = o;
            }
        }
    } else if constexpr (NORM) {
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
            seg_y[m] = f32_to_bf16(v);
        } else if constexpr (EPI == kDgResidual) {
            seg_y[m] = f32_to_bf16(bf16_to_f32(seg_y[m]) + bf16_round(v));
        } else {
            float u = 0.0f;
#pragma unroll
            for (int w = 0; w < kDgThreads / 64; ++w) u += s_acc[w][RB + r];
            const float g = bf16_round(v), up = bf16_round(u);
            a.y[0][m] = f32_to_bf16(up * (g * (1.0f / (1.0f + expf(-g)))));
        }
    }
}

// Wave-autonomous form for the harness's layer sizes (N <= 4096): 4-wave
// workgroups, each wave owning RPW output rows (RPW gate and RPW up rows for
// SwiGLU) whole.  A lane loads chunks l, l+64, ... of the input and of each
// of its rows in one round (NCH = ceil(N/512) chunks per row), so a wave
// needs no LDS and no barrier: the RMSNorm statistics and every row's dot
// product are wave sums.  A one-token projection is latency-bound, so the
// grid aims at about 2048 waves (8 per CU) with every load of a wave issued
// before its first use.  Measured on MI355X for Qwen3-0.6B's shapes
// (4-12 MB of weights): 3.4-4.9 us per projection, against 4-6 us for the
// block-cooperative kernel below; 16-wave workgroups on 32-48 CUs stream the
// same matrices from HBM at under half the rate (8.5 us for 4 MB).  The
// residual row is read at the start, with the weights; the weight rows carry
// the non-temporal hint (read once per step: 0.729 -> 0.666 ms per
// Qwen3-0.6B decode step together with the lm-head's).
constexpr int kDwWaves = 4;

template <int RPW, int NCH, bool NORM, int EPI>
__global__ __launch_bounds__(64 * kDwWaves) void decode_gemv_wave_kernel(DecodeGemvArgs a) {
    constexpr int NR = EPI == kDgSwiglu ? 2 * RPW : RPW;
    const int lane = threadIdx.x & 63;
    const uint32_t wave =
        __builtin_amdgcn_readfirstlane(blockIdx.x * kDwWaves + (threadIdx.x >> 6));
    const uint32_t N = a.n;
    uint32_t r0 = wave * RPW;
    const uint32_t spans[3] = {(a.rows[0] + RPW - 1) / RPW * RPW, (a.rows[1] + RPW - 1) / RPW * RPW,
                               (a.rows[2] + RPW - 1) / RPW * RPW};
    const int seg = segment_of(spans, a.nseg, r0);
    const uint32_t seg_rows = pick3(a.rows, seg);
    const uint16_t* const seg_w = pick3(a.w, seg);
    uint16_t* const seg_y = pick3(a.y, seg);
    if (r0 >= seg_rows) return;  // a grid's last waves may have no rows
    const uint32_t nrows = min((uint32_t)RPW, seg_rows - r0);
    const uint32_t row_bytes = 2 * N;
    __amdgpu_buffer_rsrc_t rw[EPI == kDgSwiglu ? 2 : 1];
    rw[0] = make_rsrc(seg_w + (size_t)r0 * N, nrows * row_bytes);
    if constexpr (EPI == kDgSwiglu) rw[1] = make_rsrc(a.w[1] + (size_t)r0 * N, nrows * row_bytes);
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, row_bytes);
    uint4 wv[NR][NCH], xv[NCH], gv[NCH];
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
        // Chunks past the row's end read zeros: their offset is moved past
        // every buffer's range (not into the next row).
        const uint32_t off = 16 * (lane + 64 * k);
        const bool in = off < row_bytes;
#pragma unroll
        for (int r = 0; r < NR; ++r)
            wv[r][k] = buf_load16_nt(rw[r / RPW], in ? (r % RPW) * row_bytes + off : 0x80000000u);
        xv[k] = buf_load16(rx, off);
        if constexpr (NORM) gv[k] = buf_load16(make_rsrc(a.norm_w, row_bytes), off);
    }
    uint16_t res = 0;
    if (EPI == kDgResidual && (uint32_t)lane < nrows) res = seg_y[r0 + lane];

    if constexpr (NORM) {
        float ss = 0.0f;
#pragma unroll
        for (int k = 0; k < NCH; ++k)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t wd = word_of(xv[k], i);
                ss = fmaf(bf16_lo(wd), bf16_lo(wd), ss);
                ss = fmaf(bf16_hi(wd), bf16_hi(wd), ss);
            }
        const float inv = rsqrtf(fmaf(wave_sum(ss), 1.0f / (float)N, a.eps));
#pragma unroll
        for (int k = 0; k < NCH; ++k) {
            uint32_t* ow = reinterpret_cast<uint32_t*>(&xv[k]);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t p = ow[i], q = word_of(gv[k], i);
                ow[i] = pack_bf16x2(bf16_lo(p) * inv * bf16_lo(q), bf16_hi(p) * inv * bf16_hi(q));
            }
        }
    }
    float sum[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < NCH; ++k) acc = dot8(wv[r][k], xv[k], acc);
        sum[r] = wave_sum(acc);
    }
    // Lane r writes row r (sums are in every lane; pick lane r's by a chain
    // of selects, no dynamic register indexing).
    float v = 0.0f, u = 0.0f;
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        v = lane == r ? sum[r] : v;
        if constexpr (EPI == kDgSwiglu) u = lane == r ? sum[RPW + r] : u;
    }
    if ((uint32_t)lane < nrows) {
        const uint32_t m = r0 + lane;
        if constexpr (EPI == kDgPlain) {
            seg_y[m] = f32_to_bf16(v);
        } else if constexpr (EPI == kDgResidual) {
            seg_y[m] = f32_to_bf16(bf16_to_f32(res) + bf16_round(v));
        } else {
            const float g = bf16_round(v), up = bf16_round(u);
            a.y[0][m] = f32_to_bf16(up * (g * (1.0f / (1.0f + expf(-g)))));
        }
    }
}

template <int RPW, int NCH, bool NORM, int EPI>
hipError_t dw_launch(const DecodeGemvArgs& a, hipStream_t stream) {
    uint32_t waves = 0;
    for (int s = 0; s < a.nseg; ++s) waves += (a.rows[s] + RPW - 1) / RPW;
    const uint32_t groups = (waves + kDwWaves - 1) / kDwWaves;
    decode_gemv_wave_kernel<RPW, NCH, NORM, EPI><<<groups, 64 * kDwWaves, 0, stream>>>(a);
    return hipGetLastError();
}

template <int NCH, bool NORM, int EPI>
hipError_t dw_rows(const DecodeGemvArgs& a, uint32_t total, hipStream_t stream) {
    // Rows per wave: about 2048 waves in the grid, at most 16 row loads per
    // lane.
    constexpr int PAIRS = EPI == kDgSwiglu ? 2 : 1;
    constexpr int CAP = 16 / (NCH * PAIRS) >= 8 ? 8 : 16 / (NCH * PAIRS) >= 4 ? 4 : 16 / (NCH * PAIRS) >= 2 ? 2 : 1;
    const uint32_t want = total / 2048;
    const int rpw = want >= 8 ? 8 : want >= 4 ? 4 : want >= 2 ? 2 : 1;
    const int r = rpw < CAP ? rpw : CAP;
    if (r >= 8 && CAP >= 8) return dw_launch<(CAP >= 8 ? 8 : 1), NCH, NORM, EPI>(a, stream);
    if (r >= 4 && CAP >= 4) return dw_launch<(CAP >= 4 ? 4 : 1), NCH, NORM, EPI>(a, stream);
    if (r >= 2 && CAP >= 2) return dw_launch<(CAP >= 2 ? 2 : 1), NCH, NORM, EPI>(a, stream);
    return dw_launch<1, NCH, NORM, EPI>(a, stream);
}

template <bool NORM, int EPI>
hipError_t dw_dispatch(const DecodeGemvArgs& a, uint32_t total, hipStream_t stream) {
    const uint32_t nch = (a.n / 8 + 63) / 64;
    if (nch <= 2) return dw_rows<2, NORM, EPI>(a, total, stream);
    if (nch <= 4) return dw_rows<4, NORM, EPI>(a, total, stream);
    if (nch <= 6) return dw_rows<6, NORM, EPI>(a, total, stream);
    return dw_rows<8, NORM, EPI>(a, total, stream);
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
    if (a.n <= 4096 && a.n % 8 == 0) return dw_dispatch<NORM, EPI>(a, total, stream);
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
constexpr int kAmBlocks = 64, kAmThreads = 512;
constexpr int kAmUnroll = 8;  // loads per lane in flight (one round for V <= 262144)

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
    constexpr uint32_t kStride = kAmBlocks * kAmThreads;
    for (uint32_t i0 = blockIdx.x * kAmThreads + threadIdx.x; i0 < n; i0 += kAmUnroll * kStride) {
        float v[kAmUnroll];
#pragma unroll
        for (int u = 0; u < kAmUnroll; ++u) {
            const uint32_t i = i0 + u * kStride;
            v[u] = i < n ? logits[i] : -INFINITY;
        }
#pragma unroll
        for (int u = 0; u < kAmUnroll; ++u) {
            const uint32_t i = i0 + u * kStride;
            const uint64_t k = i < n ? am_key(v[u], i) : 0;
            best = k > best ? k : best;
        }
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
