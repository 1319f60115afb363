// Split-K decode attention for gfx950.
//
// Replaces the reference's three-kernel decode pipeline
// (gqa_qk_gemv_bf16 -> softmax_f32 -> apply_score2v_f32 + convert,
// src/decode.cu:399-744) with one streaming pass over the KV cache plus a
// small combine.  Work unit: one workgroup = (sequence, KV head, group of up
// to 4 query heads, slice of the cached positions).  Each K/V row is read
// from HBM once and used by every query head of its GQA group.
//
// Per 16-position tile a wave issues, per lane, 4 (D=128) 16-byte loads of K
// and of V: lane (n = lane%16, g = lane/16) reads row t0+n, dims [g*D/4,
// (g+1)*D/4).  Scores come from v_mfma_f32_16x16x32_bf16 with K as the B
// operand (column n = position) and Q as the A operand with row m holding
// head (m % HG) of the workgroup's head group, so lane (n, g) receives its
// heads' scores of its own position and needs no shuffles.  A workgroup
// takes at most two query heads (HG <= 2: 64 fp32 accumulators per lane);
// the split count is a multiple of 8 whenever a KV head has several head
// groups, so the workgroups of one (sequence, KV head, split) differ in
// block id by a multiple of 8, run on the same XCD, and the second read of
// each K/V row is served by that XCD's L2.  Softmax is online across
// 128-position iterations in the log2 domain; P.V runs as fp32 FMAs on the
// lane's own V slice.  Partials (m, l, o[D]) are merged across the 4 waves
// in LDS and written once per workgroup; the combine kernel merges splits.
#include <math.h>

#include "common.hpp"
#include "kernels.hpp"

namespace tiattn {
namespace {

constexpr int kDecWaves = 4;
constexpr int kDecTilesPerWave = 2;
constexpr int kDecIterRows = kDecWaves * kDecTilesPerWave * 16;  // 128 positions

__device__ __forceinline__ uint32_t seq_length(const DecodeProblem& p, uint32_t b) {
    if (p.len_mode == kLenHost) return p.len_host;
    if (p.len_mode == kLenDevice) {
        const uint32_t L = p.len_dev[b];
        return L < p.len_cap ? L : p.len_cap;
    }
    const uint32_t pos = p.len_dev[0];
    return (pos < p.len_cap ? pos : p.len_cap - 1) + 1;
}

__device__ __forceinline__ void split_range(uint32_t L, uint32_t splits, uint32_t split,
                                            uint32_t* begin, uint32_t* end) {
    uint32_t per = (L + splits - 1) / splits;
    per = (per + kDecIterRows - 1) / kDecIterRows * kDecIterRows;
    const uint64_t b = (uint64_t)split * per;
    *begin = b < L ? (uint32_t)b : L;
    *end = (uint64_t)*begin + per < L ? *begin + per : L;
}

template <int D, int HG>
__global__ __launch_bounds__(256, 2) void decode_split_kernel(DecodeProblem p, DecodePartials part,
                                                              float scale_log2) {
    constexpr int DG = D / 4;    // dims per lane group
    constexpr int NLD = DG / 8;  // 16-byte loads per row slice == MFMA k-steps
    constexpr int TPW = kDecTilesPerWave;
    constexpr int STEP = kDecIterRows;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n = lane & 15, g = lane >> 4;
    const uint32_t group = p.hq / p.hkv;
    const uint32_t n_hg = (group + HG - 1) / HG;
    const uint32_t kvh = blockIdx.y / n_hg, hgi = blockIdx.y % n_hg;
    const uint32_t b = blockIdx.z;
    const uint32_t h0 = kvh * group + hgi * HG;
    const uint32_t nh = min((uint32_t)HG, group - hgi * HG);
    const int64_t bh0 = (int64_t)b * p.hq + h0;

    const uint32_t L = seq_length(p, b);
    uint32_t t_begin, t_end;
    split_range(L, p.splits, blockIdx.x, &t_begin, &t_end);
    if (t_begin >= t_end) {
        if (threadIdx.x < nh) {
            float* ml = part.ml + (bh0 + threadIdx.x) * part.ml_head + blockIdx.x * 2;
            ml[0] = -INFINITY;
            ml[1] = 0.0f;
        }
        return;
    }

    // A operand: row m = n of the 16x32 tile holds head slot m % HG, so
    // result row 4g + r (lane (n, g), value r) is head slot r % HG.
    const uint32_t slot_a = n % HG;
    const uint32_t qh = h0 + (slot_a < nh ? slot_a : 0);
    const uint16_t* qrow = p.q + ((int64_t)b * p.hq + qh) * D + DG * g;
    bf16x8_t qa[NLD];
#pragma unroll
    for (int i = 0; i < NLD; ++i) qa[i] = as_bf16x8(ldg16(qrow + 8 * i));

    const int64_t row_stride = (int64_t)p.hkv * D;
    const uint16_t* kbase = p.k + (int64_t)b * p.kv_stride + (int64_t)kvh * D + DG * g;
    const uint16_t* vbase = p.v + (int64_t)b * p.kv_stride + (int64_t)kvh * D + DG * g;

    float m_run[HG], l_run[HG], acc[HG][DG];
#pragma unroll
    for (int s = 0; s < HG; ++s) {
        m_run[s] = -INFINITY;
        l_run[s] = 0.0f;
#pragma unroll
        for (int d = 0; d < DG; ++d) acc[s][d] = 0.0f;
    }

    for (uint32_t base = t_begin; base < t_end; base += STEP) {
        uint4 kr[TPW][NLD], vr[TPW][NLD];
        bool valid[TPW];
#pragma unroll
        for (int j = 0; j < TPW; ++j) {
            const uint32_t t = base + (wave * TPW + j) * 16 + n;
            valid[j] = t < t_end;
            const uint32_t tc = valid[j] ? t : t_end - 1;
            const uint16_t* kp = kbase + (int64_t)tc * row_stride;
            const uint16_t* vp = vbase + (int64_t)tc * row_stride;
#pragma unroll
            for (int i = 0; i < NLD; ++i) kr[j][i] = ldg16(kp + 8 * i);
#pragma unroll
            for (int i = 0; i < NLD; ++i) vr[j][i] = ldg16(vp + 8 * i);
        }

        // Scores: lane (n, g) value r = head slot r % HG at position n.
        float s[TPW][HG];
#pragma unroll
        for (int j = 0; j < TPW; ++j) {
            f32x4_t c = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int i = 0; i < NLD; ++i) c = mfma16x16x32(qa[i], as_bf16x8(kr[j][i]), c);
#pragma unroll
            for (int sl = 0; sl < HG; ++sl) s[j][sl] = valid[j] ? c[sl] : -INFINITY;
        }

        // Online softmax; the running max is made wave-uniform (row 0's value).
#pragma unroll
        for (int sl = 0; sl < HG; ++sl) {
            float cm = s[0][sl];
#pragma unroll
            for (int j = 1; j < TPW; ++j) cm = fmaxf(cm, s[j][sl]);
            cm = row16_max(cm);
            cm = __builtin_bit_cast(float,
                                    __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, cm)));
            const float m_new = fmaxf(m_run[sl], cm * scale_log2);
            if (m_new > m_run[sl]) {
                const float alpha = exp2f(m_run[sl] - m_new);
                l_run[sl] *= alpha;
#pragma unroll
                for (int d = 0; d < DG; ++d) acc[sl][d] *= alpha;
                m_run[sl] = m_new;
            }
        }

#pragma unroll
        for (int j = 0; j < TPW; ++j) {
            float pj[HG];
#pragma unroll
            for (int sl = 0; sl < HG; ++sl) {
                const float mref = m_run[sl] == -INFINITY ? 0.0f : m_run[sl];
                pj[sl] = exp2f(fmaf(s[j][sl], scale_log2, -mref));
                l_run[sl] += pj[sl];
            }
#pragma unroll
            for (int i = 0; i < NLD; ++i) {
                const uint32_t w[4] = {vr[j][i].x, vr[j][i].y, vr[j][i].z, vr[j][i].w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float v0 = bf16_lo(w[e]), v1 = bf16_hi(w[e]);
#pragma unroll
                    for (int sl = 0; sl < HG; ++sl) {
                        acc[sl][8 * i + 2 * e] = fmaf(pj[sl], v0, acc[sl][8 * i + 2 * e]);
                        acc[sl][8 * i + 2 * e + 1] = fmaf(pj[sl], v1, acc[sl][8 * i + 2 * e + 1]);
                    }
                }
            }
        }
    }

    // Sum over the 16 positions held by each row, then merge the 4 waves.
#pragma unroll
    for (int sl = 0; sl < HG; ++sl) {
        l_run[sl] = row16_sum(l_run[sl]);
#pragma unroll
        for (int d = 0; d < DG; ++d) acc[sl][d] = row16_sum(acc[sl][d]);
    }
    __shared__ float s_o[kDecWaves][HG][D];
    __shared__ float s_ml[kDecWaves][HG][2];
    if (n == 0) {
#pragma unroll
        for (int sl = 0; sl < HG; ++sl)
#pragma unroll
            for (int d = 0; d < DG; ++d) s_o[wave][sl][DG * g + d] = acc[sl][d];
    }
    if (lane == 0) {
#pragma unroll
        for (int sl = 0; sl < HG; ++sl) {
            s_ml[wave][sl][0] = m_run[sl];
            s_ml[wave][sl][1] = l_run[sl];
        }
    }
    __syncthreads();
    for (int e = threadIdx.x; e < HG * D; e += blockDim.x) {
        const int sl = e / D, d = e % D;
        if (sl >= (int)nh) continue;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < kDecWaves; ++w) M = fmaxf(M, s_ml[w][sl][0]);
        float o = 0.0f, l = 0.0f;
#pragma unroll
        for (int w = 0; w < kDecWaves; ++w) {
            const float mw = s_ml[w][sl][0];
            if (mw == -INFINITY) continue;
            const float sc = exp2f(mw - M);
            o = fmaf(sc, s_o[w][sl][d], o);
            l = fmaf(sc, s_ml[w][sl][1], l);
        }
        const int64_t bh = bh0 + sl;
        part.o[bh * part.o_head + (int64_t)blockIdx.x * part.o_split + d] = o;
        if (d == 0) {
            float* ml = part.ml + bh * part.ml_head + blockIdx.x * 2;
            ml[0] = M;
            ml[1] = l;
        }
    }
}

// Merge the splits of one (sequence, q-head): thread d produces o[d].
template <int D>
__device__ __forceinline__ void merge_splits(const DecodePartials& part, int64_t bh,
                                             uint32_t splits, int d, float* out, float* m_out,
                                             float* l_out) {
    const float* ml = part.ml + bh * part.ml_head;
    const float* po = part.o + bh * part.o_head;
    float M = -INFINITY;
    for (uint32_t s = 0; s < splits; ++s) M = fmaxf(M, ml[2 * s]);
    float num = 0.0f, den = 0.0f;
    if (M != -INFINITY) {
        for (uint32_t s = 0; s < splits; ++s) {
            const float ms = ml[2 * s];
            if (ms == -INFINITY) continue;
            const float w = exp2f(ms - M);
            num = fmaf(w, po[(int64_t)s * part.o_split + d], num);
            den = fmaf(w, ml[2 * s + 1], den);
        }
    }
    *out = den > 0.0f ? num / den : 0.0f;
    *m_out = M;
    *l_out = den;
}

template <int D>
__global__ __launch_bounds__(D) void decode_combine_kernel(DecodePartials part, uint32_t splits,
                                                           uint16_t* o) {
    const int64_t bh = blockIdx.x;
    const int d = threadIdx.x;
    float r, m, l;
    merge_splits<D>(part, bh, splits, d, &r, &m, &l);
    o[bh * D + d] = f32_to_bf16(r);
}

// Reference-contract finaliser for one sequence: block h merges head h's
// partials, writes O_buffer/O, then rewrites score row h with the softmax
// probabilities (recomputing q.k for t < L) and zeros for L <= t < msl.  A
// block only touches its own head's rows, and reads every partial before
// the barrier, so partials may live inside score/O_buffer/O rows of head h.
template <int D>
__global__ __launch_bounds__(256) void decode_finalize_compat_kernel(DecodeProblem p,
                                                                     DecodePartials part,
                                                                     float* score, uint32_t msl,
                                                                     float* o_buffer, uint16_t* o,
                                                                     float scale_log2) {
    const uint32_t h = blockIdx.x;
    const uint32_t L = seq_length(p, 0);
    __shared__ float s_stats[2];
    __shared__ float s_q[D];
    float my_o = 0.0f;
    if (threadIdx.x < D) {
        float m, l;
        merge_splits<D>(part, h, p.splits, threadIdx.x, &my_o, &m, &l);
        if (threadIdx.x == 0) {
            s_stats[0] = m;
            s_stats[1] = l;
        }
        s_q[threadIdx.x] = bf16_to_f32(p.q[(int64_t)h * D + threadIdx.x]);
    }
    __syncthreads();
    if (threadIdx.x < D) {
        o_buffer[(int64_t)h * D + threadIdx.x] = my_o;
        o[(int64_t)h * D + threadIdx.x] = f32_to_bf16(my_o);
    }
    const float M = s_stats[0], den = s_stats[1];
    const float inv = den > 0.0f ? 1.0f / den : 0.0f;
    const float mref = M == -INFINITY ? 0.0f : M;
    const uint32_t kvh = h / (p.hq / p.hkv);
    float* srow = score + (int64_t)h * msl;
    for (uint32_t t = threadIdx.x; t < msl; t += blockDim.x) {
        float val = 0.0f;
        if (t < L) {
            const uint16_t* kr = p.k + ((int64_t)t * p.hkv + kvh) * D;
            float dot = 0.0f;
#pragma unroll
            for (int c = 0; c < D / 8; ++c) {
                const uint4 w = ldg16(kr + 8 * c);
                const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    dot = fmaf(s_q[8 * c + 2 * e], bf16_lo(ws[e]), dot);
                    dot = fmaf(s_q[8 * c + 2 * e + 1], bf16_hi(ws[e]), dot);
                }
            }
            val = exp2f(fmaf(dot, scale_log2, -mref)) * inv;
        }
        srow[t] = val;
    }
}

template <int D, int HG>
hipError_t launch_split_t(const DecodeProblem& p, const DecodePartials& part, hipStream_t st) {
    const uint32_t group = p.hq / p.hkv;
    const uint32_t n_hg = (group + HG - 1) / HG;
    const dim3 grid(p.splits, p.hkv * n_hg, p.batch);
    const float sl2 = kLog2e / sqrtf((float)D);
    hipLaunchKernelGGL((decode_split_kernel<D, HG>), grid, dim3(256), 0, st, p, part, sl2);
    return hipGetLastError();
}

template <int D>
hipError_t launch_split_d(const DecodeProblem& p, const DecodePartials& part, hipStream_t st) {
    const uint32_t group = p.hq / p.hkv;
    if (group == 1) return launch_split_t<D, 1>(p, part, st);
    return launch_split_t<D, 2>(p, part, st);
}

}  // namespace

uint32_t decode_head_groups(uint32_t group) { return group == 1 ? 1 : (group + 1) / 2; }

uint32_t decode_default_splits(uint32_t batch, uint32_t hq, uint32_t hkv, uint32_t d,
                               uint32_t seq_len) {
    (void)d;
    const uint32_t group = hq / hkv;
    const uint32_t n_hg = decode_head_groups(group);
    const uint64_t wgs_per_split = (uint64_t)batch * hkv * n_hg;
    const uint64_t target = 1024;  // about 4 workgroups per CU on 256 CUs
    uint64_t s = (target + wgs_per_split - 1) / wgs_per_split;
    const uint64_t max_s = ((uint64_t)seq_len + kDecIterRows - 1) / kDecIterRows;
    if (s > max_s) s = max_s;
    if (n_hg > 1) s = (s + 7) / 8 * 8;  // same-XCD pairing, see the file header
    if (s < 1) s = 1;
    return (uint32_t)s;
}

hipError_t launch_decode_split(const DecodeProblem& p, const DecodePartials& part,
                               hipStream_t stream) {
    if (p.d == 64) return launch_split_d<64>(p, part, stream);
    return launch_split_d<128>(p, part, stream);
}

hipError_t launch_decode_combine(const DecodeProblem& p, const DecodePartials& part, uint16_t* o,
                                 hipStream_t stream) {
    const dim3 grid(p.batch * p.hq);
    if (p.d == 64)
        hipLaunchKernelGGL(decode_combine_kernel<64>, grid, dim3(64), 0, stream, part, p.splits, o);
    else
        hipLaunchKernelGGL(decode_combine_kernel<128>, grid, dim3(128), 0, stream, part, p.splits,
                           o);
    return hipGetLastError();
}

hipError_t launch_decode_finalize_compat(const DecodeProblem& p, const DecodePartials& part,
                                         float* score, uint32_t msl, float* o_buffer,
                                         uint16_t* o, hipStream_t stream) {
    const dim3 grid(p.hq);
    const float sl2 = kLog2e / sqrtf((float)p.d);
    if (p.d == 64)
        hipLaunchKernelGGL(decode_finalize_compat_kernel<64>, grid, dim3(256), 0, stream, p, part,
                           score, msl, o_buffer, o, sl2);
    else
        hipLaunchKernelGGL(decode_finalize_compat_kernel<128>, grid, dim3(256), 0, stream, p, part,
                           score, msl, o_buffer, o, sl2);
    return hipGetLastError();
}

}  // namespace tiattn
