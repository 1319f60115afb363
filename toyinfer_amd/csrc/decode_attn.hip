// Split-K decode attention for gfx950.
//
// Replaces the reference's three-kernel decode pipeline
// (gqa_qk_gemv_bf16 -> softmax_f32 -> apply_score2v_f32 + convert,
// src/decode.cu:399-744) with one streaming pass over the KV cache plus a
// small combine.  Work unit: one workgroup = (sequence, KV head, slice of
// the cached positions) for all query heads of the GQA group (up to 16), so
// each K/V row is read from HBM exactly once.
//
// Per iteration a wave takes 32 positions (two 16-row tiles):
// * K: lane (n = lane%16, g = lane/16) loads rows t0+n and t0+16+n with
//   16-byte loads, directly in the A-operand layout of
//   v_mfma_f32_16x16x32_bf16; B = Q^T (column n = head n of the group).
//   Load i of lane (n, g) takes dims [32i + 8g, 32i + 8g + 8): the k-order
//   of a dot product is free as long as Q uses the same one, and this order
//   makes each load instruction read 64 contiguous bytes per row.  The next
//   iteration's K/V loads are issued as soon as this iteration's registers
//   are consumed, so they overlap the softmax and P.V.
//   The result S^T leaves lane (head n, g) holding positions
//   {4g..4g+3, 16+4g..16+4g+3} of its head: softmax is in-lane plus two
//   shuffles across the four lanes of a head.
// * Those eight probabilities, as bf16, are exactly the B operand (P^T) of
//   O^T += V^T P^T.  V goes registers -> the wave's own LDS tile (row-major,
//   16-byte chunks XOR-swizzled by row), and the A operand V^T comes back
//   with ds_read_b64_tr_b16, which transposes 16-bit elements across each
//   16-lane group: source lane s points at row p(g, s/4), column
//   16*db + 4*(s%4), and lane i receives rows p(g, 0..3) of column 16*db + i.
// * O^T accumulates in lane (head n, g) as d = 16*db + 4g + r: 32 fp32
//   accumulators per lane for D = 128, nothing to reduce across lanes.
// Softmax is online in the log2 domain; each wave keeps its own (m, l, O)
// and the four waves are merged in LDS into one partial (m, l, o[D]) per
// head and workgroup; the combine kernel merges the splits.
#include <math.h>

#include "common.hpp"
#include "kernels.hpp"
#include "norm_rope.hpp"

namespace tiattn {
namespace {

typedef short v4i16_t __attribute__((ext_vector_type(4)));

constexpr int kDecWaves = 4;
constexpr int kDecWaveRows = 32;                          // positions per wave-iteration
constexpr int kDecIterRows = kDecWaves * kDecWaveRows;    // 128 positions
constexpr int kDecMaxHeads = 16;                          // MFMA columns = query heads

__device__ __forceinline__ uint32_t seq_length(const DecodeProblem& p, uint32_t b) {
    if (p.len_mode == kLenHost) return p.len_host;
    if (p.len_mode == kLenDevice) {
        const uint32_t L = p.len_dev[b];
        return L < p.len_cap ? L : p.len_cap;
    }
    const uint32_t pos = p.len_dev[0];
    return (pos < p.len_cap ? pos : p.len_cap - 1) + 1;
}

// Split s of `splits` covers L/splits rows, plus one for the first L%splits
// splits: every workgroup streams the same number of bytes (the slowest one
// sets the kernel time).
__device__ __forceinline__ void split_range(uint32_t L, uint32_t splits, uint32_t split,
                                            uint32_t* begin, uint32_t* end) {
    const uint32_t per = L / splits, rem = L % splits;
    *begin = split * per + min(split, rem);
    *end = *begin + per + (split < rem ? 1u : 0u);
}

// Row-major K/V tile of one wave in LDS: element (row, col) at
// row*D + 8*((col/8) ^ swz(row)) + col%8.  With swz(r) = 2r mod D/8 the
// tile's stores, the K operand reads and the transposing V reads all run
// without bank conflicts (measured with SQ_LDS_BANK_CONFLICT on each access
// pattern alone).
template <int D>
__device__ __forceinline__ int vt_swz(int row) {
    return (2 * row) & (D / 8 - 1);
}

__device__ __forceinline__ v4i16_t ds_read_tr16(const uint16_t* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) v4i16_t*)(p));
}

constexpr int kMaxSplits = 1024;


// Reference-contract decode with the partials in the score rows
// ([Hq][msl] fp32, part.ml = score, row stride msl).  When the rows past
// the length L have room for the partials of at least half of the splits,
// the split pass also stores every raw score (q.k times
// log2(e)/sqrt(D)) at its position and puts the partials after them: the
// probabilities are then a rescale of the stored scores, with no second
// pass over K.  Otherwise (a position near msl) the partials start at the
// row head and the score pass recomputes q.k.  Every kernel of the
// contract path derives the same layout from L on the device, so a graph
// captured once serves every position.
struct CompatLayout {
    bool raw;
    uint32_t splits;       // splits that carry a slice (raw: fewer than the grid holds)
    DecodePartials part;
};

__device__ __forceinline__ CompatLayout compat_layout(const DecodeProblem& p,
                                                      const DecodePartials& part, uint32_t L) {
    const uint32_t room = p.len_cap - L;
    uint32_t fit = room / (p.d + 2);
    if (fit > p.splits) fit = p.splits;
    CompatLayout c;
    // Fewer splits stream more slowly (B=1, 32/8 heads, pos 32767 of 40960:
    // 63 of 96 splits take 29.4 us where 96 take 23); at half the splits
    // that loss is about what the skipped pass over K would cost.
    c.raw = fit >= 2 && 2 * fit >= p.splits;
    c.splits = c.raw ? fit : p.splits;
    c.part = part;
    if (c.raw) {
        c.part.ml = part.ml + L;
        c.part.o = part.ml + L + 2 * (size_t)fit;
    }
    return c;
}

// Workgroup blockIdx.x takes a fixed slice [t_begin, t_end) of the positions
// (split_range), its wave w the 32-row chunks w, w+4, ... of that slice.
// PRO: the engine's form with the token's q/k norm + RoPE and cache-row
// writes folded in (DecodePrologue).
// COMPAT: the reference-contract pass (B = 1, partials in the score rows,
// raw scores stored when compat_layout says so).
// FIXED (PRO only): p.slice_rows == 128, split s owns rows [128 s, 128 s +
// 128) whatever the length.
template <int D, bool PRO, bool COMPAT = false, bool FIXED = false>
__device__ __forceinline__ void decode_split_body(const DecodeProblem& p,
                                                  const DecodePartials& part_in, float scale_log2,
                                                  const DecodePrologue& pro) {
    constexpr int NLD = D / 32;  // 16-byte loads per row and lane == QK k-steps
    constexpr int NDB = D / 16;  // PV output blocks of 16 dims
    constexpr int V_ELEMS = kDecWaveRows * D;
    // LDS: per-wave V tiles during the loop, the cross-wave merge afterwards.
    constexpr int LDS_BYTES_V = kDecWaves * V_ELEMS * 2;
    constexpr int OP = D + 4;  // merge row pitch (floats): the 16-byte stores of 4 head rows
                               // land in distinct banks
    constexpr int LDS_BYTES_O = kDecWaves * kDecMaxHeads * OP * 4;
    __shared__ __align__(16) unsigned char s_raw[LDS_BYTES_V > LDS_BYTES_O ? LDS_BYTES_V
                                                                            : LDS_BYTES_O];
    __shared__ float s_ml[kDecWaves][kDecMaxHeads][2];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n = lane & 15, g = lane >> 4;
    const uint32_t group = p.hq / p.hkv;
    const uint32_t n_hg = (group + kDecMaxHeads - 1) / kDecMaxHeads;
    const uint32_t kvh = blockIdx.y / n_hg, hgi = blockIdx.y % n_hg;
    const uint32_t b = blockIdx.z;
    const uint32_t h0 = kvh * group + hgi * kDecMaxHeads;
    const uint32_t nh = min((uint32_t)kDecMaxHeads, group - hgi * kDecMaxHeads);
    const int64_t bh0 = (int64_t)b * p.hq + h0;

    // Global loads: instruction j of lane l reads row (l>>3) + 8*(j / CPL) of the
    // wave's 32, 16-byte chunk (l&7) + 8*(j % CPL): each instruction covers 8
    // whole 128-byte lines, the shape the memory pipeline streams fastest.
    // The cache is read exactly once, so the loads carry the non-temporal hint
    // (6.4-6.6 TB/s for this pattern where plain loads reach 5.6-5.9).
    constexpr int CPR = D / 8;        // 16-byte chunks per row
    constexpr int CPL = CPR / 8;      // 128-byte lines per row
    constexpr int NJ = kDecWaveRows * CPR / 64;
    const int lrow = lane >> 3, lchunk = lane & 7;
    const int64_t row_stride = (int64_t)p.hkv * D;
    const uint16_t* kbase = p.k + (int64_t)b * p.kv_stride + (int64_t)kvh * D;
    const uint16_t* vbase = p.v + (int64_t)b * p.kv_stride + (int64_t)kvh * D;
    uint4 kr[NJ], vr[NJ];
    auto load_rows = [&](uint32_t tb, uint32_t lim) {  // rows tb .. tb+31, clamped below lim
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const uint32_t t = tb + lrow + 8 * (j / CPL);
            const uint32_t tc = t < lim ? t : lim - 1;
            const int64_t off = (int64_t)tc * row_stride + 8 * (lchunk + 8 * (j % CPL));
            kr[j] = ldg16_nt(kbase + off);
            vr[j] = ldg16_nt(vbase + off);
        }
    };
    // PRO: rows of LPR lanes each (lane group prow) load the q heads (rows
    // 0 .. nh-1) and the token's raw k and v rows (rows kDecMaxHeads,
    // kDecMaxHeads + 1; every workgroup loads them, the one whose slice holds
    // the token uses them).  Nothing here depends on the device length (the
    // rotary row of the position is pro.rope), so these loads go out first
    // and the arithmetic waits for them alone.
    constexpr int LPR = D / 16;
    constexpr int kNewK = kDecMaxHeads, kNewV = kDecMaxHeads + 1;
    __shared__ __align__(16) uint16_t s_pro[PRO ? (kDecMaxHeads + 2) * D : 8];
    const int prow = threadIdx.x / LPR, pc = threadIdx.x % LPR;
    int pmode = -1;  // -1: no prologue row in this lane
    NormRopeIn pin;
    uint4 pro_a, pro_b;  // the lane's two output chunks of its prologue row
    if constexpr (PRO) {
        // Every lane runs one unconditional load sequence (per-lane sources;
        // lanes without a row re-read q row 0, the v row loads weights and
        // angles it does not use): loads under a branch would make the
        // compiler wait for every load in flight, the K/V chunk's included,
        // before the arithmetic.
        const bool is_q = (uint32_t)prow < nh, is_k = prow == kNewK, is_v = prow == kNewV;
        pmode = is_q || is_k ? (kRowNorm | kRowRope) : (is_v ? 0 : -1);
        const uint16_t* src = is_k   ? pro.k_raw + (int64_t)kvh * D
                              : is_v ? pro.v_raw + (int64_t)kvh * D
                                     : p.q + (bh0 + (is_q ? prow : 0)) * D;
        const uint16_t* wsrc = is_k ? pro.k_w : pro.q_w;
        pin = norm_rope_load<D>(src, wsrc, nullptr, pro.rope, 0, pc, kRowNorm | kRowRope);
        // Keep these loads ahead of the K/V chunk's in the instruction
        // stream: loads complete in order, so the prologue's wait then leaves
        // the chunk in flight.
        __builtin_amdgcn_sched_barrier(0);
    }
    // Normalise + rotate the rows (row kNewV is a copy) into LDS; needs no
    // length.
    auto pro_compute = [&]() {
        if (pmode >= 0) {
            norm_rope_compute<D>(pin, true, pro.eps, 0, pmode, &pro_a, &pro_b);
            *reinterpret_cast<uint4*>(s_pro + prow * D + 8 * pc) = pro_a;
            *reinterpret_cast<uint4*>(s_pro + prow * D + 8 * pc + D / 2) = pro_b;
        }
    };

    // FIXED: the slice does not depend on the length, so its chunk (one
    // 32-row chunk per wave) is requested before the device length arrives,
    // its rows clamped to the cache (len_cap); rows at or past the length are
    // masked and their V zeroed in the loop.  The prologue rows are computed
    // meanwhile.
    // PRO takes its length from len_dev (kLenDevice); FIXED requests it
    // behind the chunk (a scalar load: its wait leaves the vector loads in
    // flight) and uses it after the prologue arithmetic.
    uint32_t len_pro = 0;
    if constexpr (FIXED) {
        load_rows(blockIdx.x * kDecIterRows + wave * kDecWaveRows, p.len_cap);
        __builtin_amdgcn_sched_barrier(0);
        len_pro = p.len_dev[b];
        pro_compute();
    } else if constexpr (PRO) {
        len_pro = p.len_dev[b];
    }

    const uint32_t L = PRO ? min(len_pro, p.len_cap) : seq_length(p, b);
    DecodePartials part = part_in;
    uint32_t nsplits = p.splits;
    bool raw = false;
    if constexpr (COMPAT) {
        const CompatLayout cl = compat_layout(p, part_in, L);
        if (blockIdx.x >= cl.splits) return;  // raw layout: this split carries no slice
        part = cl.part;
        nsplits = cl.splits;
        raw = cl.raw;
    }
    uint32_t t_begin, t_end;
    if (FIXED) {
        t_begin = blockIdx.x * kDecIterRows;
        t_end = min(t_begin + kDecIterRows, L);
    } else {
        split_range(L, nsplits, blockIdx.x, &t_begin, &t_end);
    }
    if (t_begin >= t_end) {
        if (threadIdx.x < nh) {
            float* ml = part.ml + (bh0 + threadIdx.x) * part.ml_head + blockIdx.x * 2;
            ml[0] = -INFINITY;
            ml[1] = 0.0f;
        }
        return;
    }

    const uint32_t pos = L - 1;
    const bool has_new = PRO && t_end == L;

    // B operand Q^T: column n = head h0 + n (zero beyond the group).
    bf16x8_t qb[NLD];
    if constexpr (!PRO) {
        const bool has = (uint32_t)n < nh;
        const uint16_t* qrow = p.q + (bh0 + (has ? n : 0)) * D + 8 * g;
#pragma unroll
        for (int i = 0; i < NLD; ++i) {
            uint4 x = ldg16(qrow + 32 * i);
            if (!has) x = make_uint4(0, 0, 0, 0);
            qb[i] = as_bf16x8(x);
        }
    }

    uint16_t* vs = reinterpret_cast<uint16_t*>(s_raw) + wave * V_ELEMS;

    f32x4_t acc[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db) acc[db] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    float m_run = -INFINITY, l_run = 0.0f;

    // tr16 read addresses (element offsets) of this lane for both halves.
    int tr_off[2][NDB];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
        const int row = 16 * hh + 4 * g + (n >> 2);
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
            const int col = 16 * db + 4 * (n & 3);
            tr_off[hh][db] = row * D + 8 * ((col >> 3) ^ vt_swz<D>(row)) + (col & 7);
        }
    }

    int st_off[NJ];  // LDS element offset of instruction j's chunk
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int row = lrow + 8 * (j / CPL), chunk = lchunk + 8 * (j % CPL);
        st_off[j] = row * D + 8 * (chunk ^ vt_swz<D>(row));
    }
    // PRO: row t_end - 1 is not written yet and rows past it hold older or
    // no data, so V of rows at or past t_end is zeroed (their scores are
    // masked, but 0 * NaN is NaN).
    auto zero_v_past_end = [&](uint32_t tb) {
#pragma unroll
        for (int j = 0; j < NJ; ++j)
            if (tb + lrow + 8 * (j / CPL) >= t_end) vr[j] = make_uint4(0, 0, 0, 0);
    };
    auto load_kv = [&](uint32_t tb) { load_rows(tb, t_end); };
    // Chunk c = rows [t_begin + 32c, t_begin + 32c + 32) (masked at t_end).
    const uint32_t nchunks = (t_end - t_begin + kDecWaveRows - 1) / kDecWaveRows;
    uint32_t cur = wave;
    // PRO: a wave without a chunk still loads one (rows clamped to t_end - 1,
    // never used), so that no branch separates these loads from the
    // prologue's.
    if (!FIXED && (PRO || cur < nchunks)) load_kv(t_begin + cur * kDecWaveRows);

    // PRO: the token's k/v rows also to cache row pos (one head group writes
    // them), then Q^T from LDS.
    if constexpr (PRO) {
        if constexpr (!FIXED) pro_compute();
        if (pmode >= 0 && prow >= kNewK && has_new && hgi == 0) {
            uint16_t* crow = (prow == kNewK ? pro.k_cache : pro.v_cache) +
                             ((int64_t)pos * p.hkv + kvh) * D;
            *reinterpret_cast<uint4*>(crow + 8 * pc) = pro_a;
            *reinterpret_cast<uint4*>(crow + 8 * pc + D / 2) = pro_b;
        }
        lds_barrier();
        const bool has = (uint32_t)n < nh;
#pragma unroll
        for (int i = 0; i < NLD; ++i) {
            uint4 x = *reinterpret_cast<const uint4*>(s_pro + (has ? n : 0) * D + 8 * g + 32 * i);
            if (!has) x = make_uint4(0, 0, 0, 0);
            qb[i] = as_bf16x8(x);
        }
    }
    while (cur < nchunks) {
        const uint32_t t0 = t_begin + cur * kDecWaveRows;
        // K -> this wave's LDS tile, then the A operand (row 16*tt + n, chunk
        // 4i + g) back out of it.
#pragma unroll
        for (int j = 0; j < NJ; ++j) *reinterpret_cast<uint4*>(vs + st_off[j]) = kr[j];
        // PRO: the token's own row, from s_pro (LDS operations of a wave
        // complete in order, so this lands after the tile store above).
        const uint32_t rnew = pos - t0;
        const bool put_new = has_new && rnew < (uint32_t)kDecWaveRows && lane < D / 8;
        if (PRO && put_new)
            *reinterpret_cast<uint4*>(vs + rnew * D + 8 * (lane ^ vt_swz<D>(rnew))) =
                *reinterpret_cast<const uint4*>(s_pro + kNewK * D + 8 * lane);
        bf16x8_t ka[2][NLD];
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            const int row = 16 * tt + n;
#pragma unroll
            for (int i = 0; i < NLD; ++i)
                ka[tt][i] = as_bf16x8(*reinterpret_cast<const uint4*>(
                    vs + row * D + 8 * ((4 * i + g) ^ vt_swz<D>(row))));
        }
        // V -> the same tile (LDS operations of a wave complete in order, so
        // the K reads above see K).
        if (PRO) zero_v_past_end(t0);
#pragma unroll
        for (int j = 0; j < NJ; ++j) *reinterpret_cast<uint4*>(vs + st_off[j]) = vr[j];
        if (PRO && put_new)
            *reinterpret_cast<uint4*>(vs + rnew * D + 8 * (lane ^ vt_swz<D>(rnew))) =
                *reinterpret_cast<const uint4*>(s_pro + kNewV * D + 8 * lane);
        // S^T: lane (head n, g) value r of tile tt = position t0 + 16*tt + 4g + r.
        f32x4_t st[2];
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            st[tt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int i = 0; i < NLD; ++i) st[tt] = mfma16x16x32(ka[tt][i], qb[i], st[tt]);
        }
        if (COMPAT && raw && (uint32_t)n < nh) {
            float* srow = part_in.ml + (int64_t)(h0 + n) * part_in.ml_head;
#pragma unroll
            for (int tt = 0; tt < 2; ++tt)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const uint32_t t = t0 + 16 * tt + 4 * g + r;
                    if (t < t_end) srow[t] = st[tt][r] * scale_log2;
                }
        }
        // The load registers are free: the next chunk's loads overlap this
        // chunk's softmax and P.V.
        const uint32_t nxt = cur + kDecWaves;
        if (nxt < nchunks) load_kv(t_begin + nxt * kDecWaveRows);
        float mx = -INFINITY;
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t t = t0 + 16 * tt + 4 * g + r;
                if (t >= t_end) st[tt][r] = -INFINITY;
                mx = fmaxf(mx, st[tt][r]);
            }
        mx = xor32_max(xor16_max(mx));
        const float m_new = fmaxf(m_run, mx * scale_log2);
        if (m_new > m_run) {
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
            l_run *= alpha;
#pragma unroll
            for (int db = 0; db < NDB; ++db) acc[db] *= alpha;
            m_run = m_new;
        }
        const float mref = m_run == -INFINITY ? 0.0f : m_run;
        float pr[8];
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                pr[4 * tt + r] = __builtin_amdgcn_exp2f(fmaf(st[tt][r], scale_log2, -mref));
        // P.V multiplies the bf16-rounded probabilities, so the denominator
        // sums exactly those values: numerator and denominator see the same P.
        const uint4 pw = make_uint4(pack_bf16x2(pr[0], pr[1]), pack_bf16x2(pr[2], pr[3]),
                                    pack_bf16x2(pr[4], pr[5]), pack_bf16x2(pr[6], pr[7]));
        l_run = sum_bf16x8(pw, l_run);
        const bf16x8_t pb = as_bf16x8(pw);
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
            const v4i16_t lo = ds_read_tr16(vs + tr_off[0][db]);
            const v4i16_t hi = ds_read_tr16(vs + tr_off[1][db]);
            const uint4 a = make_uint4(__builtin_bit_cast(uint2, lo).x, __builtin_bit_cast(uint2, lo).y,
                                       __builtin_bit_cast(uint2, hi).x, __builtin_bit_cast(uint2, hi).y);
            acc[db] = mfma16x16x32(as_bf16x8(a), pb, acc[db]);
        }
        cur = nxt;
    }

    // Merge the four waves: per head n, l summed over the 4 lanes of the head.
    l_run = xor32_sum(xor16_sum(l_run));
    __syncthreads();  // every wave is done with its V tile; s_raw becomes s_o
    float* s_o = reinterpret_cast<float*>(s_raw);  // [wave][head][D]
    if ((uint32_t)n < nh) {
#pragma unroll
        for (int db = 0; db < NDB; ++db)
            *reinterpret_cast<f32x4_t*>(s_o + (wave * kDecMaxHeads + n) * OP + 16 * db + 4 * g) = acc[db];
        if (g == 0) {
            s_ml[wave][n][0] = m_run;
            s_ml[wave][n][1] = l_run;
        }
    }
    __syncthreads();
    // Four dims of one head per thread; every LDS load is unconditional (a
    // wave that saw no row holds o = 0 and gets weight 0).
    for (int e = threadIdx.x; e < (int)nh * (D / 4); e += blockDim.x) {
        const int hs = e / (D / 4), d = 4 * (e % (D / 4));
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < kDecWaves; ++w) M = fmaxf(M, s_ml[w][hs][0]);
        f32x4_t o = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
        float l = 0.0f;
#pragma unroll
        for (int w = 0; w < kDecWaves; ++w) {
            const float mw = s_ml[w][hs][0];
            const float sc = mw == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mw - M);
            o += sc * *reinterpret_cast<const f32x4_t*>(s_o + (w * kDecMaxHeads + hs) * OP + d);
            l = fmaf(sc, s_ml[w][hs][1], l);
        }
        const int64_t bh = bh0 + hs;
        // Dword stores: the reference-contract layout keeps partials at
        // 4-byte alignment only.
        float* po = part.o + bh * part.o_head + (int64_t)blockIdx.x * part.o_split + d;
#pragma unroll
        for (int r = 0; r < 4; ++r) po[r] = o[r];
        if (d == 0) {
            float* ml = part.ml + bh * part.ml_head + blockIdx.x * 2;
            ml[0] = M;
            ml[1] = l;
        }
    }
}

// Three 4-wave workgroups per CU (the batched grids fill the chip).
template <int D>
__global__ __launch_bounds__(256, 3) void decode_split_kernel(DecodeProblem p, DecodePartials part,
                                                              float scale_log2) {
    decode_split_body<D, false>(p, part, scale_log2, DecodePrologue{});
}

// Reference-contract split pass (compat_layout).
template <int D>
__global__ __launch_bounds__(256, 3) void decode_split_compat_kernel(DecodeProblem p,
                                                                     DecodePartials part,
                                                                     float scale_log2) {
    decode_split_body<D, false, true>(p, part, scale_log2, DecodePrologue{});
}

// The engine's single-sequence grid (splits x Hkv workgroups) is far below
// one per CU, so the register budget is not cut for occupancy.
template <int D, bool FIXED>
__global__ __launch_bounds__(256, 1) void decode_split_pro_kernel(DecodeProblem p,
                                                                  DecodePartials part,
                                                                  float scale_log2,
                                                                  DecodePrologue pro) {
    decode_split_body<D, true, false, FIXED>(p, part, scale_log2, pro);
}

// Merge the splits of one (sequence, q-head) in a 256-thread block.  The
// per-split weights 2^(m_s - M) go to LDS first, so the pass over the
// partial outputs is a set of independent loads.  Empty splits (m = -inf)
// get weight 0 and their never-written o is not used.
constexpr int kCombineThreads = 256;

__device__ __forceinline__ float block_reduce(float x, bool is_max, float* s_red) {
    x = is_max ? fmaxf(x, dpp_f32<kDppXor1>(x)) : x + dpp_f32<kDppXor1>(x);
    x = is_max ? fmaxf(x, dpp_f32<kDppXor2>(x)) : x + dpp_f32<kDppXor2>(x);
    x = is_max ? fmaxf(x, dpp_f32<kDppRowHalfMirror>(x)) : x + dpp_f32<kDppRowHalfMirror>(x);
    x = is_max ? fmaxf(x, dpp_f32<kDppRowMirror>(x)) : x + dpp_f32<kDppRowMirror>(x);
    x = is_max ? xor32_max(xor16_max(x)) : xor32_sum(xor16_sum(x));
    const int wave = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) s_red[wave] = x;
    __syncthreads();
    float r = s_red[0];
    for (int w = 1; w < kCombineThreads / 64; ++w) r = is_max ? fmaxf(r, s_red[w]) : r + s_red[w];
    return r;
}

// Returns o[d] for d = threadIdx.x % D (valid in threads < D); M and the
// softmax denominator in *m_out / *l_out (all threads).
template <int D>
__device__ float merge_splits(const DecodePartials& part, int64_t bh, uint32_t splits,
                              float* m_out, float* l_out) {
    __shared__ float s_w[kMaxSplits];
    __shared__ float s_red[kCombineThreads / 64];
    __shared__ float s_part[kCombineThreads];
    const float* ml = part.ml + bh * part.ml_head;
    const float* po = part.o + bh * part.o_head;
    const int tid = threadIdx.x;
    float mloc = -INFINITY;
    for (uint32_t s = tid; s < splits; s += kCombineThreads) mloc = fmaxf(mloc, ml[2 * s]);
    const float M = block_reduce(mloc, true, s_red);
    float lloc = 0.0f;
    for (uint32_t s = tid; s < splits; s += kCombineThreads) {
        const float ms = ml[2 * s];
        const float w = ms == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ms - M);
        s_w[s] = w;
        lloc = fmaf(w, ml[2 * s + 1], lloc);
    }
    const float den = block_reduce(lloc, false, s_red);  // also orders the s_w writes
    constexpr int NPART = kCombineThreads / D;
    const int d = tid % D, q = tid / D;
    float num = 0.0f;
#pragma unroll 8
    for (uint32_t s = q; s < splits; s += NPART) {
        const float w = s_w[s];
        const float o = po[(int64_t)s * part.o_split + d];
        num += w != 0.0f ? w * o : 0.0f;
    }
    s_part[tid] = num;
    __syncthreads();
    float tot = 0.0f;
    if (tid < D)
        for (int k = 0; k < NPART; ++k) tot += s_part[k * D + tid];
    *m_out = M;
    *l_out = den;
    return den > 0.0f ? tot / den : 0.0f;
}

// Combine for the batched path: block = (sequence, q-head) with W waves
// (W = blockDim.x / 64, up to kCombineMaxWaves).  Wave w merges the splits
// w, w+W, ... online (running maximum with rescaling; lane l owns dims
// DPL*l .. +DPL-1), eight splits' loads in flight together, so one round of
// global loads suffices for up to 8 W splits; the W partial merges then meet
// in LDS.  A split that saw no position (m = -inf) gets weight 0 and its
// never-written o is not used.
constexpr int kCombineMaxWaves = 16;

__device__ __forceinline__ void merge_partial(float& M, float& den, float* acc, int n, float m,
                                              float l, const float* o) {
    const float Mn = fmaxf(M, m);
    const float a = M == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(M - Mn);
    const float b = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - Mn);
    den = fmaf(den, a, b * l);
    for (int e = 0; e < n; ++e) {
        const float t = fmaf(b, o[e], acc[e] * a);
        acc[e] = b != 0.0f ? t : acc[e] * a;
    }
    M = Mn;
}

// VEC: partial rows are 8-byte aligned (the batched workspace), so a lane's
// two dims load as one float2; else (partials in the reference contract's
// score rows, 4-byte aligned) as two floats.  o_f32 (optional) receives the
// fp32 result as well.
template <int D, bool VEC>
__global__ __launch_bounds__(64 * kCombineMaxWaves) void decode_combine_kernel(DecodePartials part,
                                                                             uint32_t splits,
                                                                             uint16_t* o,
                                                                             float* o_f32) {
    constexpr int DPL = D / 64;
    constexpr int U = 8;
    __shared__ float s_acc[kCombineMaxWaves][D];
    __shared__ float s_ml[kCombineMaxWaves][2];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n_waves = blockDim.x >> 6;
    const int64_t bh = blockIdx.x;
    const float* ml = part.ml + bh * part.ml_head;
    const float* po = part.o + bh * part.o_head + DPL * lane;

    float M = -INFINITY, den = 0.0f, acc[DPL];
#pragma unroll
    for (int e = 0; e < DPL; ++e) acc[e] = 0.0f;
    for (uint32_t s0 = wave; s0 < splits; s0 += U * n_waves) {
        float m[U], l[U], v[U][DPL];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t sp = s0 + u * n_waves < splits ? s0 + u * n_waves : s0;
            m[u] = ml[2 * sp];
            l[u] = ml[2 * sp + 1];
            const float* src = po + (int64_t)sp * part.o_split;
            if constexpr (DPL == 2 && VEC) {
                const float2 x = *reinterpret_cast<const float2*>(src);
                v[u][0] = x.x;
                v[u][1] = x.y;
            } else {
#pragma unroll
                for (int e = 0; e < DPL; ++e) v[u][e] = src[e];
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
            merge_partial(M, den, acc, DPL, s0 + u * n_waves < splits ? m[u] : -INFINITY, l[u],
                          v[u]);
    }
#pragma unroll
    for (int e = 0; e < DPL; ++e) s_acc[wave][DPL * lane + e] = acc[e];
    if (lane == 0) {
        s_ml[wave][0] = M;
        s_ml[wave][1] = den;
    }
    __syncthreads();
    if (wave != 0) return;
    float Mt = -INFINITY, dt = 0.0f, tot[DPL];
#pragma unroll
    for (int e = 0; e < DPL; ++e) tot[e] = 0.0f;
    for (int w = 0; w < n_waves; ++w) {
        float x[DPL];
#pragma unroll
        for (int e = 0; e < DPL; ++e) x[e] = s_acc[w][DPL * lane + e];
        merge_partial(Mt, dt, tot, DPL, s_ml[w][0], s_ml[w][1], x);
    }
    const float inv = dt > 0.0f ? 1.0f / dt : 0.0f;
    if (o_f32) {
#pragma unroll
        for (int e = 0; e < DPL; ++e) o_f32[bh * D + DPL * lane + e] = tot[e] * inv;
    }
    if constexpr (DPL == 2)
        *reinterpret_cast<uint32_t*>(o + bh * D + 2 * lane) = pack_bf16x2(tot[0] * inv, tot[1] * inv);
    else
        o[bh * D + lane] = f32_to_bf16(tot[0] * inv);
}

// Combine for few (sequence, q-head) pairs with many splits (one long
// sequence): block = (pair, 32-dim slice), 256 threads = 8 split groups x 32
// dims.  Thread (g, d) merges splits g, g+8, ... of dim d online, four
// splits' loads in flight together; the eight groups meet in LDS.  With B=1
// and 32 heads the per-pair kernel above runs 32 blocks that each pull all
// the pair's partials through one CU; this grid spreads the same bytes over
// D/32 times as many blocks.  Loads are dwords, so any partial alignment is
// accepted.
constexpr int kSliceDims = 32;
constexpr int kSliceGroups = 8;
// Below this many (sequence, q-head) pairs the sliced combine is used
// (B=1, 32 heads, 96 splits: 2.9 against 3.8 us; at 256 pairs the two are
// level).
constexpr uint32_t kSlicedCombineBelowPairs = 256;

template <int D>
__global__ __launch_bounds__(kSliceDims * kSliceGroups) void decode_combine_sliced_kernel(
    DecodePartials part, uint32_t splits, uint16_t* o, float* o_f32) {
    constexpr int U = 4;
    __shared__ float s_acc[kSliceGroups][kSliceDims];
    __shared__ float s_ml[kSliceGroups][2];
    const int dl = threadIdx.x % kSliceDims, sg = threadIdx.x / kSliceDims;
    const int64_t bh = blockIdx.x;
    const int d = blockIdx.y * kSliceDims + dl;
    const float* ml = part.ml + bh * part.ml_head;
    const float* po = part.o + bh * part.o_head + d;
    float M = -INFINITY, den = 0.0f, acc = 0.0f;
    for (uint32_t s0 = sg; s0 < splits; s0 += U * kSliceGroups) {
        float m[U], l[U], v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t sp = s0 + u * kSliceGroups < splits ? s0 + u * kSliceGroups : s0;
            m[u] = ml[2 * sp];
            l[u] = ml[2 * sp + 1];
            v[u] = po[(int64_t)sp * part.o_split];
        }
        // Every load above in flight before the first use.
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < U; ++u)
            merge_partial(M, den, &acc, 1, s0 + u * kSliceGroups < splits ? m[u] : -INFINITY, l[u],
                          &v[u]);
    }
    s_acc[sg][dl] = acc;
    if (dl == 0) {
        s_ml[sg][0] = M;
        s_ml[sg][1] = den;
    }
    __syncthreads();
    if (sg != 0) return;
    float Mt = -INFINITY, dt = 0.0f, tot = 0.0f;
#pragma unroll
    for (int g = 0; g < kSliceGroups; ++g) {
        const float x = s_acc[g][dl];
        merge_partial(Mt, dt, &tot, 1, s_ml[g][0], s_ml[g][1], &x);
    }
    const float inv = dt > 0.0f ? 1.0f / dt : 0.0f;
    const float r = tot * inv;
    if (o_f32) o_f32[bh * D + d] = r;
    o[bh * D + d] = f32_to_bf16(r);
}

// Reference-contract finaliser for one sequence: block h merges head h's
// partials, writes O_buffer/O, then rewrites score row h with the softmax
// probabilities (recomputing q.k for t < L) and zeros for L <= t < msl.  A
// block only touches its own head's rows, and reads every partial before
// the barrier, so partials may live inside score/O_buffer/O rows of head h.
template <int D>
__global__ __launch_bounds__(kCombineThreads) void decode_finalize_compat_kernel(
    DecodeProblem p, DecodePartials part, float* score, uint32_t msl, float* o_buffer,
    uint16_t* o, float scale_log2) {
    const uint32_t h = blockIdx.x;
    const uint32_t L = seq_length(p, 0);
    __shared__ float s_q[D];
    float M, den;
    const float my_o = merge_splits<D>(part, h, p.splits, &M, &den);
    if (threadIdx.x < D) s_q[threadIdx.x] = bf16_to_f32(p.q[(int64_t)h * D + threadIdx.x]);
    __syncthreads();  // all partial reads of this head are done
    if (threadIdx.x < D) {
        o_buffer[(int64_t)h * D + threadIdx.x] = my_o;
        o[(int64_t)h * D + threadIdx.x] = f32_to_bf16(my_o);
    }
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
            val = __builtin_amdgcn_exp2f(fmaf(dot, scale_log2, -mref)) * inv;
        }
        srow[t] = val;
    }
}

template <int D>
hipError_t launch_split_t(const DecodeProblem& p, const DecodePartials& part, hipStream_t st) {
    const uint32_t group = p.hq / p.hkv;
    const dim3 grid(p.splits, p.hkv * decode_head_groups(group), p.batch);
    const float sl2 = kLog2e / sqrtf((float)D);
    hipLaunchKernelGGL((decode_split_kernel<D>), grid, dim3(256), 0, st, p, part, sl2);
    return hipGetLastError();
}

template <int D>
hipError_t launch_split_pro_t(const DecodeProblem& p, const DecodePartials& part,
                              const DecodePrologue& pro, hipStream_t st) {
    const uint32_t group = p.hq / p.hkv;
    const dim3 grid(p.splits, p.hkv * decode_head_groups(group), 1);
    const float sl2 = kLog2e / sqrtf((float)D);
    if (p.slice_rows != 0)
        hipLaunchKernelGGL((decode_split_pro_kernel<D, true>), grid, dim3(256), 0, st, p, part, sl2,
                           pro);
    else
        hipLaunchKernelGGL((decode_split_pro_kernel<D, false>), grid, dim3(256), 0, st, p, part,
                           sl2, pro);
    return hipGetLastError();
}

// Concurrent split workgroups the device holds (CUs x resident blocks per
// CU), queried once per device; 256 CUs x 3 when no device is visible.
uint32_t split_slots(uint32_t d) {
    static int cache[2][64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
        (void)hipGetLastError();
        return 256 * 3;
    }
    const int which = d == 64 ? 0 : 1;
    int v = __atomic_load_n(&cache[which][dev], __ATOMIC_RELAXED);
    if (v > 0) return (uint32_t)v;
    int cus = 0, per = 0;
    hipError_t e1 = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    hipError_t e2 = d == 64
        ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, decode_split_kernel<64>, 256, 0)
        : hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, decode_split_kernel<128>, 256, 0);
    if (e1 != hipSuccess || e2 != hipSuccess || cus <= 0 || per <= 0) {
        (void)hipGetLastError();
        return 256 * 3;
    }
    v = cus * per;
    __atomic_store_n(&cache[which][dev], v, __ATOMIC_RELAXED);
    return (uint32_t)v;
}

// Reference contract, split partials in the score rows (two or more
// splits): the score rows hold partials until every head is merged, so the
// work is three stream-ordered kernels after the split pass.
//  1. decode_compat_merge_kernel (block = head): merges the head's partials,
//     writes O_buffer, and leaves (M, 1/den) in the first 8 bytes of the
//     head's O row (O is written last).
//  2. decode_compat_score_kernel (block = 128 positions of one KV head):
//     p = 2^(s*log2e/sqrt(D) - M) / den for its positions and up to 16 query
//     heads of the group (s recomputed from Q and K on MFMA), zeros past
//     the length, over the whole score row.
//  3. decode_compat_out_kernel: O = bf16(O_buffer).
__device__ __forceinline__ void stash_put(uint16_t* o_row, float a, float b) {
    const uint32_t ua = __float_as_uint(a), ub = __float_as_uint(b);
    o_row[0] = (uint16_t)(ua & 0xffffu);
    o_row[1] = (uint16_t)(ua >> 16);
    o_row[2] = (uint16_t)(ub & 0xffffu);
    o_row[3] = (uint16_t)(ub >> 16);
}
__device__ __forceinline__ float2 stash_get(const uint16_t* o_row) {
    return make_float2(__uint_as_float((uint32_t)o_row[0] | ((uint32_t)o_row[1] << 16)),
                       __uint_as_float((uint32_t)o_row[2] | ((uint32_t)o_row[3] << 16)));
}

template <int D>
__global__ __launch_bounds__(kCombineThreads) void decode_compat_merge_kernel(
    DecodeProblem p, DecodePartials part, float* o_buffer, uint16_t* o) {
    const uint32_t h = blockIdx.x;
    const CompatLayout cl = compat_layout(p, part, seq_length(p, 0));
    float M, den;
    const float my_o = merge_splits<D>(cl.part, h, cl.splits, &M, &den);
    if (threadIdx.x < D) o_buffer[(int64_t)h * D + threadIdx.x] = my_o;
    if (threadIdx.x == 0)
        stash_put(o + (int64_t)h * D, M == -INFINITY ? 0.0f : M, den > 0.0f ? 1.0f / den : 0.0f);
}

// Score pass: block = 128 positions (32 per wave) of one KV head and up to
// 16 of its query heads.  S^T = K Q^T is computed exactly as the split pass
// computes it (the same K load pattern, LDS tile and 16x16x32 MFMA operand
// order), so the probabilities use the same scores as O's weights; then
// p = 2^(s*log2e/sqrt(D) - M) / den per head, zeros past the length.  One
// chunk per wave: a loop over four chunks with the next one's loads in
// flight measured 5 % slower at a 32k position of a 40960-row cache.
template <int D>
__global__ __launch_bounds__(256) void decode_compat_score_kernel(
    DecodeProblem p, float* score, uint32_t msl, const uint16_t* o, float scale_log2) {
    constexpr int NLD = D / 32;
    constexpr int CPR = D / 8, CPL = CPR / 8, NJ = kDecWaveRows * CPR / 64;
    __shared__ __align__(16) uint16_t s_tile[kDecWaves][kDecWaveRows * D];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n = lane & 15, g = lane >> 4;
    const uint32_t group = p.hq / p.hkv;
    const uint32_t n_hg = (group + kDecMaxHeads - 1) / kDecMaxHeads;
    const uint32_t kvh = blockIdx.y / n_hg, hgi = blockIdx.y % n_hg;
    const uint32_t h0 = kvh * group + hgi * kDecMaxHeads;
    const uint32_t nh = min((uint32_t)kDecMaxHeads, group - hgi * kDecMaxHeads);
    const uint32_t L = seq_length(p, 0);
    // Raw layout: the split pass stored q.k * log2(e)/sqrt(D) at every
    // position below L; the probability is a rescale of it.  Wave w takes
    // heads w, w+4, ... of the group, lane l positions 2l, 2l+1 of the
    // wave's 128 (whole lines per instruction).
    DecodePartials sp{};
    sp.ml = score;
    if (compat_layout(p, sp, L).raw) {
        const uint32_t tb = blockIdx.x * kDecIterRows + 2 * lane;
        for (uint32_t hs = wave; hs < nh; hs += kDecWaves) {
            float* row = score + (int64_t)(h0 + hs) * msl;
            const float2 sv = stash_get(o + (int64_t)(h0 + hs) * D);
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const uint32_t t = tb + e;
                if (t < msl) row[t] = t < L ? __builtin_amdgcn_exp2f(row[t] - sv.x) * sv.y : 0.0f;
            }
        }
        return;
    }
    const uint32_t t0 = blockIdx.x * kDecIterRows + wave * kDecWaveRows;
    if (t0 >= msl) return;
    const bool has = (uint32_t)n < nh;
    float* srow = score + (int64_t)(h0 + (has ? n : 0)) * msl;
    if (t0 >= L) {  // the whole chunk is past the length
        if (has) {
#pragma unroll
            for (int tt = 0; tt < 2; ++tt)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const uint32_t t = t0 + 16 * tt + 4 * g + r;
                    if (t < msl) srow[t] = 0.0f;
                }
        }
        return;
    }
    // K rows t0 .. t0+31 (clamped below L), lane l: row l/8 (+8 per CPL
    // instructions), 16-byte chunk l%8 (+8).
    const int64_t row_stride = (int64_t)p.hkv * D;
    const uint16_t* kbase = p.k + (int64_t)kvh * D;
    const int lrow = lane >> 3, lchunk = lane & 7;
    uint4 kr[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const uint32_t t = t0 + lrow + 8 * (j / CPL);
        const uint32_t tc = t < L ? t : L - 1;
        kr[j] = ldg16(kbase + (int64_t)tc * row_stride + 8 * (lchunk + 8 * (j % CPL)));
    }
    bf16x8_t qb[NLD];
    {
        const uint16_t* qrow = p.q + (int64_t)(h0 + (has ? n : 0)) * D + 8 * g;
#pragma unroll
        for (int i = 0; i < NLD; ++i) {
            uint4 x = ldg16(qrow + 32 * i);
            if (!has) x = make_uint4(0, 0, 0, 0);
            qb[i] = as_bf16x8(x);
        }
    }
    const float2 st = has ? stash_get(o + (int64_t)(h0 + n) * D) : make_float2(0.0f, 0.0f);
    uint16_t* vs = s_tile[wave];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int row = lrow + 8 * (j / CPL), chunk = lchunk + 8 * (j % CPL);
        *reinterpret_cast<uint4*>(vs + row * D + 8 * (chunk ^ vt_swz<D>(row))) = kr[j];
    }
    f32x4_t s4[2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
        const int row = 16 * tt + n;
        s4[tt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int i = 0; i < NLD; ++i)
            s4[tt] = mfma16x16x32(as_bf16x8(*reinterpret_cast<const uint4*>(
                                      vs + row * D + 8 * ((4 * i + g) ^ vt_swz<D>(row)))),
                                  qb[i], s4[tt]);
    }
    if (has) {
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t t = t0 + 16 * tt + 4 * g + r;
                if (t < msl)
                    srow[t] = t < L ? __builtin_amdgcn_exp2f(fmaf(s4[tt][r], scale_log2, -st.x)) * st.y
                                    : 0.0f;
            }
    }
}

__global__ __launch_bounds__(256) void decode_compat_out_kernel(const float* o_buffer, uint16_t* o,
                                                                uint32_t n) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) o[i] = f32_to_bf16(o_buffer[i]);
}

}  // namespace

uint32_t decode_head_groups(uint32_t group) {
    return (group + kDecMaxHeads - 1) / kDecMaxHeads;
}

uint32_t decode_max_splits() { return kMaxSplits; }


uint32_t decode_default_splits(uint32_t batch, uint32_t hq, uint32_t hkv, uint32_t d,
                               uint32_t seq_len) {
    const uint32_t group = hq / hkv;
    const uint64_t wgs_per_split = (uint64_t)batch * hkv * decode_head_groups(group);
    const uint64_t slots = split_slots(d);
    uint64_t s = slots / wgs_per_split;  // one round of resident workgroups
    const uint64_t max_s = ((uint64_t)seq_len + kDecIterRows - 1) / kDecIterRows;
    if (s > max_s) s = max_s;
    if (s > kMaxSplits) s = kMaxSplits;
    if (s < 1) s = 1;
    return (uint32_t)s;
}

hipError_t launch_decode_split(const DecodeProblem& p, const DecodePartials& part,
                               hipStream_t stream) {
    if (p.d == 64) return launch_split_t<64>(p, part, stream);
    return launch_split_t<128>(p, part, stream);
}

hipError_t launch_decode_split_compat(const DecodeProblem& p, const DecodePartials& part,
                                      hipStream_t stream) {
    const dim3 grid(p.splits, p.hkv * decode_head_groups(p.hq / p.hkv), 1);
    const float sl2 = kLog2e / sqrtf((float)p.d);
    if (p.d == 64)
        hipLaunchKernelGGL((decode_split_compat_kernel<64>), grid, dim3(256), 0, stream, p, part, sl2);
    else
        hipLaunchKernelGGL((decode_split_compat_kernel<128>), grid, dim3(256), 0, stream, p, part, sl2);
    return hipGetLastError();
}

hipError_t launch_decode_split_prologue(const DecodeProblem& p, const DecodePartials& part,
                                        const DecodePrologue& pro, hipStream_t stream) {
    if (p.batch != 1 || p.len_mode != kLenDevice) return hipErrorInvalidValue;
    if (p.d == 64) return launch_split_pro_t<64>(p, part, pro, stream);
    return launch_split_pro_t<128>(p, part, pro, stream);
}

hipError_t launch_decode_combine(const DecodeProblem& p, const DecodePartials& part, uint16_t* o,
                                 hipStream_t stream, float* o_f32, bool aligned8) {
    const uint32_t heads = p.batch * p.hq;
    // A single split may keep its partial inside the pair's own output rows
    // (the reference contract with short score rows): only the per-pair
    // kernel, which reads everything before it writes, handles that.
    if (heads < kSlicedCombineBelowPairs && p.splits > 1) {
        const dim3 grid(heads, p.d / kSliceDims), block(kSliceDims * kSliceGroups);
        if (p.d == 64)
            hipLaunchKernelGGL((decode_combine_sliced_kernel<64>), grid, block, 0, stream, part,
                               p.splits, o, o_f32);
        else
            hipLaunchKernelGGL((decode_combine_sliced_kernel<128>), grid, block, 0, stream, part,
                               p.splits, o, o_f32);
        return hipGetLastError();
    }
    // One wave per eight splits (one round of loads each), up to 16 waves.
    uint32_t waves = (p.splits + 7) / 8;
    if (waves > kCombineMaxWaves) waves = kCombineMaxWaves;
    if (waves < 1) waves = 1;
    const dim3 grid(heads), block(64 * waves);
    if (p.d == 64)
        hipLaunchKernelGGL((decode_combine_kernel<64, false>), grid, block, 0, stream, part,
                           p.splits, o, o_f32);
    else if (aligned8)
        hipLaunchKernelGGL((decode_combine_kernel<128, true>), grid, block, 0, stream, part,
                           p.splits, o, o_f32);
    else
        hipLaunchKernelGGL((decode_combine_kernel<128, false>), grid, block, 0, stream, part,
                           p.splits, o, o_f32);
    return hipGetLastError();
}

hipError_t launch_decode_finalize_compat(const DecodeProblem& p, const DecodePartials& part,
                                         float* score, uint32_t msl, float* o_buffer,
                                         uint16_t* o, hipStream_t stream) {
    const dim3 grid(p.hq);
    const float sl2 = kLog2e / sqrtf((float)p.d);
    if (p.splits >= 2) {
        // Partials in the score rows: merge, score pass, O (see the kernels).
        if (p.d == 64)
            hipLaunchKernelGGL(decode_compat_merge_kernel<64>, grid, dim3(kCombineThreads), 0,
                               stream, p, part, o_buffer, o);
        else
            hipLaunchKernelGGL(decode_compat_merge_kernel<128>, grid, dim3(kCombineThreads), 0,
                               stream, p, part, o_buffer, o);
        const dim3 sgrid((msl + kDecIterRows - 1) / kDecIterRows,
                         p.hkv * decode_head_groups(p.hq / p.hkv));
        if (p.d == 64)
            hipLaunchKernelGGL(decode_compat_score_kernel<64>, sgrid, dim3(64 * kDecWaves), 0, stream,
                               p, score, msl, o, sl2);
        else
            hipLaunchKernelGGL(decode_compat_score_kernel<128>, sgrid, dim3(64 * kDecWaves), 0, stream,
                               p, score, msl, o, sl2);
        const uint32_t n = p.hq * p.d;
        hipLaunchKernelGGL(decode_compat_out_kernel, dim3((n + 255) / 256), dim3(256), 0, stream,
                           o_buffer, o, n);
        return hipGetLastError();
    }
    if (p.d == 64)
        hipLaunchKernelGGL(decode_finalize_compat_kernel<64>, grid, dim3(kCombineThreads), 0,
                           stream, p, part, score, msl, o_buffer, o, sl2);
    else
        hipLaunchKernelGGL(decode_finalize_compat_kernel<128>, grid, dim3(kCombineThreads), 0,
                           stream, p, part, score, msl, o_buffer, o, sl2);
    return hipGetLastError();
}

}  // namespace tiattn
