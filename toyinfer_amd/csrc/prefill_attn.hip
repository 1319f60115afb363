// Causal GQA prefill attention for gfx950 (bf16 MFMA, fp32 online softmax).
//
// Replaces flash_attention_v1_bf16_kernel (src/prefill.cu:224-379), which
// runs scalar fp32 dots out of LDS, re-reads every K/V tile per query head
// and visits all ceil(S/32) tiles whatever the causal mask.  Here:
//
// * One workgroup = 4 waves = 128 query rows (32 per wave) of one q-head.
//   Workgroups of the same KV head are launched on the same XCD (block id
//   % Hkv picks the KV head, and the hardware deals block ids round-robin
//   over the 8 XCDs), so a K/V tile fetched into one XCD's L2 serves every
//   q-head of its group; the heaviest (last) query tiles are launched first.
// * Per 64-key tile: S^T = K Q^T on v_mfma_f32_32x32x16_bf16 (A = K from
//   LDS, B = Q^T held in registers for the whole kernel).  In the result
//   lane (q = lane%32, half = lane/32) holds 32 keys of query q, so the row
//   max and row sum are in-lane plus one lane^32 exchange.
// * O^T += V^T P^T on the same MFMA: B = P^T is exactly the lane's own
//   probabilities (converted to bf16 in place); A = V^T comes from the
//   row-major V tile in LDS through ds_read_b64_tr_b16, which transposes
//   16-bit elements across each 16-lane group (source lane s addresses key
//   row base + s/4, dims d0 + 4*(s%4); lane i receives keys base..base+3 of
//   dim d0 + i).  The output lane again owns one query row, so the running
//   rescale is in-lane.
// * The exponentials are taken against a running reference (0 at first)
//   that moves only when a tile's probabilities would leave range: then the
//   tile's row maximum is computed, a row's first tile takes it, and later
//   tiles move the reference up by more than 2^8 only.  The sum and output
//   share the reference, so the result does not depend on it; fully masked
//   tiles past the diagonal are never visited.
// * K and V tiles are double-buffered in LDS: the next tile's global loads
//   (buffer loads whose range check returns zeros past row S-1) are in
//   flight while the current tile computes.  LDS rows are padded (K: D+8,
//   V: D+32 elements) so that each MFMA-operand read pattern hits distinct
//   banks and every LDS address is a per-lane constant plus an immediate.
//
// Optional fused prologue (Qwen3, src/transformer.cpp:380-391): Q rows are
// RMS-normalised with gamma, rounded to bf16, rotated (RoPE at position =
// token) and rounded again while they are loaded into registers.
#include <math.h>

#include "common.hpp"
#include "kernels.hpp"

namespace tiattn {
namespace {

constexpr int kPfThreads = 256;
constexpr int kPfBM = 128;  // query rows per workgroup
constexpr int kPfBN = 64;   // keys per tile
constexpr float kRescaleThreshold = 8.0f;
constexpr float kMassMax = 0x1p64f;   // largest tile row-sum share a lane may take without a rescale
constexpr float kMassMin = 0x1p-64f;  // smallest row mass after a tile without a new reference

typedef short v4i16_t __attribute__((ext_vector_type(4)));

template <int D>
struct PfShape {
    static constexpr int CPR = D / 8;                           // 16-byte chunks per row
    static constexpr int PK = D + 8;                            // K row pitch (elements)
    static constexpr int PV = D + 32;                           // V row pitch (elements)
    static constexpr int K_ELEMS = kPfBN * PK;
    static constexpr int V_ELEMS = kPfBN * PV;
    static constexpr int LOADS = kPfBN * D / 8 / kPfThreads;    // uint4 per thread per tile
    static constexpr int ROWS_PER_LOAD = kPfThreads / CPR;      // rows covered by one load step
    static constexpr int KSTEPS = D / 16;                       // QK MFMA k-steps
    static constexpr int DBLK = D / 32;                         // PV output d-blocks
};

// 128-row kernel tiles: unpadded rows of D bf16, 16-byte chunks XOR-swizzled
// per row so that the MFMA operand reads are bank-conflict free, filled by
// buffer loads that write LDS directly (each instruction fills 1 KiB: 64
// lanes x 16 bytes in lane order, so a lane loads the global chunk that
// belongs at its LDS slot).
//   K rows (A operand reads): chunk c at c ^ (row mod D/8).
//   V rows (transposing reads, 4 rows x 64 bytes per half-wave at D = 128):
//   chunk c at c ^ 4*(row & 3) (D = 128), c ^ 2*(row & 3) (D = 64).
// With these maps, and the O staging described at the output stores,
// SQ_LDS_BANK_CONFLICT reads 0 per launch for the 128-row kernels at
// S=8192, 32/8 heads (the earlier c ^ (row & 7) / c ^ 2*(row & 3) gave
// 6.8e7 cycles).
template <int D, int NW = kPfThreads / 64>
struct DmaShape {
    static constexpr int CPR = D / 8;
    static constexpr int TILE_ELEMS = kPfBN * D;
    static constexpr int BLOCKS = kPfBN * D * 2 / 1024;        // 1 KiB blocks per tile and tensor
    static constexpr int BLOCKS_PER_WAVE = BLOCKS / NW;        // NW waves fill a tile
    static constexpr int KSTEPS = D / 16;
    static constexpr int DBLK = D / 32;
};
template <int D>
__device__ __forceinline__ int k_swz(int row) { return row & (D / 8 - 1); }
template <int D>
__device__ __forceinline__ int v_swz(int row) { return D == 128 ? 4 * (row & 3) : 2 * (row & 3); }

// This lane's byte offsets, within a tile, of the global chunks it loads
// into its LDS slots (K and V maps), for each of the wave's 1 KiB blocks
// (blocks wave, wave + NW, ... of a tile filled by NW waves).
template <int D, int NW>
struct DmaOffsets {
    uint32_t k[DmaShape<D, NW>::BLOCKS_PER_WAVE];
    uint32_t v[DmaShape<D, NW>::BLOCKS_PER_WAVE];
};

template <int D, int NW>
__device__ __forceinline__ DmaOffsets<D, NW> dma_offsets(uint32_t row_bytes, int wave, int lane) {
    using P = DmaShape<D, NW>;
    DmaOffsets<D, NW> r;
#pragma unroll
    for (int j = 0; j < P::BLOCKS_PER_WAVE; ++j) {
        const int slot = 64 * (wave + NW * j) + lane;  // 16-byte slot within the tile
        const int row = slot / P::CPR, phys = slot % P::CPR;
        r.k[j] = row * row_bytes + 16 * (phys ^ k_swz<D>(row));
        r.v[j] = row * row_bytes + 16 * (phys ^ v_swz<D>(row));
    }
    return r;
}

// Issue this wave's share of the tile at byte `tile_off` (K and V) into LDS
// tiles sk, sv.  The buffer resources are rebased at the tile (scalar
// arithmetic; the range check then still covers every byte past row S-1,
// which the scalar offset operand would escape), `wave` is a scalar (the
// LDS destination, M0, is then a scalar sum), and the per-lane offsets are
// loop invariants: a tile's issue costs no vector instructions.
template <int D, int NW>
__device__ __forceinline__ void dma_tile(const uint16_t* k_head, const uint16_t* v_head, uint32_t kv_bytes,
                                         const uint32_t* offk, const uint32_t* offv, int wave, uint32_t tile_off,
                                         uint16_t* sk, uint16_t* sv) {
    using P = DmaShape<D, NW>;
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(reinterpret_cast<const char*>(k_head) + tile_off, kv_bytes - tile_off);
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(reinterpret_cast<const char*>(v_head) + tile_off, kv_bytes - tile_off);
#pragma unroll
    for (int j = 0; j < P::BLOCKS_PER_WAVE; ++j) {
        const int blk = wave + NW * j;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (__attribute__((address_space(3))) void*)(sk + 512 * blk), 16, offk[j], 0, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (__attribute__((address_space(3))) void*)(sv + 512 * blk), 16, offv[j], 0, 0, 0);
    }
}

template <int D>
struct TileRegs {
    uint4 k[PfShape<D>::LOADS];
    uint4 v[PfShape<D>::LOADS];
};

__device__ __forceinline__ v4i16_t ds_read_tr16(const uint16_t* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) v4i16_t*)(p));
}

// Tile starting at byte `tile_off` of K and V into registers; voff is this
// thread's byte offset of its first chunk within a tile.
template <int D>
__device__ __forceinline__ void load_tile(TileRegs<D>& r, __amdgpu_buffer_rsrc_t rk,
                                          __amdgpu_buffer_rsrc_t rv, uint32_t voff,
                                          uint32_t row_bytes, uint32_t tile_off) {
    using P = PfShape<D>;
#pragma unroll
    for (int it = 0; it < P::LOADS; ++it) {
        const uint32_t o = tile_off + voff + it * P::ROWS_PER_LOAD * row_bytes;
        r.k[it] = buf_load16(rk, o);
        r.v[it] = buf_load16(rv, o);
    }
}


template <int D>
__device__ __forceinline__ void store_tile(const TileRegs<D>& r, uint16_t* sk, uint16_t* sv) {
    using P = PfShape<D>;
    const int tid = threadIdx.x;
    const int row = tid / P::CPR, c = tid % P::CPR;
#pragma unroll
    for (int it = 0; it < P::LOADS; ++it) {
        const int rr = row + it * P::ROWS_PER_LOAD;
        *reinterpret_cast<uint4*>(sk + rr * P::PK + 8 * c) = r.k[it];
        *reinterpret_cast<uint4*>(sv + rr * P::PV + 8 * c) = r.v[it];
    }
}

// Q^T fragment of this lane: query row qq, dims {ks*16 + 8*kg + j}.  With
// FUSED, applies RMSNorm(gamma) -> bf16 -> RoPE(position qq) -> bf16.
template <int D, bool FUSED>
__device__ __forceinline__ void load_q(bf16x8_t (&qf)[PfShape<D>::KSTEPS], const PrefillProblem& p,
                                       uint32_t qq, uint32_t h, int kg) {
    constexpr int KS = PfShape<D>::KSTEPS;
    uint4 raw[KS];
    const uint32_t qc = qq < p.s ? qq : p.s - 1;
    const uint16_t* qrow = p.q + ((int64_t)qc * p.hq + h) * D + 8 * kg;
#pragma unroll
    // Q is read once: the non-temporal hint keeps it from displacing the
    // K/V tiles that every query tile of the KV head re-reads from L2.
    for (int ks = 0; ks < KS; ++ks) raw[ks] = ldg16_nt(qrow + ks * 16);
    if constexpr (!FUSED) {
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) qf[ks] = as_bf16x8(raw[ks]);  // rows past S: row S-1, never stored
    } else {
#pragma clang fp contract(off)
        // gamma and the (cos, sin) pairs of this row go out with the Q loads,
        // before anything waits on Q.  Rows past S read row S-1 (unused).
        const float4* rope = reinterpret_cast<const float4*>(p.rope + (int64_t)qc * D);
        uint4 gam[KS];
        float4 cs[KS / 2][4];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) gam[ks] = ldg16(p.q_gamma + ks * 16 + 8 * kg);
#pragma unroll
        for (int ks = 0; ks < KS / 2; ++ks)
#pragma unroll
            for (int e = 0; e < 4; ++e) cs[ks][e] = rope[(ks * 16 + 8 * kg) / 2 + e];
        // Keep every load above ahead of the first use of Q.
        __builtin_amdgcn_sched_barrier(0);
        if (qq >= p.s) {
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) raw[ks] = make_uint4(0, 0, 0, 0);
        }
        float ss = 0.0f;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t w = word_of(raw[ks], e);
                const float a = bf16_lo(w), b = bf16_hi(w);
                ss += a * a;
                ss += b * b;
            }
        ss = xor32_sum(ss);
        const float inv = 1.0f / sqrtf(ss / (float)D + p.eps);
        // Chunk ks (dims < D/2) pairs with chunk ks + KS/2 (dims + D/2).
#pragma unroll
        for (int ks = 0; ks < KS / 2; ++ks) {
            const uint4 g_re = gam[ks];
            const uint4 g_im = gam[ks + KS / 2];
            const float4* cs4 = cs[ks];
            uint32_t o_re[4], o_im[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t xr = word_of(raw[ks], e), xi = word_of(raw[ks + KS / 2], e);
                const uint32_t gr = word_of(g_re, e), gi = word_of(g_im, e);
                float r2[2], i2[2];
#pragma unroll
                for (int hlf = 0; hlf < 2; ++hlf) {
                    const float xre = hlf ? bf16_hi(xr) : bf16_lo(xr);
                    const float xim = hlf ? bf16_hi(xi) : bf16_lo(xi);
                    const float gre = hlf ? bf16_hi(gr) : bf16_lo(gr);
                    const float gim = hlf ? bf16_hi(gi) : bf16_lo(gi);
                    const float re = bf16_lo(pack_bf16x2(xre * inv * gre, 0.0f));
                    const float im = bf16_lo(pack_bf16x2(xim * inv * gim, 0.0f));
                    const float cs = hlf ? cs4[e].z : cs4[e].x;
                    const float sn = hlf ? cs4[e].w : cs4[e].y;
                    r2[hlf] = cs * re - sn * im;
                    i2[hlf] = cs * im + sn * re;
                }
                o_re[e] = pack_bf16x2(r2[0], r2[1]);
                o_im[e] = pack_bf16x2(i2[0], i2[1]);
            }
            qf[ks] = as_bf16x8(make_uint4(o_re[0], o_re[1], o_re[2], o_re[3]));
            qf[ks + KS / 2] = as_bf16x8(make_uint4(o_im[0], o_im[1], o_im[2], o_im[3]));
        }
    }
}

// PAIR: eight waves, the two query heads of a GQA pair over the same 128
// rows (waves w and w + 4, which share a SIMD, take head 2j and 2j + 1 of
// pair j), so that one K/V tile in LDS serves both: half the DMA and L2
// reads per head; one workgroup per CU instead of two.
template <int D, bool FUSED, bool PAIR>
__global__ __launch_bounds__(PAIR ? 512 : kPfThreads, PAIR ? 1 : 2) void prefill_kernel(PrefillProblem p, float scale_log2) {
    constexpr int NW = PAIR ? 8 : kPfThreads / 64;
    using P = DmaShape<D, NW>;
    // Four separate arrays (not one indexed by buffer): the compiler can then
    // tell the tile being computed from the one the LDS DMA is filling, and
    // does not make the operand reads wait for the in-flight loads.
    __shared__ __align__(1024) uint16_t s_k0[P::TILE_ELEMS];
    __shared__ __align__(1024) uint16_t s_k1[P::TILE_ELEMS];
    __shared__ __align__(1024) uint16_t s_v0[P::TILE_ELEMS];
    __shared__ __align__(1024) uint16_t s_v1[P::TILE_ELEMS];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int ql = lane & 31, kg = lane >> 5;
    const uint32_t group = p.hq / p.hkv;
    const uint32_t n_qtiles = (p.s + kPfBM - 1) / kPfBM;
    const uint32_t bid = blockIdx.x;
    const uint32_t kvh = bid % p.hkv;
    const uint32_t r = bid / p.hkv;
    const uint32_t hpw = PAIR ? 2 : 1;  // heads per workgroup
    const uint32_t h = kvh * group + hpw * (r % (group / hpw)) + (PAIR ? wave >> 2 : 0);
    const uint32_t qt = n_qtiles - 1 - r / (group / hpw);

    const uint32_t q_end = min(p.s, (qt + 1) * kPfBM);
    const uint32_t n_tiles = (q_end + kPfBN - 1) / kPfBN;
    const uint32_t q0 = qt * kPfBM + (wave & 3) * 32;
    const uint32_t qq = q0 + ql;
    const uint32_t wave_tiles = q0 < p.s ? (min(q0 + 31, p.s - 1) / kPfBN + 1) : 0;
    // K/V rows of this KV head: row t at byte t*row_bytes from the head's
    // first element; the buffer range ends after row S-1's D elements.
    const uint32_t row_bytes = p.hkv * D * 2;
    const uint32_t kv_bytes = (p.s - 1) * row_bytes + D * 2;
    const uint16_t* k_head = p.k + (int64_t)kvh * D;
    const uint16_t* v_head = p.v + (int64_t)kvh * D;

    const int swave = __builtin_amdgcn_readfirstlane(wave);
    const DmaOffsets<D, NW> doff = dma_offsets<D, NW>(row_bytes, swave, lane);
    dma_tile<D, NW>(k_head, v_head, kv_bytes, doff.k, doff.v, swave, 0, s_k0, s_v0);
    bf16x8_t qf[P::KSTEPS];
    load_q<D, FUSED>(qf, p, qq, h, kg);

    f32x16_t oacc[P::DBLK];
#pragma unroll
    for (int db = 0; db < P::DBLK; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) oacc[db][i] = 0.0f;
    float m_run = 0.0f, l_run = 0.0f;

    // Operand read offsets (elements) within a tile.  K: row ql (and +32),
    // chunk 2*ks + kg; V^T (transposing read): rows 4*kg + s16/4 (+16*tt, +8),
    // dims 32*db + 16*(g16 & 1) + 4*(s16 & 3).
    const int s16 = lane & 15, g16 = lane >> 4;
    int k_off[P::KSTEPS], v_off[P::DBLK];
#pragma unroll
    for (int ks = 0; ks < P::KSTEPS; ++ks) k_off[ks] = ql * D + 8 * ((2 * ks + kg) ^ k_swz<D>(ql));
    {
        const int vrow = 4 * kg + (s16 >> 2);
#pragma unroll
        for (int db = 0; db < P::DBLK; ++db) {
            const int c = 4 * db + 2 * (g16 & 1) + ((s16 & 3) >> 1);
            v_off[db] = vrow * D + 8 * (c ^ v_swz<D>(vrow)) + 4 * (s16 & 1);
        }
    }
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);  // the first tile (and Q)
    __syncthreads();

    // Tile t computes from (kb, vb) while tile t+1 streams into (kn, vn),
    // whose last readers passed the previous barrier.
    auto step = [&](uint32_t t, const uint16_t* kb, const uint16_t* vb, uint16_t* kn,
                    uint16_t* vn) __attribute__((always_inline)) {
        if (t + 1 < n_tiles) dma_tile<D, NW>(k_head, v_head, kv_bytes, doff.k, doff.v, swave, (t + 1) * kPfBN * row_bytes, kn, vn);

        if (t < wave_tiles) {
            const uint32_t n0 = t * kPfBN;
            f32x16_t st0, st1;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                st0[i] = 0.0f;
                st1[i] = 0.0f;
            }
            // K operands one k-step ahead of their MFMAs.
            uint4 ka[2][2];
            ka[0][0] = *reinterpret_cast<const uint4*>(kb + k_off[0]);
            ka[0][1] = *reinterpret_cast<const uint4*>(kb + 32 * D + k_off[0]);
#pragma unroll
            for (int ks = 0; ks < P::KSTEPS; ++ks) {
                if (ks + 1 < P::KSTEPS) {
                    ka[(ks + 1) & 1][0] = *reinterpret_cast<const uint4*>(kb + k_off[ks + 1]);
                    ka[(ks + 1) & 1][1] = *reinterpret_cast<const uint4*>(kb + 32 * D + k_off[ks + 1]);
                }
                st0 = mfma32x32x16(as_bf16x8(ka[ks & 1][0]), qf[ks], st0);
                st1 = mfma32x32x16(as_bf16x8(ka[ks & 1][1]), qf[ks], st1);
            }
            // Keep the reads a k-step ahead (the scheduler would otherwise
            // pair each read with its MFMA and expose the LDS latency).
            __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
            for (int ks = 0; ks + 2 < P::KSTEPS; ++ks) {
                __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
            // Causal mask: lane holds keys n0 + 32*blk + 8*(i/4) + 4*kg + i%4.
            if (n0 + kPfBN - 1 > q0) {
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const uint32_t key = n0 + 8 * (i / 4) + 4 * kg + (i % 4);
                    if (key > qq) st0[i] = -INFINITY;
                    if (key + 32 > qq) st1[i] = -INFINITY;
                }
            }
            // Probabilities against the running reference m_run (a row
            // constant, 0 before the first tile): P = bf16(2^(s*c - m_run)),
            // and this lane's share of the tile's row sum, taken from the
            // bf16 values the P.V product uses.  The quotient O / l does not
            // depend on m_run; it only has to keep P finite and the row's
            // mass clear of underflow, so the tile's row maximum is computed
            // only for a tile that fails that check.
            bf16x8_t pf[4];
            auto probs = [&](float mref) __attribute__((always_inline)) {
#pragma unroll
                for (int tt = 0; tt < 4; ++tt) {
                    const f32x16_t& src = tt < 2 ? st0 : st1;
                    const int o8 = 8 * (tt & 1);
                    float e[8];
#pragma unroll
                    for (int j = 0; j < 8; ++j)
                        e[j] = __builtin_amdgcn_exp2f(fmaf(src[o8 + j], scale_log2, -mref));
                    pf[tt] = as_bf16x8(make_uint4(pack_bf16x2(e[0], e[1]), pack_bf16x2(e[2], e[3]),
                                                  pack_bf16x2(e[4], e[5]), pack_bf16x2(e[6], e[7])));
                }
                return sum_bf16x8(__builtin_bit_cast(uint4, pf[0]),
                                  sum_bf16x8(__builtin_bit_cast(uint4, pf[1]), 0.0f)) +
                       sum_bf16x8(__builtin_bit_cast(uint4, pf[2]),
                                  sum_bf16x8(__builtin_bit_cast(uint4, pf[3]), 0.0f));
            };
            float ts = probs(m_run);
            // The check: every lane's share at most 2^64 (a NaN fails too)
            // and the row's mass after this tile at least 2^-64.
            const float row_mass = xor32_sum(l_run + ts);
            if (__any(!(ts <= kMassMax) || !(row_mass >= kMassMin))) {
                // The tile's row maximum (two chains of three-input maxima).
                float ma = fmaxf(st0[0], st0[1]), mb = fmaxf(st1[0], st1[1]);
#pragma unroll
                for (int i = 2; i < 16; i += 2) {
                    ma = fmaxf(fmaxf(ma, st0[i]), st0[i + 1]);
                    mb = fmaxf(fmaxf(mb, st1[i]), st1[i + 1]);
                }
                const float mt = xor32_max(fmaxf(ma, mb)) * scale_log2;
                // A row's first tile (no mass yet) takes its maximum as the
                // reference; later tiles move it only up, and only by more
                // than 2^8, rescaling what has accumulated.
                const bool first = xor32_sum(l_run) == 0.0f;
                const bool need = !first && mt > m_run + kRescaleThreshold;
                if (first) m_run = mt;
                if (__any(need)) {
                    float alpha = 1.0f;
                    if (need) {
                        alpha = __builtin_amdgcn_exp2f(m_run - mt);
                        m_run = mt;
                    }
                    l_run *= alpha;
#pragma unroll
                    for (int db = 0; db < P::DBLK; ++db)
#pragma unroll
                        for (int i = 0; i < 16; ++i) oacc[db][i] *= alpha;
                }
                ts = probs(m_run);
            }
            l_run += ts;
            // A = V^T for k-step tt: lane group G = lane/16 (kg = G/2) reads key
            // rows 16*tt + 4*kg + s/4 (+8 for the second half) at dims
            // 32*db + 16*(G%2) + 4*(s%4), s = lane%16.  The d-blocks are
            // independent accumulators, so each k-step issues DBLK
            // independent MFMAs, their operands read one k-step ahead.
            uint4 va[2][P::DBLK];
            auto read_v = [&](int tt, uint4 (&a)[P::DBLK]) __attribute__((always_inline)) {
#pragma unroll
                for (int db = 0; db < P::DBLK; ++db) {
                    const v4i16_t lo = ds_read_tr16(vb + v_off[db] + 16 * tt * D);
                    const v4i16_t hi = ds_read_tr16(vb + v_off[db] + (16 * tt + 8) * D);
                    a[db] = make_uint4(__builtin_bit_cast(uint2, lo).x, __builtin_bit_cast(uint2, lo).y,
                                       __builtin_bit_cast(uint2, hi).x, __builtin_bit_cast(uint2, hi).y);
                }
            };
            read_v(0, va[0]);
#pragma unroll
            for (int tt = 0; tt < 4; ++tt) {
                if (tt + 1 < 4) read_v(tt + 1, va[(tt + 1) & 1]);
#pragma unroll
                for (int db = 0; db < P::DBLK; ++db)
                    oacc[db] = mfma32x32x16(as_bf16x8(va[tt & 1][db]), pf[tt], oacc[db]);
            }
            __builtin_amdgcn_sched_group_barrier(0x100, 4 * P::DBLK, 0);
#pragma unroll
            for (int tt = 0; tt < 3; ++tt) {
                __builtin_amdgcn_sched_group_barrier(0x008, P::DBLK, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 2 * P::DBLK, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, P::DBLK, 0);
        }

        // This wave's tile loads, then every wave.  The wait is explicit: the
        // compiler's tracking of loads that write LDS is not relied on.
        __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
        __syncthreads();
    };
    for (uint32_t t = 0; t < n_tiles; t += 2) {
        step(t, s_k0, s_v0, s_k1, s_v1);
        if (t + 1 < n_tiles) step(t + 1, s_k1, s_v1, s_k0, s_v0);
    }

    // O goes out through LDS, so that each store instruction writes whole
    // 256-byte rows (16 lanes per row) with the non-temporal hint: O is not
    // read again, and the per-lane 8-byte pieces would otherwise occupy L2
    // lines beside the K/V tiles the other query tiles of this KV head
    // re-read.  The tile buffers are free: every wave passed the last
    // step's barrier.  Each wave uses its own 32 x D region (16-byte chunk c
    // of row r at c ^ (r mod D/8)) and reads back only what it wrote (LDS
    // operations of a wave complete in order).  The 8-byte stores go to the
    // banks 16 lanes at a time (128 bytes, 32 banks): lanes whose chunk
    // positions differ by 8 (D = 128) or whose rows differ by 8 (D = 64)
    // would meet on the same banks, so those with bit 3 of the position
    // (D = 128) or of the row (D = 64) set store the two 8-byte halves of
    // the chunk swapped, and the read-back swaps them again.
    const float l_tot = xor32_sum(l_run);  // all lanes take part in the exchange
    {
        constexpr int CPR = D / 8;
        const float inv = 1.0f / l_tot;  // (rows past S: not stored)
        uint16_t* so = ((wave >> 1) == 0 ? s_k0 : (wave >> 1) == 1 ? s_k1 : (wave >> 1) == 2 ? s_v0 : s_v1) +
                       (wave & 1) * 32 * D;
        // Whether row r keeps the halves of the chunk at position pos swapped.
        auto swapped = [](int r, int pos) { return ((D == 128 ? pos : r) >> 3) & 1; };
#pragma unroll
        for (int db = 0; db < P::DBLK; ++db)
#pragma unroll
            for (int i4 = 0; i4 < 4; ++i4) {
                uint2 w;
                w.x = pack_bf16x2(oacc[db][4 * i4] * inv, oacc[db][4 * i4 + 1] * inv);
                w.y = pack_bf16x2(oacc[db][4 * i4 + 2] * inv, oacc[db][4 * i4 + 3] * inv);
                const int pos = (4 * db + i4) ^ (ql & (CPR - 1));
                *reinterpret_cast<uint2*>(so + ql * D + 8 * pos + 4 * (kg ^ swapped(ql, pos))) = w;
            }
#pragma unroll
        for (int j = 0; j < 32 * CPR / 64; ++j) {
            const int f = 64 * j + lane, row = f / CPR, c = f % CPR;
            const int pos = c ^ (row & (CPR - 1));
            uint4 v = *reinterpret_cast<const uint4*>(so + row * D + 8 * pos);
            if (swapped(row, pos)) v = make_uint4(v.z, v.w, v.x, v.y);
            const uint32_t q = q0 + row;
            if (q < p.s) stg16_nt(p.o + ((int64_t)q * p.hq + h) * D + 8 * c, v);
        }
    }
}

// ---------------------------------------------------------------------------
// Short-sequence variant: intra-workgroup split over keys.
//
// With few query tiles (S=1371 gives ceil(S/128) x Hq = 176 workgroups for
// 256 CUs) the kernel above is bound by its longest workgroup, which walks
// every key tile of the last rows alone.  Here a workgroup takes 32 query
// rows of one head and its four waves split that row block's key tiles (32
// keys each) round-robin; every wave streams its own tiles through a
// private LDS region (register prefetch of its next tile, no barriers), and
// the four partial (m, l, O) are merged through LDS at the end.
constexpr int kSkBM = 32;
constexpr int kSkBN = 32;

constexpr uint32_t kSkOob = 0xF0000000u;  // a byte offset past any K/V buffer range here

template <int D>
struct SkShape {
    static constexpr int CPR = D / 8;
    static constexpr int PK = D + 8;
    static constexpr int PV = D + 32;
    static constexpr int K_ELEMS = kSkBN * PK;
    static constexpr int WAVE_ELEMS = kSkBN * PK + kSkBN * PV;
    static constexpr int LOADS = kSkBN * D / 8 / 64;  // uint4 per lane per tile
    static constexpr int ROWS_PER_LOAD = 64 / CPR;
    static constexpr int KSTEPS = D / 16;
    static constexpr int DBLK = D / 32;
    static constexpr int OPITCH = D + 4;              // merge buffer pitch (floats, 16-byte rows)
};

// Work item i = (query head, 32-row query tile), heaviest (last) tiles first;
// consecutive items walk the KV heads, so with Hkv = 8 each XCD sees one KV
// head's K/V.
struct SkItem {
    uint32_t h, kvh, q0, n_tiles;
};

__device__ __forceinline__ SkItem sk_item(const PrefillProblem& p, uint32_t i, uint32_t group,
                                          uint32_t n_qt) {
    SkItem it;
    it.kvh = i % p.hkv;
    const uint32_t r = i / p.hkv;
    it.h = it.kvh * group + r % group;
    it.q0 = (n_qt - 1 - r / group) * kSkBM;
    it.n_tiles = (min(p.s, it.q0 + kSkBM) + kSkBN - 1) / kSkBN;
    return it;
}

// Workgroup g of G takes, in round r, item r*G + g on even rounds and, on
// odd ones, the mirror item in reverse order of g's block of eight (g % 8
// kept): the heaviest item of one round pairs with the lightest of the
// next, and a workgroup stays on the KV head (item % Hkv, with Hkv = 8) whose
// K/V its XCD's L2 already holds (workgroups go to the XCDs round-robin).
__device__ __forceinline__ uint32_t sk_item_index(uint32_t round, uint32_t g, uint32_t G) {
    if (!(round & 1)) return round * G + g;
    const uint32_t m = G % 8 == 0 ? (G / 8 - 1 - g / 8) * 8 + g % 8 : G - 1 - g;
    return round * G + m;
}

template <int D, bool FUSED>
__global__ __launch_bounds__(kPfThreads, 2) void prefill_splitkv_kernel(PrefillProblem p,
                                                                        float scale_log2,
                                                                        uint32_t n_items) {
    using P = SkShape<D>;
    constexpr int LDS_TILES = 4 * P::WAVE_ELEMS * 2;
    constexpr int LDS_MERGE = 4 * kSkBM * P::OPITCH * 4;
    static_assert(LDS_MERGE <= LDS_TILES, "merge buffer must fit in the tile buffers");
    __shared__ __align__(16) unsigned char s_raw[LDS_TILES];
    __shared__ float s_ml[4][kSkBM][2];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int ql = lane & 31, kg = lane >> 5;
    const uint32_t group = p.hq / p.hkv;
    const uint32_t n_qt = (p.s + kSkBM - 1) / kSkBM;

    const uint32_t row_bytes = p.hkv * D * 2;
    const uint32_t kv_bytes = (p.s - 1) * row_bytes + D * 2;
    const uint32_t voff = (lane / P::CPR) * row_bytes + (lane % P::CPR) * 16;
    uint16_t* sk = reinterpret_cast<uint16_t*>(s_raw) + wave * P::WAVE_ELEMS;
    uint16_t* sv = sk + P::K_ELEMS;

    uint32_t round = 0;
    SkItem it = sk_item(p, blockIdx.x, group, n_qt);
    __amdgpu_buffer_rsrc_t rk = make_rsrc(p.k + (int64_t)it.kvh * D, kv_bytes);
    __amdgpu_buffer_rsrc_t rv = make_rsrc(p.v + (int64_t)it.kvh * D, kv_bytes);

    uint4 kreg[P::LOADS], vreg[P::LOADS];
    // Tile t of the item's keys; `base` overrides the tile's byte offset (a
    // value past every buffer range makes the loads return zeros without
    // touching memory).
    auto load_k_at = [&](uint32_t base) {
#pragma unroll
        for (int i = 0; i < P::LOADS; ++i)
            kreg[i] = buf_load16(rk, base + voff + i * P::ROWS_PER_LOAD * row_bytes);
    };
    auto load_v_at = [&](uint32_t base) {
#pragma unroll
        for (int i = 0; i < P::LOADS; ++i)
            vreg[i] = buf_load16(rv, base + voff + i * P::ROWS_PER_LOAD * row_bytes);
    };
    auto load_k = [&](uint32_t t) { load_k_at(t * kSkBN * row_bytes); };
    auto load_v = [&](uint32_t t) { load_v_at(t * kSkBN * row_bytes); };
    auto load = [&](uint32_t t) {
        load_k(t);
        load_v(t);
    };
    const int st_row = lane / P::CPR, st_c = lane % P::CPR;  // this lane's chunk of a tile row
    // The first tile's loads go out before anything waits on Q (after the
    // fused prologue, whose loads need the registers, when FUSED).
    bf16x8_t qf[P::KSTEPS];
    if constexpr (FUSED) load_q<D, FUSED>(qf, p, it.q0 + ql, it.h, kg);
    if ((uint32_t)wave < it.n_tiles) load(wave);
    if constexpr (!FUSED) load_q<D, FUSED>(qf, p, it.q0 + ql, it.h, kg);

    while (true) {
        const uint32_t q0 = it.q0, qq = q0 + ql, n_tiles = it.n_tiles;
        f32x16_t oacc[P::DBLK];
#pragma unroll
        for (int db = 0; db < P::DBLK; ++db)
#pragma unroll
            for (int i = 0; i < 16; ++i) oacc[db][i] = 0.0f;
        float m_run = -INFINITY, l_run = 0.0f;

        // Q and the first tile have landed before the loop (the first tile's
        // stores need it anyway).  Without this explicit wait the compiler
        // cannot tell, inside the loop, that Q is no longer in flight, and
        // holds the QK products for the prefetch of the next tile.
        __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
        // Per tile: K is stored (and its next tile requested) first, so the
        // QK operand reads queue behind 8 KB of stores, not 16; V follows
        // while the QK products run.
        for (uint32_t t = wave; t < n_tiles; t += 4) {
#pragma unroll
            for (int i = 0; i < P::LOADS; ++i)
                *reinterpret_cast<uint4*>(sk + (st_row + i * P::ROWS_PER_LOAD) * P::PK + 8 * st_c) = kreg[i];
            // The next tile's loads are unconditional (out of range past the
            // item's last tile), so that the compiler's wait before the next
            // iteration's K stores counts exactly the K loads and leaves the
            // V loads in flight.
            const uint32_t next = t + 4 < n_tiles ? (t + 4) * kSkBN * row_bytes : kSkOob;
            load_k_at(next);
            // Keep the K requests here and the V stores after the QK
            // products: the scheduler would otherwise hoist the V stores
            // (and their wait for V) above both.
            __builtin_amdgcn_sched_barrier(0);
            const uint32_t n0 = t * kSkBN;
            f32x16_t st;
#pragma unroll
            for (int i = 0; i < 16; ++i) st[i] = 0.0f;
            const uint16_t* ka = sk + ql * P::PK + 8 * kg;
#pragma unroll
            for (int ks = 0; ks < P::KSTEPS; ++ks)
                st = mfma32x32x16(as_bf16x8(*reinterpret_cast<const uint4*>(ka + 16 * ks)), qf[ks], st);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < P::LOADS; ++i)
                *reinterpret_cast<uint4*>(sv + (st_row + i * P::ROWS_PER_LOAD) * P::PV + 8 * st_c) = vreg[i];
            load_v_at(next);
            if (n0 + kSkBN - 1 > q0) {
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const uint32_t key = n0 + 8 * (i / 4) + 4 * kg + (i % 4);
                    if (key > qq) st[i] = -INFINITY;
                }
            }
            float ma = fmaxf(st[0], st[1]), mb = fmaxf(st[8], st[9]);
#pragma unroll
            for (int i = 2; i < 8; i += 2) {
                ma = fmaxf(fmaxf(ma, st[i]), st[i + 1]);
                mb = fmaxf(fmaxf(mb, st[i + 8]), st[i + 9]);
            }
            float mx = fmaxf(ma, mb);
            mx = xor32_max(mx);
            const float mt = mx * scale_log2;
            const bool need = mt > m_run + kRescaleThreshold;
            if (__any(need)) {
                float alpha = 1.0f;
                if (need) {
                    alpha = __builtin_amdgcn_exp2f(m_run - mt);
                    m_run = mt;
                }
                l_run *= alpha;
#pragma unroll
                for (int db = 0; db < P::DBLK; ++db)
#pragma unroll
                    for (int i = 0; i < 16; ++i) oacc[db][i] *= alpha;
            }
            const float mref = m_run == -INFINITY ? 0.0f : m_run;
#pragma unroll
            for (int i = 0; i < 16; ++i) st[i] = __builtin_amdgcn_exp2f(fmaf(st[i], scale_log2, -mref));
            bf16x8_t pf[2];
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                const int o8 = 8 * tt;
                pf[tt] = as_bf16x8(make_uint4(pack_bf16x2(st[o8 + 0], st[o8 + 1]),
                                              pack_bf16x2(st[o8 + 2], st[o8 + 3]),
                                              pack_bf16x2(st[o8 + 4], st[o8 + 5]),
                                              pack_bf16x2(st[o8 + 6], st[o8 + 7])));
            }
            l_run += sum_bf16x8(__builtin_bit_cast(uint4, pf[0]),
                                sum_bf16x8(__builtin_bit_cast(uint4, pf[1]), 0.0f));
            const int s16 = lane & 15, grp = lane >> 4;
            const uint16_t* va = sv + (4 * kg + (s16 >> 2)) * P::PV + 16 * (grp & 1) + 4 * (s16 & 3);
#pragma unroll
            for (int db = 0; db < P::DBLK; ++db)
#pragma unroll
                for (int tt = 0; tt < 2; ++tt) {
                    const v4i16_t lo = ds_read_tr16(va + 16 * tt * P::PV + 32 * db);
                    const v4i16_t hi = ds_read_tr16(va + (16 * tt + 8) * P::PV + 32 * db);
                    const uint4 a = make_uint4(__builtin_bit_cast(uint2, lo).x, __builtin_bit_cast(uint2, lo).y,
                                               __builtin_bit_cast(uint2, hi).x, __builtin_bit_cast(uint2, hi).y);
                    oacc[db] = mfma32x32x16(as_bf16x8(a), pf[tt], oacc[db]);
                }
        }

        // The next item's first tile and Q loads go out now and land while
        // this item's partials are merged.  (With FUSED the grid holds every
        // item: its Q prologue would not fit beside the merge's registers.)
        ++round;
        const uint32_t nxt = sk_item_index(round, blockIdx.x, gridDim.x);
        const bool more = !FUSED && nxt < n_items;
        const uint32_t h = it.h;
        if (more) {
            it = sk_item(p, nxt, group, n_qt);
            rk = make_rsrc(p.k + (int64_t)it.kvh * D, kv_bytes);
            rv = make_rsrc(p.v + (int64_t)it.kvh * D, kv_bytes);
            if ((uint32_t)wave < it.n_tiles) load(wave);
            load_q<D, FUSED>(qf, p, it.q0 + ql, it.h, kg);
        }

        // Merge the four waves' partials of the 32 rows.
        const float l_tot = xor32_sum(l_run);
        lds_barrier();  // all waves are done with their tile buffers
        float* s_o = reinterpret_cast<float*>(s_raw);  // [wave][row][OPITCH]
        // Each lane's accumulator values come in runs of four adjacent
        // columns: 16-byte stores; rows 528 bytes apart put a half-wave's
        // stores in distinct bank groups.
#pragma unroll
        for (int db = 0; db < P::DBLK; ++db)
#pragma unroll
            for (int g = 0; g < 4; ++g)
                *reinterpret_cast<float4*>(s_o + (wave * kSkBM + ql) * P::OPITCH + db * 32 + 8 * g + 4 * kg) =
                    make_float4(oacc[db][4 * g], oacc[db][4 * g + 1], oacc[db][4 * g + 2], oacc[db][4 * g + 3]);
        if (kg == 0) {
            s_ml[wave][ql][0] = m_run;
            s_ml[wave][ql][1] = l_tot;
        }
        lds_barrier();
        // Final pass: float4 f = tid + 256 k of the 32 x D/4 output block
        // (row f / (D/4), column group f % (D/4)), so each 16 lanes read 256
        // contiguous bytes of one merge row: no bank conflicts.  Every load is
        // unconditional: a wave that saw no key has o = 0 and weight 0.
        constexpr int C4 = D / 4;
        constexpr int NF = kSkBM * C4 / kPfThreads;
#pragma unroll
        for (int k = 0; k < NF; ++k) {
            const int f = threadIdx.x + kPfThreads * k;
            const int row = f / C4, c4 = f % C4;
            float M = -INFINITY;
#pragma unroll
            for (int w = 0; w < 4; ++w) M = fmaxf(M, s_ml[w][row][0]);
            float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            float den = 0.0f;
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const float mw = s_ml[w][row][0];
                const float wgt = mw == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mw - M);
                den = fmaf(wgt, s_ml[w][row][1], den);
                const float4 x = *reinterpret_cast<const float4*>(s_o + (w * kSkBM + row) * P::OPITCH + 4 * c4);
                acc.x = fmaf(wgt, x.x, acc.x);
                acc.y = fmaf(wgt, x.y, acc.y);
                acc.z = fmaf(wgt, x.z, acc.z);
                acc.w = fmaf(wgt, x.w, acc.w);
            }
            const uint32_t orow_q = q0 + row;
            if (orow_q < p.s) {
                const float inv = 1.0f / den;
                *reinterpret_cast<uint2*>(p.o + ((int64_t)orow_q * p.hq + h) * D + 4 * c4) =
                    make_uint2(pack_bf16x2(acc.x * inv, acc.y * inv), pack_bf16x2(acc.z * inv, acc.w * inv));
            }
        }
        if (!more) break;
        lds_barrier();  // the merge buffer's reads are done before tiles are written again
    }
}

// ---------------------------------------------------------------------------
// Split over keys with both query heads of a GQA pair in one workgroup.
//
// Eight waves take 32 query rows of the two heads 2j, 2j + 1 of pair j of a
// KV head: waves w and w + 4 (which share a SIMD) run heads 2j and 2j + 1
// over the same key tiles, stream w % 4 taking tiles w % 4, w % 4 + 4, ....
// A stream's 32-key K and V tiles reach LDS by buffer loads that write LDS
// (each of its two waves fills half), double-buffered, so one fetch serves
// both heads, no registers stage a tile and no ds_write is issued; one
// barrier per step of four tiles.  After the last step the four streams'
// partials merge in LDS in two exchange rounds in which every wave takes part
// (each then writes a quarter of its head's output), while the next item's
// first tiles and Q are already in flight.
constexpr int kSpThreads = 512;

template <int D>
struct SpShape {
    static constexpr int CPR = D / 8;
    static constexpr int TILE = kSkBN * D;          // elements of one K or V tile
    static constexpr int BLOCKS = TILE * 2 / 1024;  // 1 KiB DMA blocks per tile
    static constexpr int BPW = BLOCKS / 2;          // per wave (two waves per stream)
    static constexpr int STREAM = 2 * TILE;         // K then V
    static constexpr int STAGE = 4 * STREAM;        // the four streams of one buffer
    static constexpr int KSTEPS = D / 16;
    static constexpr int DBLK = D / 32;
};

// Work item i = (KV head i % Hkv, head pair, 32-row block), heaviest (last)
// row blocks first, as sk_item orders them.
struct SpItem {
    uint32_t h0, kvh, q0, n_tiles;
};

__device__ __forceinline__ SpItem sp_item(const PrefillProblem& p, uint32_t i, uint32_t group,
                                          uint32_t n_qt) {
    SpItem it;
    const uint32_t pairs = group / 2;
    it.kvh = i % p.hkv;
    const uint32_t r = i / p.hkv;
    it.h0 = it.kvh * group + 2 * (r % pairs);
    it.q0 = (n_qt - 1 - r / pairs) * kSkBM;
    it.n_tiles = (min(p.s, it.q0 + kSkBM) + kSkBN - 1) / kSkBN;
    return it;
}

// One stream's tile at byte `off` of the KV head's K and V into LDS at sk
// (K) and sk + TILE (V): this wave's blocks sub, sub + 2, ....
template <int D>
__device__ __forceinline__ void sp_dma_tile(const uint16_t* k_head, const uint16_t* v_head,
                                            uint32_t kv_bytes, uint32_t off, const uint32_t* offk,
                                            const uint32_t* offv, int sub, uint16_t* sk) {
    using P = SpShape<D>;
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(reinterpret_cast<const char*>(k_head) + off, kv_bytes - off);
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(reinterpret_cast<const char*>(v_head) + off, kv_bytes - off);
#pragma unroll
    for (int j = 0; j < P::BPW; ++j) {
        const int blk = sub + 2 * j;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (__attribute__((address_space(3))) void*)(sk + 512 * blk), 16, offk[j], 0, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (__attribute__((address_space(3))) void*)(sk + P::TILE + 512 * blk), 16, offv[j], 0, 0, 0);
    }
}

// Workgroup barrier that waits for this wave's LDS operations only, leaving
// its global loads (also those that write LDS) in flight; the memory clobber
// keeps the compiler from moving memory accesses across it.
__device__ __forceinline__ void lds_ops_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// A partner's N float4 (1 KiB apart: lane l at src + 16 l) and its (m, l)
// pair, read from LDS in one asm block that also waits for them.  In asm
// the reads are not LDS accesses to the compiler, which would otherwise make
// them wait for every buffer load writing LDS (the next item's first tiles,
// in flight into the other buffer).
template <int N>
__device__ __forceinline__ float2 sp_read(float4 (&x)[N], const float4* src, const float2* ml, int lane) {
    const uint32_t a = (uint32_t)(size_t)(const __attribute__((address_space(3))) void*)(src + lane);
    const uint32_t b = (uint32_t)(size_t)(const __attribute__((address_space(3))) void*)(ml + lane);
    f32x4_t v[N];
    float2 r;
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    f32x2_t m;
    static_assert(N == 2 || N == 4 || N == 8, "read count");
    if constexpr (N == 2) {
        asm volatile(
            "ds_read_b128 %0, %3\n\t"
            "ds_read_b128 %1, %3 offset:1024\n\t"
            "ds_read_b64 %2, %4\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(v[0]), "=&v"(v[1]), "=&v"(m)
            : "v"(a), "v"(b)
            : "memory");
    } else if constexpr (N == 4) {
        asm volatile(
            "ds_read_b128 %0, %5\n\t"
            "ds_read_b128 %1, %5 offset:1024\n\t"
            "ds_read_b128 %2, %5 offset:2048\n\t"
            "ds_read_b128 %3, %5 offset:3072\n\t"
            "ds_read_b64 %4, %6\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(m)
            : "v"(a), "v"(b)
            : "memory");
    } else {
        asm volatile(
            "ds_read_b128 %0, %9\n\t"
            "ds_read_b128 %1, %9 offset:1024\n\t"
            "ds_read_b128 %2, %9 offset:2048\n\t"
            "ds_read_b128 %3, %9 offset:3072\n\t"
            "ds_read_b128 %4, %9 offset:4096\n\t"
            "ds_read_b128 %5, %9 offset:5120\n\t"
            "ds_read_b128 %6, %9 offset:6144\n\t"
            "ds_read_b128 %7, %9 offset:7168\n\t"
            "ds_read_b64 %8, %10\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]), "=&v"(v[6]),
              "=&v"(v[7]), "=&v"(m)
            : "v"(a), "v"(b)
            : "memory");
    }
#pragma unroll
    for (int i = 0; i < N; ++i) x[i] = make_float4(v[i].x, v[i].y, v[i].z, v[i].w);
    r = make_float2(m.x, m.y);
    return r;
}
// This wave's N float4 (lane l at dst + 16 l, 1 KiB apart) and its (m, l)
// pair, written to LDS in asm for the same reason as sp_read (the barrier
// that follows waits for them).
template <int N>
__device__ __forceinline__ void sp_write(float4* dst, float2* ml, int lane, const float4 (&x)[N], float2 mlv) {
    const uint32_t a = (uint32_t)(size_t)(__attribute__((address_space(3))) void*)(dst + lane);
    const uint32_t b = (uint32_t)(size_t)(__attribute__((address_space(3))) void*)(ml + lane);
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    f32x4_t v[N];
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = f32x4_t{x[i].x, x[i].y, x[i].z, x[i].w};
    const f32x2_t m = f32x2_t{mlv.x, mlv.y};
    static_assert(N == 2 || N == 4 || N == 8, "write count");
    if constexpr (N == 2) {
        asm volatile(
            "ds_write_b128 %0, %2\n\t"
            "ds_write_b128 %0, %3 offset:1024\n\t"
            "ds_write_b64 %1, %4"
            :
            : "v"(a), "v"(b), "v"(v[0]), "v"(v[1]), "v"(m)
            : "memory");
    } else if constexpr (N == 4) {
        asm volatile(
            "ds_write_b128 %0, %2\n\t"
            "ds_write_b128 %0, %3 offset:1024\n\t"
            "ds_write_b128 %0, %4 offset:2048\n\t"
            "ds_write_b128 %0, %5 offset:3072\n\t"
            "ds_write_b64 %1, %6"
            :
            : "v"(a), "v"(b), "v"(v[0]), "v"(v[1]), "v"(v[2]), "v"(v[3]), "v"(m)
            : "memory");
    } else {
        asm volatile(
            "ds_write_b128 %0, %2\n\t"
            "ds_write_b128 %0, %3 offset:1024\n\t"
            "ds_write_b128 %0, %4 offset:2048\n\t"
            "ds_write_b128 %0, %5 offset:3072\n\t"
            "ds_write_b128 %0, %6 offset:4096\n\t"
            "ds_write_b128 %0, %7 offset:5120\n\t"
            "ds_write_b128 %0, %8 offset:6144\n\t"
            "ds_write_b128 %0, %9 offset:7168\n\t"
            "ds_write_b64 %1, %10"
            :
            : "v"(a), "v"(b), "v"(v[0]), "v"(v[1]), "v"(v[2]), "v"(v[3]), "v"(v[4]), "v"(v[5]), "v"(v[6]),
              "v"(v[7]), "v"(m)
            : "memory");
    }
}
// Weights of two partials with running maxima ma, mb (log2 units) in their
// merge: exp2(m - max(ma, mb)), 0 for a partial that saw no key.
__device__ __forceinline__ void sp_weights(float ma, float mb, float& wa, float& wb) {
    const float M = fmaxf(ma, mb);
    wa = ma == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ma - M);
    wb = mb == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mb - M);
}
// The two exchange rounds of an item's merge for the waves of stream K (all
// indices compile-time): give half GIVE_H of the float4 to the partner k ^ 2
// and fold its copy of half KEEP_H in, then give quarter K ^ 1 to partner
// k ^ 1 (through slot sw ^ 2, which only this wave read in the first round)
// and fold its copy of quarter K in.  On return `part` holds quarter K of
// the merged O and m_run / l_tot the merged statistics.
template <int K, int DB>
__device__ __forceinline__ void sp_merge_stream(f32x16_t (&o)[DB], float4* area, float2 (*s_ml)[64], int sw,
                                                int lane, float& m_run, float& l_tot, float4 (&part)[DB]) {
    constexpr int NF = DB * 4, HALF = NF / 2, QTR = NF / 4;
    constexpr int KEEP_H = (K & 2) ? HALF : 0, GIVE_H = HALF - KEEP_H;
    constexpr int KEEP_Q = K * QTR, GIVE_Q = (K ^ 1) * QTR;
    {
        float4 g[HALF];
#pragma unroll
        for (int i = 0; i < HALF; ++i) {
            const int f = GIVE_H + i;
            g[i] = make_float4(o[f / 4][4 * (f % 4)], o[f / 4][4 * (f % 4) + 1], o[f / 4][4 * (f % 4) + 2],
                               o[f / 4][4 * (f % 4) + 3]);
        }
        sp_write<HALF>(area + sw * HALF * 64, s_ml[sw], lane, g, make_float2(m_run, l_tot));
    }
    lds_ops_barrier();
    {
        float4 x[HALF];
        const float2 ml = sp_read<HALF>(x, area + (sw ^ 2) * HALF * 64, s_ml[sw ^ 2], lane);
        float wa, wb;
        sp_weights(m_run, ml.x, wa, wb);
#pragma unroll
        for (int i = 0; i < HALF; ++i) {
            const int f = KEEP_H + i;
            o[f / 4][4 * (f % 4)] = fmaf(wb, x[i].x, wa * o[f / 4][4 * (f % 4)]);
            o[f / 4][4 * (f % 4) + 1] = fmaf(wb, x[i].y, wa * o[f / 4][4 * (f % 4) + 1]);
            o[f / 4][4 * (f % 4) + 2] = fmaf(wb, x[i].z, wa * o[f / 4][4 * (f % 4) + 2]);
            o[f / 4][4 * (f % 4) + 3] = fmaf(wb, x[i].w, wa * o[f / 4][4 * (f % 4) + 3]);
        }
        l_tot = fmaf(wb, ml.y, wa * l_tot);
        m_run = fmaxf(m_run, ml.x);
    }
    {
        float4 g[QTR];
#pragma unroll
        for (int i = 0; i < QTR; ++i) {
            const int f = GIVE_Q + i;
            g[i] = make_float4(o[f / 4][4 * (f % 4)], o[f / 4][4 * (f % 4) + 1], o[f / 4][4 * (f % 4) + 2],
                               o[f / 4][4 * (f % 4) + 3]);
        }
        sp_write<QTR>(area + (sw ^ 2) * HALF * 64, s_ml[sw ^ 2], lane, g, make_float2(m_run, l_tot));
    }
    lds_ops_barrier();
    {
        float4 x[QTR];
        const float2 ml = sp_read<QTR>(x, area + (sw ^ 3) * HALF * 64, s_ml[sw ^ 3], lane);
        float wa, wb;
        sp_weights(m_run, ml.x, wa, wb);
#pragma unroll
        for (int i = 0; i < QTR; ++i) {
            const int f = KEEP_Q + i;
            part[i] = make_float4(fmaf(wb, x[i].x, wa * o[f / 4][4 * (f % 4)]),
                                  fmaf(wb, x[i].y, wa * o[f / 4][4 * (f % 4) + 1]),
                                  fmaf(wb, x[i].z, wa * o[f / 4][4 * (f % 4) + 2]),
                                  fmaf(wb, x[i].w, wa * o[f / 4][4 * (f % 4) + 3]));
        }
        l_tot = fmaf(wb, ml.y, wa * l_tot);
        m_run = fmaxf(m_run, ml.x);
    }
    // A distinct instruction closing each stream's copy, so that the
    // compiler does not merge the four copies into one indexed by stream
    // (which would put the accumulators in scratch memory).
    if constexpr (K == 0) asm volatile("; merge, stream 0");
    else if constexpr (K == 1) asm volatile("; merge, stream 1");
    else if constexpr (K == 2) asm volatile("; merge, stream 2");
    else asm volatile("; merge, stream 3");
}

template <int D, bool FUSED>
__global__ __launch_bounds__(kSpThreads, 1) void prefill_splitkv_pair_kernel(PrefillProblem p,
                                                                             float scale_log2,
                                                                             uint32_t n_items) {
    using P = SpShape<D>;
    // Two buffers as separate arrays, so that the compiler can tell the one
    // being read from the one the loads are filling.  The merge reuses the
    // second (s_b): 8 waves x 64 lanes x D/4 floats = one buffer exactly.
    __shared__ __align__(1024) uint16_t s_a[P::STAGE];
    __shared__ __align__(1024) uint16_t s_b[P::STAGE];
    __shared__ float2 s_ml8[8][64];
    static_assert(8 * 64 * (D / 4) * 4 == P::STAGE * 2, "merge area is one buffer");

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int ql = lane & 31, kg = lane >> 5;
    const int sw = __builtin_amdgcn_readfirstlane(wave);
    const int stream = sw & 3, sub = sw >> 2;
    const uint32_t group = p.hq / p.hkv;
    const uint32_t n_qt = (p.s + kSkBM - 1) / kSkBM;
    const uint32_t row_bytes = p.hkv * D * 2;
    const uint32_t kv_bytes = (p.s - 1) * row_bytes + D * 2;

    // This lane's global chunk for each of its blocks of a tile (blocks
    // sub, sub + 2, ...), laid out as the 128-row kernel's tiles.
    uint32_t offk[P::BPW], offv[P::BPW];
#pragma unroll
    for (int j = 0; j < P::BPW; ++j) {
        const int slot = 64 * (sub + 2 * j) + lane;
        const int row = slot / P::CPR, phys = slot % P::CPR;
        offk[j] = row * row_bytes + 16 * (phys ^ k_swz<D>(row));
        offv[j] = row * row_bytes + 16 * (phys ^ v_swz<D>(row));
    }
    // Operand read offsets within a stream's tiles (elements).
    int k_off[P::KSTEPS], v_off[P::DBLK];
#pragma unroll
    for (int ks = 0; ks < P::KSTEPS; ++ks) k_off[ks] = ql * D + 8 * ((2 * ks + kg) ^ k_swz<D>(ql));
    {
        const int s16 = lane & 15, g16 = lane >> 4;
        const int vrow = 4 * kg + (s16 >> 2);
#pragma unroll
        for (int db = 0; db < P::DBLK; ++db) {
            const int c = 4 * db + 2 * (g16 & 1) + ((s16 & 3) >> 1);
            v_off[db] = vrow * D + 8 * (c ^ v_swz<D>(vrow)) + 4 * (s16 & 1);
        }
    }

    uint32_t round = 0;
    SpItem it = sp_item(p, blockIdx.x, group, n_qt);
    const uint16_t* k_head = p.k + (int64_t)it.kvh * D;
    const uint16_t* v_head = p.v + (int64_t)it.kvh * D;
    // Tile t of the current item into buffer `buf` (this stream's part).
    auto dma = [&](uint32_t t, uint16_t* buf) __attribute__((always_inline)) {
        sp_dma_tile<D>(k_head, v_head, kv_bytes, t * kSkBN * row_bytes, offk, offv, sub,
                       buf + stream * P::STREAM);
    };
    bf16x8_t qf[P::KSTEPS];
    if ((uint32_t)stream < it.n_tiles) dma(stream, s_a);
    load_q<D, FUSED>(qf, p, it.q0 + ql, it.h0 + sub, kg);

    while (true) {
        const uint32_t q0 = it.q0, qq = q0 + ql, n_tiles = it.n_tiles;
        const uint32_t n_steps = (n_tiles + 3) / 4;
        f32x16_t oacc[P::DBLK];
#pragma unroll
        for (int db = 0; db < P::DBLK; ++db)
#pragma unroll
            for (int i = 0; i < 16; ++i) oacc[db][i] = 0.0f;
        float m_run = -INFINITY, l_run = 0.0f;

        // This stream's key tile t, from buffer `cur`.
        auto tile = [&](uint32_t t, const uint16_t* cur) __attribute__((always_inline)) {
            const uint16_t* kb = cur + stream * P::STREAM;
            const uint16_t* vb = kb + P::TILE;
            const uint32_t n0 = t * kSkBN;
            f32x16_t st;
#pragma unroll
            for (int i = 0; i < 16; ++i) st[i] = 0.0f;
            uint4 ka[P::KSTEPS];
#pragma unroll
            for (int ks = 0; ks < P::KSTEPS; ++ks) ka[ks] = *reinterpret_cast<const uint4*>(kb + k_off[ks]);
#pragma unroll
            for (int ks = 0; ks < P::KSTEPS; ++ks) st = mfma32x32x16(as_bf16x8(ka[ks]), qf[ks], st);
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
            for (int ks = 0; ks + 2 < P::KSTEPS; ++ks) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
            if (n0 + kSkBN - 1 > q0) {
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const uint32_t key = n0 + 8 * (i / 4) + 4 * kg + (i % 4);
                    if (key > qq) st[i] = -INFINITY;
                }
            }
            float ma = fmaxf(st[0], st[1]), mb = fmaxf(st[8], st[9]);
#pragma unroll
            for (int i = 2; i < 8; i += 2) {
                ma = fmaxf(fmaxf(ma, st[i]), st[i + 1]);
                mb = fmaxf(fmaxf(mb, st[i + 8]), st[i + 9]);
            }
            const float mt = xor32_max(fmaxf(ma, mb)) * scale_log2;
            const bool need = mt > m_run + kRescaleThreshold;
            if (__any(need)) {
                float alpha = 1.0f;
                if (need) {
                    alpha = __builtin_amdgcn_exp2f(m_run - mt);
                    m_run = mt;
                }
                l_run *= alpha;
#pragma unroll
                for (int db = 0; db < P::DBLK; ++db)
#pragma unroll
                    for (int i = 0; i < 16; ++i) oacc[db][i] *= alpha;
            }
#pragma unroll
            for (int i = 0; i < 16; ++i) st[i] = __builtin_amdgcn_exp2f(fmaf(st[i], scale_log2, -m_run));
            bf16x8_t pf[2];
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                const int o8 = 8 * tt;
                pf[tt] = as_bf16x8(make_uint4(pack_bf16x2(st[o8 + 0], st[o8 + 1]),
                                              pack_bf16x2(st[o8 + 2], st[o8 + 3]),
                                              pack_bf16x2(st[o8 + 4], st[o8 + 5]),
                                              pack_bf16x2(st[o8 + 6], st[o8 + 7])));
            }
            l_run += sum_bf16x8(__builtin_bit_cast(uint4, pf[0]),
                                sum_bf16x8(__builtin_bit_cast(uint4, pf[1]), 0.0f));
#pragma unroll
            for (int tt = 0; tt < 2; ++tt)
#pragma unroll
                for (int db = 0; db < P::DBLK; ++db) {
                    const v4i16_t lo = ds_read_tr16(vb + v_off[db] + 16 * tt * D);
                    const v4i16_t hi = ds_read_tr16(vb + v_off[db] + (16 * tt + 8) * D);
                    const uint4 a = make_uint4(__builtin_bit_cast(uint2, lo).x, __builtin_bit_cast(uint2, lo).y,
                                               __builtin_bit_cast(uint2, hi).x, __builtin_bit_cast(uint2, hi).y);
                    oacc[db] = mfma32x32x16(as_bf16x8(a), pf[tt], oacc[db]);
                }
        };
        // Step s: step s + 1's tiles go to the other buffer (every wave was
        // done with it at the previous step's barrier) and this stream's tile
        // of step s is computed; then every wave waits for its loads and for
        // the other waves.  The waits for the loads are explicit: the
        // compiler does not track loads that write LDS across the loop's
        // back edge.
        auto step = [&](uint32_t s, const uint16_t* cur, uint16_t* nxt) __attribute__((always_inline)) {
            const uint32_t tn = stream + 4 * (s + 1);
            if (tn < n_tiles) dma(tn, nxt);
            const uint32_t t = stream + 4 * s;
            if (t < n_tiles) tile(t, cur);
            __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
            __syncthreads();
        };
        __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);  // step 0's tiles and Q
        __syncthreads();
        for (uint32_t s = 0; s < n_steps; s += 2) {
            step(s, s_a, s_b);
            if (s + 1 < n_steps) step(s + 1, s_b, s_a);
        }
        // Every wave is done with both buffers (the last step's barrier): the
        // next item's first tiles go to s_a and its Q to registers, landing
        // while this item merges in s_b.  (With FUSED the grid holds every
        // item: its Q prologue would not fit beside the merge's registers.)
        ++round;
        const uint32_t nxt = sk_item_index(round, blockIdx.x, gridDim.x);
        const bool more = !FUSED && nxt < n_items;
        const uint32_t h = it.h0 + sub;
        if (more) {
            it = sp_item(p, nxt, group, n_qt);
            k_head = p.k + (int64_t)it.kvh * D;
            v_head = p.v + (int64_t)it.kvh * D;
            if ((uint32_t)stream < it.n_tiles) dma(stream, s_a);
            load_q<D, FUSED>(qf, p, it.q0 + ql, it.h0 + sub, kg);
        }

        // Merge: the four streams' partials of each head in two exchange
        // rounds in which every wave takes part (streams k and k ^ 2 swap
        // halves of their O values, then k and k ^ 1 quarters of the kept
        // half), in s_b; stream k then writes quarter k of its head's output.
        float l_tot = xor32_sum(l_run);
        float4 part[P::DBLK];
        float4* const area = reinterpret_cast<float4*>(s_b);
        switch (stream) {
            case 0: sp_merge_stream<0>(oacc, area, s_ml8, sw, lane, m_run, l_tot, part); break;
            case 1: sp_merge_stream<1>(oacc, area, s_ml8, sw, lane, m_run, l_tot, part); break;
            case 2: sp_merge_stream<2>(oacc, area, s_ml8, sw, lane, m_run, l_tot, part); break;
            default: sp_merge_stream<3>(oacc, area, s_ml8, sw, lane, m_run, l_tot, part); break;
        }
        if (qq < p.s) {
            const float inv = 1.0f / l_tot;
            uint16_t* orow = p.o + ((int64_t)qq * p.hq + h) * D + 4 * kg;
#pragma unroll
            for (int i = 0; i < P::DBLK; ++i) {
                const int f = P::DBLK * stream + i;  // wave-uniform
                *reinterpret_cast<uint2*>(orow + 32 * (f / 4) + 8 * (f % 4)) =
                    make_uint2(pack_bf16x2(part[i].x * inv, part[i].y * inv),
                               pack_bf16x2(part[i].z * inv, part[i].w * inv));
            }
        }
        if (!more) break;
    }
}

// Below this many 128-row workgroups the split-over-keys variant wins: the
// 128-row kernel would leave CUs idle and be bound by its longest tile walk.
constexpr uint32_t kSplitKvBelowWgs = 257;

// Workgroups of a persistent split kernel the device holds at once (CUs x
// resident blocks per CU), queried once per device into the caller's
// per-kernel `cache`; `fallback` per CU when no device is visible.
template <typename Kern>
uint32_t resident_slots(Kern kern, int threads, int fallback, int (&cache)[64]) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
        (void)hipGetLastError();
        return 256 * fallback;
    }
    int v = __atomic_load_n(&cache[dev], __ATOMIC_RELAXED);
    if (v > 0) return (uint32_t)v;
    int cus = 0, per = 0;
    const hipError_t e1 = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    const hipError_t e2 = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, kern, threads, 0);
    if (e1 != hipSuccess || e2 != hipSuccess || cus <= 0 || per <= 0) {
        (void)hipGetLastError();
        return 256 * fallback;
    }
    v = cus * per;
    __atomic_store_n(&cache[dev], v, __ATOMIC_RELAXED);
    return (uint32_t)v;
}

template <int D>
hipError_t launch_pairs(const PrefillProblem& p, float sl2, uint32_t items, uint32_t slots,
                        hipStream_t st) {
    const dim3 grid(min(items, slots));
    hipLaunchKernelGGL((prefill_splitkv_pair_kernel<D, false>), grid, dim3(kSpThreads), 0, st, p,
                       sl2, items);
    return hipGetLastError();
}

template <int D, bool FUSED>
hipError_t launch_t(const PrefillProblem& p, hipStream_t st) {
    const uint32_t n_qtiles = (p.s + kPfBM - 1) / kPfBM;
    const float sl2 = kLog2e / sqrtf((float)D);
    const bool split = prefill_uses_split(p);
    // Short sequences with an even GQA group take the pair kernel when asked
    // (variant 3), or by shape when it has more items than the device holds
    // workgroups of it at D = 128: with fewer it leaves CUs idle, and at
    // D = 64 a tile's work is too small for its per-step barrier and merge
    // (measured on MI355X: S = 1371, 16/8 heads, 21.3 -> 18.7 us at D = 128,
    // 12.1 -> 12.5 us at D = 64; S = 512: 9.1 -> 10.8 us).  The fused Q
    // prologue stays with the single-head kernel.
    if (!FUSED && split && (p.hq / p.hkv) % 2 == 0 && p.variant != 1) {
        static int cache[64];
        const uint32_t items = ((p.s + kSkBM - 1) / kSkBM) * p.hkv * (p.hq / p.hkv / 2);
        const uint32_t slots = resident_slots(prefill_splitkv_pair_kernel<D, false>, kSpThreads, 1, cache);
        if (p.variant == 3 || (D == 128 && items > slots)) return launch_pairs<D>(p, sl2, items, slots, st);
    }
    if (split) {
        const uint32_t items = ((p.s + kSkBM - 1) / kSkBM) * p.hq;
        static int cache[64];
        const dim3 grid(FUSED ? items : min(items, resident_slots(prefill_splitkv_kernel<D, FUSED>, kPfThreads, 2, cache)));
        hipLaunchKernelGGL((prefill_splitkv_kernel<D, FUSED>), grid, dim3(kPfThreads), 0, st, p,
                           sl2, items);
    } else {
        // Head pairs per workgroup when the GQA group is even and the pair
        // grid is at least two rounds of the device (measured on MI355X,
        // 32/8 heads: S = 8192 490 -> 479 us, S = 4096 150 -> 143 us, but
        // S = 2048, one round, 50 -> 58 us).
        static int cache[64];
        const uint32_t pair_wgs = n_qtiles * (p.hq / 2);
        const bool even = (p.hq / p.hkv) % 2 == 0;
        if (even && (p.variant == 4 ||
                     (p.variant == 0 && pair_wgs >= 2 * resident_slots(prefill_kernel<D, FUSED, true>, 512, 1, cache)))) {
            hipLaunchKernelGGL((prefill_kernel<D, FUSED, true>), dim3(pair_wgs), dim3(512), 0, st, p, sl2);
        } else {
            hipLaunchKernelGGL((prefill_kernel<D, FUSED, false>), dim3(n_qtiles * p.hq), dim3(kPfThreads), 0,
                               st, p, sl2);
        }
    }
    return hipGetLastError();
}

}  // namespace

bool prefill_uses_split(const PrefillProblem& p) {
    const uint32_t n_qtiles = (p.s + kPfBM - 1) / kPfBM;
    return p.variant == 1 || p.variant == 3 || (p.variant == 0 && n_qtiles * p.hq < kSplitKvBelowWgs);
}

hipError_t launch_prefill(const PrefillProblem& p, hipStream_t stream) {
    if (p.d == 64) return p.fused_q ? launch_t<64, true>(p, stream) : launch_t<64, false>(p, stream);
    return p.fused_q ? launch_t<128, true>(p, stream) : launch_t<128, false>(p, stream);
}

}  // namespace tiattn
