// Projections around the attention path: y = W·x for one decoded token
// (bf16 or fp32 out) and y[t] = W·x[t] for a prefill batch.
//
// W is [M][N] bf16 row-major (one output per row, as the reference stores
// its projection weights), x is [T][N] bf16, y is [T][M].  Every product is
// accumulated in fp32 and rounded once at the store.
//
//  * gemv_kernel: HBM-bound.  A workgroup of 256 lanes owns RB output rows
//    and TB tokens; each lane walks 16-byte chunks of the rows (chunk c =
//    lane + 256 j), loads the token chunk once and reuses it for all RB rows,
//    and keeps TB x RB fp32 partials.  Partials are reduced in the wave
//    (DPP rows, then v_permlane16/32_swap) and across the four waves in LDS.
//    Buffer loads with an exact range return zeros past the last row or
//    token, so the tails need no branches.  The weight rows, read once per
//    call, carry the non-temporal hint (the lm-head's 1.24 GB then streams
//    at 6.95 TB/s where plain loads reach 6.2).
//  * gemm_kernel: MFMA-bound (prefill, T > kGemvMaxTokens).  K in 64-wide
//    slices double-buffered in LDS by buffer-load DMA, v_mfma_f32_32x32x16_bf16
//    on 32 x 32 blocks.  256 x 256 tiles (8 waves of 128 x 64) when they
//    alone fill every CU, else 128 x 128 tiles (4 waves of 64 x 64, two
//    workgroups per CU).  Tiles are ordered in 8 x 8 groups and the groups
//    are dealt to XCDs in contiguous runs, so the blocks resident on one XCD
//    share W and x slices in that XCD's L2.  The results leave through LDS
//    as whole 16-byte chunks of token rows.
#include "common.hpp"
#include "kernels.hpp"

namespace tiattn {
namespace {

// ------------------------------------------------------------------ GEMV

constexpr int kGvThreads = 256;
constexpr uint32_t kOob = 0xF0000000u;  // a byte offset past every range below

// E bf16 values per load: 8 (16-byte chunks), 2 (bf16 pairs) or 1.
template <int E>
struct GvChunk {
    static constexpr int WORDS = E == 8 ? 4 : 1;
    uint32_t w[WORDS];
};

// POL: the loads' cache-policy bits (kGvStream for the weight rows, which
// one call reads exactly once).
constexpr int kGvStream = 2;  // nt

template <int E, int POL = 0>
__device__ __forceinline__ GvChunk<E> gv_load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    GvChunk<E> c;
    if constexpr (E == 8) {
        const uint4 v = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, POL));
        c.w[0] = v.x; c.w[1] = v.y; c.w[2] = v.z; c.w[3] = v.w;
    } else if constexpr (E == 2) {
        c.w[0] = __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, POL);
    } else {
        c.w[0] = __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, POL);
    }
    return c;
}

template <int E>
__device__ __forceinline__ float gv_dot(const GvChunk<E>& w, const GvChunk<E>& x, float acc) {
    if constexpr (E == 1) {
        return fmaf(bf16_lo(w.w[0]), bf16_lo(x.w[0]), acc);
    } else {
#pragma unroll
        for (int i = 0; i < GvChunk<E>::WORDS; ++i)
            acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w.w[i]),
                                                  __builtin_bit_cast(bf16x2_t, x.w[i]), acc, false);
        return acc;
    }
}

__device__ __forceinline__ void gv_store(uint16_t* y, size_t i, float v) { y[i] = f32_to_bf16(v); }
__device__ __forceinline__ void gv_store(float* y, size_t i, float v) { y[i] = v; }

template <int E, int RB, int TB, typename OutT>
__global__ __launch_bounds__(kGvThreads) void gemv_kernel(const uint16_t* __restrict__ W,
                                                          const uint16_t* __restrict__ x,
                                                          OutT* __restrict__ y, uint32_t T,
                                                          uint32_t M, uint32_t N) {
    const uint32_t r0 = blockIdx.x * RB, t0 = blockIdx.y * TB;
    const uint32_t nrows = min((uint32_t)RB, M - r0), ntok = min((uint32_t)TB, T - t0);
    const uint32_t row_bytes = 2 * N;
    const auto rw = make_rsrc(W + (size_t)r0 * N, nrows * row_bytes);
    const auto rx = make_rsrc(x + (size_t)t0 * N, ntok * row_bytes);
    const uint32_t nchunk = N / E;

    float acc[TB][RB];
#pragma unroll
    for (int t = 0; t < TB; ++t)
#pragma unroll
        for (int r = 0; r < RB; ++r) acc[t][r] = 0.0f;

    // Two chunks per lane per trip; the second one's offset is pushed out of
    // range (zeros) when it is past the row.
    for (uint32_t c = threadIdx.x; c < nchunk; c += 2 * kGvThreads) {
        const uint32_t c2 = c + kGvThreads;
        const uint32_t off[2] = {c * 2 * E, c2 < nchunk ? c2 * 2 * E : kOob};
        GvChunk<E> xv[2][TB], wv[2][RB];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
#pragma unroll
            for (int t = 0; t < TB; ++t) xv[u][t] = gv_load<E>(rx, t * row_bytes + off[u]);
#pragma unroll
            for (int r = 0; r < RB; ++r) wv[u][r] = gv_load<E, kGvStream>(rw, r * row_bytes + off[u]);
        }
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int t = 0; t < TB; ++t)
#pragma unroll
                for (int r = 0; r < RB; ++r) acc[t][r] = gv_dot<E>(wv[u][r], xv[u][t], acc[t][r]);
    }

    __shared__ float red[kGvThreads / 64][TB * RB];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int t = 0; t < TB; ++t)
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            const float s = wave_sum(acc[t][r]);
            if (lane == 0) red[wave][t * RB + r] = s;
        }
    __syncthreads();
    if (threadIdx.x < TB * RB) {
        const uint32_t t = threadIdx.x / RB, r = threadIdx.x % RB;
        float s = 0.0f;
#pragma unroll
        for (int w = 0; w < kGvThreads / 64; ++w) s += red[w][threadIdx.x];
        if (t < ntok && r < nrows) gv_store(y, (size_t)(t0 + t) * M + r0 + r, s);
    }
}

template <int E, int RB, int TB, typename OutT>
hipError_t gemv_launch(const uint16_t* W, const uint16_t* x, OutT* y, uint32_t T, uint32_t M,
                       uint32_t N, hipStream_t stream) {
    const dim3 grid((M + RB - 1) / RB, (T + TB - 1) / TB);
    gemv_kernel<E, RB, TB, OutT><<<grid, kGvThreads, 0, stream>>>(W, x, y, T, M, N);
    return hipGetLastError();
}

// Rows per workgroup: enough workgroups (about two per CU) for small M,
// more reuse of each token chunk for large M.
template <int E, int TB, typename OutT>
hipError_t gemv_rows(const uint16_t* W, const uint16_t* x, OutT* y, uint32_t T, uint32_t M,
                     uint32_t N, hipStream_t stream) {
    if constexpr (E != 8) {
        return gemv_launch<E, 4, TB>(W, x, y, T, M, N, stream);
    } else {
        if (M >= 4096) return gemv_launch<E, 8, TB>(W, x, y, T, M, N, stream);
        if (M >= 2048) return gemv_launch<E, 4, TB>(W, x, y, T, M, N, stream);
        if (M >= 1024) return gemv_launch<E, 2, TB>(W, x, y, T, M, N, stream);
        return gemv_launch<E, 1, TB>(W, x, y, T, M, N, stream);
    }
}

template <int TB, typename OutT>
hipError_t gemv_any(const uint16_t* W, const uint16_t* x, OutT* y, uint32_t T, uint32_t M,
                    uint32_t N, hipStream_t stream) {
    const uintptr_t a = (uintptr_t)W | (uintptr_t)x;
    if (N % 8 == 0 && a % 16 == 0) return gemv_rows<8, TB>(W, x, y, T, M, N, stream);
    if (N % 2 == 0 && a % 4 == 0) return gemv_rows<2, TB>(W, x, y, T, M, N, stream);
    return gemv_rows<1, TB>(W, x, y, T, M, N, stream);
}

// ------------------------------------------------------------------ GEMM

constexpr int kGmBK = 64;    // K granularity every GEMM configuration handles
constexpr int kGmGroup = 8;  // tile groups of 8 x 8

// Block tile BM (tokens) x BN (outputs) on a WGM x WGN grid of waves; each
// wave owns IM x JN blocks of 32 x 32.  K advances in slices of BK (64 or
// 128): KS k-steps of 16 per slice.
template <int BM_, int BN_, int WGM_, int WGN_, int MINB_, int BK_ = 64>
struct GmCfg {
    static constexpr int BM = BM_, BN = BN_, WGM = WGM_, WGN = WGN_, MINB = MINB_, BK = BK_;
    static constexpr int WAVES = WGM * WGN, THREADS = 64 * WAVES;
    static constexpr int IM = BM / WGM / 32, JN = BN / WGN / 32;
    static constexpr int KS = BK / 16, CPR = BK / 8, RPB = 64 / CPR;  // chunks per row, rows per DMA
    static constexpr int A_ELEMS = BM * BK, B_ELEMS = BN * BK;
    static constexpr int A_DMA = BM / RPB / WAVES, B_DMA = BN / RPB / WAVES;  // per wave
    static_assert(A_DMA * RPB * WAVES == BM && B_DMA * RPB * WAVES == BN, "DMA split");
    static_assert(BK == 64 || BK == 128, "slice width");
};
// 64 x 64 tiles serve grids too small to fill the CUs with larger tiles; with
// few MFMAs per slice they are latency-bound, so they take 128-wide slices.
using GmMini = GmCfg<64, 64, 2, 2, 4, 128>;  // 4 waves of 32 x 32
using GmMini64 = GmCfg<64, 64, 2, 2, 4, 64>;
using GmSmall = GmCfg<128, 128, 2, 2, 2>;  // 4 waves of 64 x 64, 2 workgroups per CU
using GmMid = GmCfg<128, 192, 2, 2, 2>;    // 4 waves of 64 x 96, 2 workgroups per CU (80 KB LDS each)
using GmTall = GmCfg<192, 128, 2, 2, 2>;   // 4 waves of 96 x 64, 2 workgroups per CU (80 KB LDS each)
using GmLarge = GmCfg<256, 256, 2, 4, 1>;  // 8 waves of 128 x 64

// LDS rows of BK bf16 (CPR 16-byte chunks); chunk c of row r sits at
// c ^ gm_swz<CPR>(r).  A 16-byte LDS read serves 16 lanes per cycle from
// 64 banks (256 bytes), and the MFMA operand reads put 16 consecutive rows
// on 16 consecutive lanes, all at one logical chunk: with 256-byte rows
// (CPR 16) the swizzle r & 15 gives the 16 rows 16 different chunks; with
// 128-byte rows (CPR 8) rows r and r + 1 share a 256-byte bank line (r & 1
// picks its half), so the 8 rows of each parity need different chunks:
// (r >> 1) & 7.  (A swizzle r & 7 had rows r and r + 8 meet on the same
// banks: 4 conflict cycles per read.)  One DMA instruction fills 64 / CPR
// rows: lane l loads row l / CPR, physical chunk l % CPR, i.e. logical
// chunk (l % CPR) ^ gm_swz<CPR>(row).
template <int CPR>
__device__ __forceinline__ uint32_t gm_swz(uint32_t row) {
    return CPR == 16 ? row & 15 : (row >> 1) & 7;
}

template <int WAVES, int BLOCKS, int CPR>
__device__ __forceinline__ void gm_dma(__amdgpu_buffer_rsrc_t r, uint32_t row_bytes, uint32_t k_off,
                                       uint16_t* lds) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int j = 0; j < BLOCKS; ++j) {
        const int blk = wave + WAVES * j;
        const uint32_t row = (64 / CPR) * blk + lane / CPR;
        const uint32_t logical = (lane % CPR) ^ gm_swz<CPR>(row);
        dma16(r, lds + 512 * blk, row * row_bytes + k_off + 16 * logical);
    }
}

struct GmTile {
    uint32_t tt, tm;  // token tile, output tile
};

// Grouped order (8 output tiles x 8 token tiles per group, token-major
// inside a group), and consecutive group positions on one XCD: hardware
// deals workgroup b to XCD b % 8, so b -> (b % 8) * (n / 8) + b / 8 gives
// XCD x the run [x n / 8, (x + 1) n / 8) when n % 8 == 0.
__device__ __forceinline__ GmTile gm_tile(uint32_t b, uint32_t n_tt, uint32_t n_tm) {
    const uint32_t n = n_tt * n_tm;
    const uint32_t g = n % 8 == 0 ? (b % 8) * (n / 8) + b / 8 : b;
    const uint32_t per_group = kGmGroup * n_tt;
    const uint32_t first_tm = (g / per_group) * kGmGroup;
    const uint32_t gsize = min((uint32_t)kGmGroup, n_tm - first_tm);
    const uint32_t in = g % per_group;
    return {in / gsize, first_tm + in % gsize};
}

// Output tiles of one launch: BN columns of the stacked segments, or with
// the SwiGLU epilogue BN / 2 columns of the gate/up pair.
template <typename C, bool SW>
__device__ __host__ __forceinline__ uint32_t gm_out_tiles(const GemmArgs& g) {
    if (SW) return (g.rows[0] + C::BN / 2 - 1) / (C::BN / 2);
    uint32_t n = 0;
    for (int sg = 0; sg < g.nseg; ++sg) n += (g.rows[sg] + C::BN - 1) / C::BN;
    return n;
}

// Epilogue staging: chunk c of staged row t (CR 16-byte chunks per row)
// sits at ep_chunk<CR>(c, t), its two 8-byte halves swapped when
// ep_swap<CR>(t).  An 8-byte LDS write serves 16 lanes per cycle from 32
// banks (128 bytes), and the staging writes put 16 consecutive rows on 16
// lanes at one logical half chunk, so those 16 (chunk, half) positions must
// differ modulo 128 bytes: with 128-byte rows (CR 8) every row starts on the
// same banks, the chunk takes bits 1-3 of t and the half bit 0; with 64- or
// 192-byte rows (CR 4, 12) bit 0 of t picks the 64-byte half of the bank
// line, the chunk takes bits 1-2 (within its aligned group of four) and the
// half bit 3.  The 16-byte read-back (16 lanes per cycle from 64 banks) of
// consecutive chunks of a row stays a permutation of the row's banks.
template <int CR>
__device__ __forceinline__ int ep_chunk(int c, int t) {
    return CR == 8 ? c ^ ((t >> 1) & 7) : c ^ ((t >> 1) & 3);
}
template <int CR>
__device__ __forceinline__ int ep_swap(int t) {
    return CR == 8 ? t & 1 : (t >> 3) & 1;
}

// Epilogue LDS accesses in asm: to the compiler they are not LDS accesses,
// which it would make wait for every buffer load that writes LDS (it cannot
// tell the ring slot they use from the others).  A wave's LDS operations run
// in order, so its staging writes need no wait before its reads; ep_read
// waits for its own reads.
__device__ __forceinline__ uint32_t lds_addr(const uint16_t* p) {
    return (uint32_t)(size_t)(const __attribute__((address_space(3))) void*)p;
}
__device__ __forceinline__ void ep_write(uint16_t* p, uint32_t lo, uint32_t hi) {
    typedef unsigned v2u_t __attribute__((ext_vector_type(2)));
    const v2u_t v = {lo, hi};
    asm volatile("ds_write_b64 %0, %1" ::"v"(lds_addr(p)), "v"(v) : "memory");
}
template <int N>
__device__ __forceinline__ void ep_read(uint4 (&x)[N], const uint32_t (&a)[N]) {
    typedef unsigned v4u_t __attribute__((ext_vector_type(4)));
    v4u_t v[N];
    if constexpr (N == 2) {
        asm volatile("ds_read_b128 %0, %2\n\tds_read_b128 %1, %3\n\ts_waitcnt lgkmcnt(0)"
                     : "=&v"(v[0]), "=&v"(v[1])
                     : "v"(a[0]), "v"(a[1])
                     : "memory");
    } else if constexpr (N == 4) {
        asm volatile(
            "ds_read_b128 %0, %4\n\tds_read_b128 %1, %5\n\tds_read_b128 %2, %6\n\t"
            "ds_read_b128 %3, %7\n\ts_waitcnt lgkmcnt(0)"
            : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3])
            : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3])
            : "memory");
    } else if constexpr (N == 6) {
        asm volatile(
            "ds_read_b128 %0, %6\n\tds_read_b128 %1, %7\n\tds_read_b128 %2, %8\n\t"
            "ds_read_b128 %3, %9\n\tds_read_b128 %4, %10\n\tds_read_b128 %5, %11\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5])
            : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(a[4]), "v"(a[5])
            : "memory");
    } else {
        static_assert(N == 8, "ep_read sizes");
        asm volatile(
            "ds_read_b128 %0, %8\n\tds_read_b128 %1, %9\n\tds_read_b128 %2, %10\n\t"
            "ds_read_b128 %3, %11\n\tds_read_b128 %4, %12\n\tds_read_b128 %5, %13\n\t"
            "ds_read_b128 %6, %14\n\tds_read_b128 %7, %15\n\ts_waitcnt lgkmcnt(0)"
            : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]),
              "=&v"(v[6]), "=&v"(v[7])
            : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(a[4]), "v"(a[5]), "v"(a[6]),
              "v"(a[7])
            : "memory");
    }
#pragma unroll
    for (int k = 0; k < N; ++k) x[k] = make_uint4(v[k].x, v[k].y, v[k].z, v[k].w);
}

// Eight packed bf16 pairs: bf16(a + b) each, the sums in fp32.
__device__ __forceinline__ uint4 add_bf16x8(uint4 a, uint4 b) {
    const uint32_t x[4] = {a.x, a.y, a.z, a.w}, z[4] = {b.x, b.y, b.z, b.w};
    uint32_t o[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
        o[k] = pack_bf16x2(bf16_lo(x[k]) + bf16_lo(z[k]), bf16_hi(x[k]) + bf16_hi(z[k]));
    return make_uint4(o[0], o[1], o[2], o[3]);
}

// SW (SwiGLU epilogue): B tile row r belongs to 32-row block b = r / 32;
// even blocks are gate rows, odd blocks up rows, both of output columns
// m0 + 32 (b / 2) + r % 32, so a wave's two column blocks (JN = 2) hold
// gate and up of the same 32 columns and the epilogue pairs them in-lane.
template <typename C, bool SW>
__global__ __launch_bounds__(C::THREADS, C::MINB) void gemm_kernel(GemmArgs g) {
    constexpr int IM = C::IM, JN = C::JN;
    static_assert(!SW || JN == 2, "the SwiGLU pairing needs two column blocks per wave");
    const uint32_t T = g.T, N = g.N;
    const uint16_t* __restrict__ x = g.x;
    // One array per stage (A rows, then B rows), so that the compiler can
    // tell the stage being read from the one the DMA is filling.
    __shared__ __align__(1024) uint16_t s_0[C::A_ELEMS + C::B_ELEMS];
    __shared__ __align__(1024) uint16_t s_1[C::A_ELEMS + C::B_ELEMS];
    // Output tiles run over the segments' rows stacked, each segment
    // starting on a tile boundary.
    const uint32_t n_tm = gm_out_tiles<C, SW>(g);
    const uint32_t n_tt = (T + C::BM - 1) / C::BM;
    const GmTile tile = gm_tile(blockIdx.x, n_tt, n_tm);
    uint32_t tm = tile.tm;
    int seg = 0;
    if (!SW) {
        const uint32_t spans[3] = {(g.rows[0] + C::BN - 1) / C::BN, (g.rows[1] + C::BN - 1) / C::BN,
                                   (g.rows[2] + C::BN - 1) / C::BN};
        seg = segment_of(spans, g.nseg, tm);
    }
    constexpr uint32_t TILE_N = SW ? C::BN / 2 : C::BN;  // output columns per tile
    const uint32_t M = pick3(g.rows, seg);
    uint16_t* __restrict__ y = pick3(g.y, seg);
    const uint32_t t0 = tile.tt * C::BM, m0 = tm * TILE_N;
    const uint32_t row_bytes = 2 * N;
    const auto ra = make_rsrc(x + (size_t)t0 * N, min((uint32_t)C::BM, T - t0) * row_bytes);
    const uint32_t b_rows = min(TILE_N, M - m0);
    const auto rb = make_rsrc(pick3(g.w, seg) + (size_t)m0 * N, b_rows * row_bytes);
    const auto rb_up = make_rsrc(pick3(g.w, SW ? 1 : seg) + (size_t)m0 * N, b_rows * row_bytes);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wr = wave / C::WGN, wc = wave % C::WGN;

    // Operand read offsets (elements) inside a stage for block 0, per
    // k-step; block i adds 32 i rows.
    constexpr int BK = C::BK, KS = C::KS;
    int a_off[KS], b_off[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) {
        const int chunk = (2 * s + (lane >> 5)) ^ gm_swz<C::CPR>(lane & 31);  // rows differ by 32 i
        a_off[s] = (32 * IM * wr + (lane & 31)) * BK + 8 * chunk;
        b_off[s] = C::A_ELEMS + (32 * JN * wc + (lane & 31)) * BK + 8 * chunk;
    }

    f32x16_t acc[IM][JN];
#pragma unroll
    for (int i = 0; i < IM; ++i)
#pragma unroll
        for (int j = 0; j < JN; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

    const uint32_t nk = N / BK;
    auto dma_slice = [&](uint32_t kt, uint16_t* st) __attribute__((always_inline)) {
        gm_dma<C::WAVES, C::A_DMA, C::CPR>(ra, row_bytes, kt * BK * 2, st);
        if constexpr (!SW) {
            gm_dma<C::WAVES, C::B_DMA, C::CPR>(rb, row_bytes, kt * BK * 2, st + C::A_ELEMS);
        } else {
            // One DMA instruction fills 64 / CPR rows inside one 32-row block.
            const int wave_s = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
            for (int j = 0; j < C::B_DMA; ++j) {
                const int blk = wave_s + C::WAVES * j;
                const uint32_t r = (64 / C::CPR) * blk + lane / C::CPR;  // tile row
                const uint32_t b32 = ((64 / C::CPR) * blk) / 32;         // its 32-row block
                const uint32_t src = 32 * (b32 / 2) + r % 32;            // row of gate / up
                const uint32_t logical = (lane % C::CPR) ^ gm_swz<C::CPR>(r);
                dma16(b32 & 1 ? rb_up : rb, st + C::A_ELEMS + 512 * blk,
                      src * row_bytes + kt * BK * 2 + 16 * logical);
            }
        }
    };
    // Step kt: wait for slice kt, barrier, start slice kt + 1 into the stage
    // step kt - 1 read, then KS k-steps of MFMAs from stage kt % 2.
    auto step = [&](uint32_t kt, const uint16_t* cur, uint16_t* nxt) __attribute__((always_inline)) {
        __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
        // The reads of step kt - 1 have all been consumed by its MFMAs; the
        // memory clobber keeps this step's reads and DMA below the barrier.
        asm volatile("s_barrier" ::: "memory");
        if (kt + 1 < nk) dma_slice(kt + 1, nxt);
        // Operands of k-step s + 1 are read while the MFMAs of k-step s run
        // (two register sets).
        bf16x8_t a[2][IM], b[2][JN];
        auto read = [&](int s) __attribute__((always_inline)) {
#pragma unroll
            for (int i = 0; i < IM; ++i)
                a[s & 1][i] = as_bf16x8(*reinterpret_cast<const uint4*>(cur + a_off[s] + 32 * BK * i));
#pragma unroll
            for (int j = 0; j < JN; ++j)
                b[s & 1][j] = as_bf16x8(*reinterpret_cast<const uint4*>(cur + b_off[s] + 32 * BK * j));
        };
        read(0);
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            if (s < KS - 1) read(s + 1);
#pragma unroll
            for (int i = 0; i < IM; ++i)
#pragma unroll
                for (int j = 0; j < JN; ++j)
                    acc[i][j] = mfma32x32x16(b[s & 1][j], a[s & 1][i], acc[i][j]);  // W rows first
        }
        // Schedule: reads of k-steps 0 and 1, then each k-step's MFMAs
        // followed by the reads of the k-step after the next.
        __builtin_amdgcn_sched_group_barrier(0x100, 2 * (IM + JN), 0);
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            __builtin_amdgcn_sched_group_barrier(0x008, IM * JN, 0);
            if (s < KS - 2) __builtin_amdgcn_sched_group_barrier(0x100, IM + JN, 0);
        }
    };
    dma_slice(0, s_0);
    for (uint32_t kt = 0; kt < nk; kt += 2) {
        step(kt, s_0, s_1);
        if (kt + 1 < nk) step(kt + 1, s_1, s_0);
    }

    // Block (i, j), W rows first: lane l value v is output column
    // 32 (JN wc + j) + 8 (v / 4) + 4 (l / 32) + v % 4 of token row
    // 32 (IM wr + i) + l % 32, so v / 4 picks four consecutive outputs of one
    // token.  Each wave stages its bf16 results (rows of OUTC outputs) in
    // its part of the ring slot the last step did not read, R token blocks
    // at a time, and writes whole 16-byte chunks of token rows.
    constexpr int OUTC = SW ? 32 : 32 * JN;  // a wave's output columns
    constexpr int CR = OUTC / 8;             // 16-byte chunks per staged row
    constexpr int AREA = (C::A_ELEMS + C::B_ELEMS) / C::WAVES;  // elements per wave
    constexpr int R = IM < AREA / (32 * OUTC) ? IM : AREA / (32 * OUTC);
    static_assert(R >= 1 && (CR == 4 || CR == 8 || CR == 12), "epilogue staging");
    constexpr int PER_LANE = 32 * R * CR / 64;  // chunks a lane moves per round (R CR is even)
    uint16_t* const area = (nk % 2 ? s_1 : s_0) + wave * AREA;
    const uint32_t col0 = m0 + OUTC * wc;
    const bool residual = !SW && g.residual;
    // Whole 16-byte stores need every row start 16-byte aligned.
    const bool vec = M % 8 == 0 && (reinterpret_cast<uintptr_t>(y) & 15) == 0;
#pragma unroll
    for (int r0 = 0; r0 < IM; r0 += R) {
        const int nb = IM - r0 < R ? IM - r0 : R;  // token blocks this round
        const uint32_t row0 = t0 + 32 * (IM * wr + r0);
        // This round's old values first, so that their latency overlaps
        // the staging.
        uint4 old[PER_LANE];
        if (residual) {
#pragma unroll
            for (int k = 0; k < PER_LANE; ++k) {
                const int idx = lane + 64 * k, t = idx / CR, c = idx % CR;
                const uint32_t tok = row0 + t, m = col0 + 8 * c;
                old[k] = make_uint4(0, 0, 0, 0);
                if (vec && t < 32 * nb && tok < T && m < M)
                    old[k] = *reinterpret_cast<const uint4*>(y + (size_t)tok * M + m);
            }
        }
#pragma unroll
        for (int ii = 0; ii < R; ++ii) {
            if (ii >= nb) break;
            const int i = r0 + ii, t = 32 * ii + (lane & 31);
#pragma unroll
            for (int j = 0; j < OUTC / 32; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    float e[4];
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        if constexpr (SW)
                            e[u] = swiglu1(bf16_to_f32(f32_to_bf16(acc[i][0][4 * q + u])),
                                           bf16_to_f32(f32_to_bf16(acc[i][1][4 * q + u])));
                        else
                            e[u] = acc[i][j][4 * q + u];
                    }
                    const int pc = ep_chunk<CR>(4 * j + q, t), h = (lane >> 5) ^ ep_swap<CR>(t);
                    ep_write(area + t * OUTC + 8 * pc + 4 * h, pack_bf16x2(e[0], e[1]),
                             pack_bf16x2(e[2], e[3]));
                }
        }
        // Every lane reads its PER_LANE chunks (rows below 32 R: inside this
        // wave's area), then stores those of this round's rows.
        uint4 stg[PER_LANE];
        {
            uint32_t a[PER_LANE];
#pragma unroll
            for (int k = 0; k < PER_LANE; ++k) {
                const int idx = lane + 64 * k, t = idx / CR, c = idx % CR;
                a[k] = lds_addr(area + t * OUTC + 8 * ep_chunk<CR>(c, t));
            }
            ep_read<PER_LANE>(stg, a);
        }
#pragma unroll
        for (int k = 0; k < PER_LANE; ++k)
            if (ep_swap<CR>((lane + 64 * k) / CR)) stg[k] = make_uint4(stg[k].z, stg[k].w, stg[k].x, stg[k].y);
        if (vec) {
#pragma unroll
            for (int k = 0; k < PER_LANE; ++k) {
                const int idx = lane + 64 * k, t = idx / CR, c = idx % CR;
                const uint32_t tok = row0 + t, m = col0 + 8 * c;
                if (t < 32 * nb && tok < T && m < M)
                    *reinterpret_cast<uint4*>(y + (size_t)tok * M + m) =
                        residual ? add_bf16x8(old[k], stg[k]) : stg[k];
            }
        } else {
            // Rows not 16-byte aligned or a partial last chunk: element stores.
#pragma unroll
            for (int k = 0; k < PER_LANE; ++k) {
                const int idx = lane + 64 * k, t = idx / CR, c = idx % CR;
                const uint32_t tok = row0 + t, m = col0 + 8 * c;
                if (t >= 32 * nb || tok >= T || m >= M) continue;
                uint16_t* dst = y + (size_t)tok * M + m;
                const uint32_t w[4] = {stg[k].x, stg[k].y, stg[k].z, stg[k].w};
                for (int u = 0; u < 8 && m + u < M; ++u) {
                    const uint16_t val = uint16_t(w[u / 2] >> (16 * (u % 2)));
                    dst[u] = residual ? f32_to_bf16(bf16_to_f32(dst[u]) + bf16_to_f32(val)) : val;
                }
            }
        }
    }
}

template <typename C, bool SW = false>
uint32_t gemm_tiles(const GemmArgs& g) {
    return ((g.T + C::BM - 1) / C::BM) * gm_out_tiles<C, SW>(g);
}

template <typename C>
bool gemm_whole(const GemmArgs& g) {
    for (int sg = 0; sg < g.nseg; ++sg)
        if (g.rows[sg] % C::BN) return false;
    return true;
}

template <typename C, bool SW = false>
hipError_t gemm_launch(const GemmArgs& g, hipStream_t stream) {
    gemm_kernel<C, SW><<<gemm_tiles<C, SW>(g), C::THREADS, 0, stream>>>(g);
    return hipGetLastError();
}

int gemm_cus() {
    static int cus = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            return 256;
        return n;
    }();
    return cus;
}

}  // namespace

hipError_t launch_gemv_bf16(const uint16_t* W, const uint16_t* x, uint16_t* y, uint32_t M,
                            uint32_t N, hipStream_t stream) {
    return gemv_any<1>(W, x, y, 1, M, N, stream);
}

hipError_t launch_gemv_f32(const uint16_t* W, const uint16_t* x, float* y, uint32_t M, uint32_t N,
                           hipStream_t stream) {
    return gemv_any<1>(W, x, y, 1, M, N, stream);
}

bool proj_uses_gemm(uint32_t T, uint32_t N, const void* W, const void* x) {
    return T > kGemvMaxTokens && N % kGmBK == 0 && ((uintptr_t)W | (uintptr_t)x) % 16 == 0;
}

hipError_t launch_batch_proj_bf16(const uint16_t* W, const uint16_t* x, uint16_t* y, uint32_t T,
                                  uint32_t M, uint32_t N, hipStream_t stream) {
    if (T == 1) return gemv_any<1>(W, x, y, T, M, N, stream);
    if (!proj_uses_gemm(T, N, W, x)) return gemv_any<4>(W, x, y, T, M, N, stream);
    GemmArgs g;
    g.x = x;
    g.T = T;
    g.N = N;
    g.w[0] = W;
    g.y[0] = y;
    g.rows[0] = M;
    return launch_gemm(g, stream);
}

hipError_t launch_gemm(const GemmArgs& g, hipStream_t stream) {
    // The largest tile whose tiles alone fill every CU once; 64 x 64 below that.
    const uint32_t cus = (uint32_t)gemm_cus();
    if (g.swiglu) {
        // Tiles with two column blocks per wave: 256 x 256 when they fill the
        // CUs; 192 x 128 when 128 x 128 would need a second round and these do
        // not; else 128 x 128.
        if (gemm_tiles<GmLarge, true>(g) >= cus) return gemm_launch<GmLarge, true>(g, stream);
        if (gemm_tiles<GmSmall, true>(g) > 2 * cus && gemm_tiles<GmTall, true>(g) <= 2 * cus)
            return gemm_launch<GmTall, true>(g, stream);
        return gemm_launch<GmSmall, true>(g, stream);
    }
    if (gemm_tiles<GmLarge>(g) >= cus) return gemm_launch<GmLarge>(g, stream);
    // 128 x 128 tiles that would put two on some CUs and not on others: one
    // 192 x 128 tile per CU when those fit (the stacked q/k/v projections of
    // a 1371-token prompt: 15.7 against 16.5 us).
    if (gemm_tiles<GmSmall>(g) > cus && gemm_tiles<GmTall>(g) <= cus) return gemm_launch<GmTall>(g, stream);
    // 128 x 128 tiles that overflow the two resident workgroups per CU leave
    // a second, mostly idle round: 128 x 192 tiles, when they fit one round
    // (and every segment is whole tiles of 192), take it in one.
    if (gemm_tiles<GmSmall>(g) > 2 * cus && gemm_tiles<GmMid>(g) <= 2 * cus &&
        gemm_whole<GmMid>(g))
        return gemm_launch<GmMid>(g, stream);
    if (gemm_tiles<GmSmall>(g) >= cus) return gemm_launch<GmSmall>(g, stream);
    if (g.N % GmMini::BK == 0) return gemm_launch<GmMini>(g, stream);
    return gemm_launch<GmMini64>(g, stream);
}

}  // namespace tiattn
