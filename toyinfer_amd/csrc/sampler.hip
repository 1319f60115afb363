// Top-k / top-p sampling over fp32 logits on the device: the reference's
// Sampler::sample (src/sampler.cpp:18-67), which runs on the host over logits
// copied back every step (src/engine.cpp:183-190, 443-468).  Here the logits
// stay in HBM and the pick is one launch that a hipGraph can hold.
//
// Same arithmetic as the reference, in its order:
//   x_i = logit_i / T                          (src/sampler.cpp:24-27)
//   top-k set of x (k = min(top_k, vocab))     (:29-32, quick select)
//   p_i = exp((x_i - max x) / T) / sum         (:33-44; T enters twice)
//   sort by p descending, keep the shortest prefix whose running sum
//   exceeds top_p                              (:45-57)
//   coin = u * (that prefix's sum); the first kept token whose running sum
//   exceeds the coin                           (:58-67)
// The uniform draw u comes from the caller (a device float) or, in the model
// harness, from a counter-based hash of (seed, position), so a replayed graph
// draws a fresh coin per step without host work.
//
// Layout: G workgroups of 256 threads (G = 64 for k <= 128, else 32).
// Workgroup b takes the contiguous
// chunk b of the logits (at most 8192, held in registers: element j*256 + t
// in thread t's j-th slot), finds its local k-th largest key by a radix
// select (four 8-bit digit passes over per-wave LDS histograms), and writes
// its top k (keys and indices) to the workspace.  The last workgroup to
// finish (an agent-scope ticket) runs the same select over the G*k
// candidates, sorts the k survivors (in one wave's registers for k <= 64,
// in LDS above), and does the softmax, the top-p cut and the coin walk with
// lane or block scans.  Ties at the k-th value keep the lowest indices;
// equal values are ordered by index.
#include <hip/hip_runtime.h>

#include "../../include/toyinfer_attn.h"
#include "common.hpp"
#include "kernels.hpp"

namespace tiattn {
namespace {

constexpr int kSpThreads = 256, kSpWaves = kSpThreads / 64;
constexpr int kSpPer = 32;                             // keys per thread, held in registers
constexpr uint32_t kSpChunk = kSpPer * kSpThreads;     // logits (or candidates) per workgroup
// 64 workgroups for k <= 128 (half the chunk per workgroup), 32 above, so
// that the merge's blocks * k candidates always fit one workgroup's slots.
constexpr int kSpBlocksSmallK = 64, kSpBlocksLargeK = 32, kSpSmallK = 128;
static_assert(kSampleMaxK <= kSpThreads, "one thread per kept candidate");
static_assert(kSpBlocksSmallK * kSpSmallK <= kSpChunk && kSpBlocksLargeK * kSampleMaxK <= kSpChunk,
              "candidates fit the per-thread key slots");
static_assert(kSpBlocksLargeK * kSpChunk >= kSampleMaxVocab, "every chunk fits one workgroup");
constexpr uint32_t kSpMaxCand = kSpChunk;

// Workspace: [0, 8) argmax key, [8, 12) argmax ticket, [12, 16) sampler
// ticket, then keys [32][k] and indices [32][k] from byte 256.
constexpr size_t kSpCandOff = 256;

// Order-preserving map of a float to an unsigned key (larger float, larger key).
__device__ __forceinline__ uint32_t sp_key(float x) {
    const uint32_t b = __float_as_uint(x);
    return b ^ ((b >> 31) ? 0xffffffffu : 0x80000000u);
}
__device__ __forceinline__ float sp_val(uint32_t k) {
    return __uint_as_float((k >> 31) ? (k ^ 0x80000000u) : ~k);
}

// Exclusive prefix sum of one value per thread over the workgroup.
template <typename T>
__device__ __forceinline__ T block_scan_excl(T v, T* s_w, T& total) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    T x = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const T y = __shfl_up(x, o);
        if (lane >= o) x += y;
    }
    if (lane == 63) s_w[w] = x;
    __syncthreads();
    T base = 0;
    total = 0;
#pragma unroll
    for (int i = 0; i < kSpWaves; ++i) {
        if (i < w) base += s_w[i];
        total += s_w[i];
    }
    __syncthreads();
    return base + x - v;
}

// Inclusive prefix sum over the 64 lanes of a wave with DPP row shifts and
// row broadcasts (no LDS round trips): within each row of 16 lanes by
// shifts of 1, 2, 3, then 4 and 8 on the upper banks; then row 1 and 3 take
// lane 15 of the row before, rows 2 and 3 lane 31.
__device__ __forceinline__ uint32_t wave_scan_incl(uint32_t v) {
    uint32_t s = v;
    s += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xf, 0xf, true);
    s += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xf, 0xf, true);
    s += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x113, 0xf, 0xf, true);
    s += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)s, 0x114, 0xf, 0xe, true);
    s += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)s, 0x118, 0xf, 0xc, true);
    s += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)s, 0x142, 0xa, 0xf, true);
    s += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)s, 0x143, 0xc, 0xf, true);
    return s;
}
template <int CTRL, int ROWS, int BANKS>
__device__ __forceinline__ float dpp_f(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, ROWS, BANKS, true));
}
__device__ __forceinline__ float wave_scan_incl(float v) {
    float s = v + dpp_f<0x111, 0xf, 0xf>(v);
    s += dpp_f<0x112, 0xf, 0xf>(v);
    s += dpp_f<0x113, 0xf, 0xf>(v);
    s += dpp_f<0x114, 0xf, 0xe>(s);
    s += dpp_f<0x118, 0xf, 0xc>(s);
    s += dpp_f<0x142, 0xa, 0xf>(s);
    s += dpp_f<0x143, 0xc, 0xf>(s);
    return s;
}
// The value of lane l - 1 (0 for lane 0): DPP wave_shr:1.
__device__ __forceinline__ float lane_before(float x) { return dpp_f<0x138, 0xf, 0xf>(x); }
__device__ __forceinline__ uint32_t read_lane(uint32_t x, int l) {
    return (uint32_t)__builtin_amdgcn_readlane((int)x, l);
}

struct Sel {
    uint32_t thr;   // the k-th largest key
    uint32_t need;  // how many keys equal to thr belong to the top k
    uint32_t eq;    // how many keys equal thr
};

// The k-th largest of the valid keys of the workgroup (1 <= k <= their
// number): thread t holds element j*256 + t in key[j], valid where bit j of
// `valid` is set.  Four 8-bit digit passes; each wave counts into its own
// histogram (two sets, alternating by pass, so one barrier per pass
// suffices), and every wave then finds the digit itself from the four
// histograms with a lane scan, so no result needs broadcasting.
__device__ __forceinline__ Sel select_kth(const uint32_t (&key)[kSpPer], uint32_t valid, uint32_t k,
                          uint32_t* s_hist, int slots) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    uint32_t prefix = 0, mask = 0, need = k, eq = 0;
#pragma unroll
    for (int pass = 0; pass < 4; ++pass) {
        const int shift = 24 - 8 * pass;
        uint32_t* set = s_hist + (pass & 1) * kSpWaves * 256;
        uint32_t* own = set + w * 256;
        *reinterpret_cast<uint4*>(own + 4 * lane) = make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
        for (int j = 0; j < kSpPer; ++j) {
            if (j >= slots) break;  // workgroup-uniform: slots past the last key are skipped
            if ((valid >> j & 1u) && (key[j] & mask) == prefix)
                atomicAdd(&own[(key[j] >> shift) & 255u], 1u);
        }
        __syncthreads();
        // Lane l: digits 255-4l down to 252-4l, so that the larger digits sit
        // in the lower lanes.  `above` counts larger digits; exactly one digit
        // has above < need <= above + count.
        uint32_t h[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int ww = 0; ww < kSpWaves; ++ww) {
            const uint4 v = *reinterpret_cast<const uint4*>(set + ww * 256 + 252 - 4 * lane);
            h[0] += v.w;
            h[1] += v.z;
            h[2] += v.y;
            h[3] += v.x;
        }
        const uint32_t t = h[0] + h[1] + h[2] + h[3];
        uint32_t above = wave_scan_incl(t) - t;
        int found = -1;
        uint32_t f_need = 0, f_cnt = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (above < need && need <= above + h[i]) {
                found = 255 - 4 * lane - i;
                f_need = need - above;
                f_cnt = h[i];
            }
            above += h[i];
        }
        const int src = __builtin_ctzll(__ballot(found >= 0));
        prefix |= read_lane((uint32_t)found, src) << shift;
        mask |= 255u << shift;
        need = read_lane(f_need, src);
        eq = read_lane(f_cnt, src);
    }
    return {prefix, need, eq};
}

// Bit j set: element j*256 + t is one of the top k.  Keys above thr all are;
// of the keys equal to thr, the `need` with the smallest indices (a second
// select over the complemented indices when there are more).
__device__ __forceinline__ uint32_t top_mask(const uint32_t (&key)[kSpPer], const uint32_t (&idx)[kSpPer],
                             uint32_t valid, const Sel& s, uint32_t* s_hist, int slots) {
    uint32_t take = 0, tie = 0;
    uint32_t nidx[kSpPer];
#pragma unroll
    for (int j = 0; j < kSpPer; ++j) {
        nidx[j] = 0;
        if (j >= slots) break;
        const bool v = valid >> j & 1u;
        take |= (uint32_t)(v && key[j] > s.thr) << j;
        tie |= (uint32_t)(v && key[j] == s.thr) << j;
        nidx[j] = ~idx[j];
    }
    if (s.eq == s.need) return take | tie;  // uniform over the workgroup
    const Sel t = select_kth(nidx, tie, s.need, s_hist, slots);
#pragma unroll
    for (int j = 0; j < kSpPer; ++j) take |= (uint32_t)((tie >> j & 1u) && nidx[j] >= t.thr) << j;
    return take;
}

// Slots 0..k-1 for the set bits of `take` across the workgroup (any order):
// a wave scan of the per-thread counts and one LDS atomic per wave.
template <typename F>
__device__ __forceinline__ void emit_top(uint32_t take, uint32_t k, int slots, uint32_t* s_cnt,
                                         F&& emit) {
    const int lane = threadIdx.x & 63;
    const uint32_t n = __popc(take);
    const uint32_t incl = wave_scan_incl(n);
    uint32_t base = 0;
    if (lane == 63) base = atomicAdd(s_cnt, incl);
    uint32_t slot = read_lane(base, 63) + incl - n;
#pragma unroll
    for (int j = 0; j < kSpPer; ++j)
        if (j < slots && (take >> j & 1u) && slot < k) emit(slot++, j);  // exactly k bits are set
}

// SplitMix64 finaliser (Steele, Lea and Flood, "Fast splittable pseudorandom
// number generators", 2014) of seed + (pos + 1) * golden gamma; the top 24
// bits give u in [0, 1).
__device__ __forceinline__ float sp_coin(uint64_t seed, uint32_t pos) {
    uint64_t z = seed + (uint64_t)(pos + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    return (float)(uint32_t)(z >> 40) * 0x1p-24f;
}

// Writes the picked token (and advances the position) from thread 0.
__device__ __forceinline__ void sp_write(const SampleArgs& a, uint32_t p_out, uint32_t idx,
                                         uint32_t* ticket) {
    *ticket = 0;
    if (a.pos) {
        if (p_out + 1 < a.out_cap) a.out[p_out + 1] = idx;
        *a.pos = p_out + 1;
    } else {
        a.out[0] = idx;
    }
}

__global__ __launch_bounds__(kSpThreads) void sample_kernel(SampleArgs a) {
    __shared__ __align__(16) uint32_t s_hist[2 * kSpWaves * 256];
    __shared__ uint32_t s_wu[kSpWaves];
    __shared__ float s_wf[kSpWaves];
    __shared__ uint64_t s_top[kSampleMaxK];
    __shared__ float s_acc[kSampleMaxK];
    __shared__ uint32_t s_res[2], s_cnt;
    __shared__ bool s_last;

    const uint32_t k = a.k, tid = threadIdx.x;
    char* ws = static_cast<char*>(a.workspace);
    uint32_t* ticket = reinterpret_cast<uint32_t*>(ws + 12);
    uint32_t* ws_key = reinterpret_cast<uint32_t*>(ws + kSpCandOff);
    const uint32_t G = gridDim.x;
    uint32_t* ws_idx = ws_key + G * k;
    if (tid == 0) s_cnt = 0;

    // Phase 1: this workgroup's chunk, element j*256 + t in thread t's key[j].
    const uint32_t cs = (a.n + G - 1) / G;
    const uint32_t c0 = min(a.n, blockIdx.x * cs), m = min(a.n, c0 + cs) - c0;
    uint32_t key[kSpPer], idx[kSpPer], valid = 0;
    {
        // Range-checked buffer loads: no branch per slot, zeros past the chunk.
        const __amdgpu_buffer_rsrc_t r = make_rsrc(a.logits + c0, m * 4);
        const int slots = (int)((m + kSpThreads - 1) / kSpThreads);
        float x[kSpPer];
#pragma unroll
        for (int j = 0; j < kSpPer; ++j)
            x[j] = j < slots ? __uint_as_float((uint32_t)__builtin_amdgcn_raw_buffer_load_b32(
                                   r, 4 * (j * kSpThreads + tid), 0, 0))
                             : 0.0f;
#pragma unroll
        for (int j = 0; j < kSpPer; ++j) {
            const uint32_t e = j * kSpThreads + tid;
            key[j] = sp_key(x[j] / a.temperature);
            idx[j] = c0 + e;
            valid |= (uint32_t)(e < m) << j;
        }
    }
    uint32_t* bk = ws_key + blockIdx.x * k;
    uint32_t* bi = ws_idx + blockIdx.x * k;
    if (m <= k) {
        // The whole chunk; key 0 pads (below every key of a non-NaN float).
#pragma unroll
        for (int j = 0; j < kSpPer; ++j) {
            const uint32_t e = j * kSpThreads + tid;
            if (e < k) {
                bk[e] = e < m ? key[j] : 0u;
                bi[e] = e < m ? idx[j] : 0xffffffffu;
            }
        }
    } else {
        const int slots = (int)((m + kSpThreads - 1) / kSpThreads);
        const Sel s = select_kth(key, valid, k, s_hist, slots);
        const uint32_t take = top_mask(key, idx, valid, s, s_hist, slots);
        emit_top(take, k, slots, &s_cnt, [&](uint32_t slot, int j) {
            bk[slot] = key[j];
            bi[slot] = idx[j];
        });
    }
    // Every wave waits for its own stores to reach the L2, the barrier joins
    // them, and one agent-scope release (not one per wave) publishes the
    // chunk before the ticket; the last workgroup's acquire precedes its reads
    // of the other chunks.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0) {
        __threadfence();
        s_last = atomicAdd(ticket, 1u) == G - 1;
        if (s_last) __threadfence();
        s_cnt = 0;
    }
    __syncthreads();
    if (!s_last) return;

    // Phase 2 (last workgroup): the top k of the G*k candidates, as
    // (key << 32 | ~index) so that one ordering covers the ties.
    const uint32_t nc = G * k;
    valid = 0;
#pragma unroll
    for (int j = 0; j < kSpPer; ++j) {
        const uint32_t e = j * kSpThreads + tid;
        const bool v = e < nc && j < (int)((nc + kSpThreads - 1) / kSpThreads);
        key[j] = v ? ws_key[e] : 0u;
        idx[j] = v ? ws_idx[e] : 0xffffffffu;
        valid |= (uint32_t)v << j;
    }
    {
        const int slots = (int)((nc + kSpThreads - 1) / kSpThreads);
        const Sel s = select_kth(key, valid, k, s_hist, slots);
        const uint32_t take = top_mask(key, idx, valid, s, s_hist, slots);
        emit_top(take, k, slots, &s_cnt, [&](uint32_t slot, int j) {
            s_top[slot] = ((uint64_t)key[j] << 32) | (uint32_t)~idx[j];
        });
    }
    uint32_t p_out = 0;
    if (a.pos) p_out = *a.pos;
    const float u = a.coin ? *a.coin : sp_coin(a.seed, p_out);
    __syncthreads();

    if (k <= 64) {
        // One wave: bitonic sort in registers (descending), then softmax,
        // running sums, the top-p cut and the coin walk with lane scans.
        if (tid >= 64) return;
        const int lane = tid;
        uint64_t v = (uint32_t)lane < k ? s_top[lane] : 0ull;
#pragma unroll
        for (int size = 2; size <= 64; size <<= 1) {
#pragma unroll
            for (int stride = size >> 1; stride > 0; stride >>= 1) {
                const uint64_t o = __shfl_xor(v, stride);
                const bool keep_max = ((lane & stride) == 0) == ((lane & size) == 0);
                v = keep_max ? (v > o ? v : o) : (v < o ? v : o);
            }
        }
        const bool in = (uint32_t)lane < k;
        const float x = sp_val((uint32_t)(v >> 32));
        const float xmax = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(x)));
        const float p = in ? expf((x - xmax) / a.temperature) : 0.0f;
        const float sum = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wave_scan_incl(p)), 63));
        const float acc = wave_scan_incl(p / sum);
        const float prev = lane_before(acc);
        const uint64_t cut = __ballot(in && acc > a.top_p && (lane == 0 || !(prev > a.top_p)));
        const uint32_t kept = cut ? (uint32_t)__builtin_ctzll(cut) + 1 : k;
        const float coin = u * __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), kept - 1));
        const uint64_t hit = __ballot((uint32_t)lane < kept && acc > coin &&
                                      (lane == 0 || !(prev > coin)));
        const int pick = hit ? __builtin_ctzll(hit) : (int)kept - 1;
        const uint64_t chosen = __shfl(v, pick);
        if (lane == 0) sp_write(a, p_out, ~(uint32_t)chosen, ticket);
        return;
    }

    // k > 64: bitonic sort in LDS over the workgroup, block scans.
    if (tid >= k && tid < kSampleMaxK) s_top[tid] = 0;
    uint32_t n2 = 1;
    while (n2 < k) n2 <<= 1;
    for (uint32_t size = 2; size <= n2; size <<= 1) {
        for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
            __syncthreads();
            const uint32_t j = tid ^ stride;
            if (tid < n2 && j > tid) {
                const uint64_t x = s_top[tid], y = s_top[j];
                const bool desc = (tid & size) == 0;
                if ((x < y) == desc) {
                    s_top[tid] = y;
                    s_top[j] = x;
                }
            }
        }
    }
    __syncthreads();
    const float xmax = sp_val((uint32_t)(s_top[0] >> 32));
    const float p = tid < k ? expf((sp_val((uint32_t)(s_top[tid] >> 32)) - xmax) / a.temperature) : 0.0f;
    float sum;
    (void)block_scan_excl(p, s_wf, sum);
    const float q = p / sum;
    float qtot;
    const float acc = block_scan_excl(q, s_wf, qtot) + q;
    if (tid < k) s_acc[tid] = acc;
    if (tid == 0) {
        s_res[0] = k;
        s_res[1] = 0xffffffffu;
    }
    __syncthreads();
    // Kept prefix: through the first running sum above top_p (all k if none).
    if (tid < k && acc > a.top_p && (tid == 0 || !(s_acc[tid - 1] > a.top_p))) s_res[0] = tid + 1;
    __syncthreads();
    const uint32_t kept = s_res[0];
    const float coin = u * s_acc[kept - 1];
    if (tid < kept && acc > coin && (tid == 0 || !(s_acc[tid - 1] > coin))) s_res[1] = tid;
    __syncthreads();
    if (tid == 0) {
        const uint32_t pick = s_res[1] != 0xffffffffu ? s_res[1] : kept - 1;
        sp_write(a, p_out, ~(uint32_t)s_top[pick], ticket);
    }
}

}  // namespace

size_t sample_workspace_bytes() { return kSpCandOff + 2ull * kSpMaxCand * 4; }

int sample_config(uint32_t vocab, float temperature, uint32_t top_k, float top_p, SampleArgs& a) {
    if (vocab == 0 || !(temperature >= 0.0f)) return TOYINFER_ERR_INVALID_ARGUMENT;
    a.n = vocab;
    a.temperature = temperature;
    a.top_p = top_p;
    // src/sampler.cpp:20-22: greedy below 1e-3 or for top_k == 1.
    a.greedy = temperature < 1e-3f || top_k == 1;
    if (a.greedy) {
        a.k = 1;
        return TOYINFER_OK;
    }
    if (top_k == 0) return TOYINFER_ERR_INVALID_ARGUMENT;  // the reference asserts k > 0
    a.k = top_k < vocab ? top_k : vocab;                   // :29-30
    return a.k <= kSampleMaxK && vocab <= kSampleMaxVocab ? TOYINFER_OK : TOYINFER_ERR_UNSUPPORTED;
}

hipError_t launch_sample(const SampleArgs& a, hipStream_t stream) {
    if (a.greedy) {
        char* ws = static_cast<char*>(a.workspace);
        return launch_argmax_wide(a.logits, a.n, a.out, a.pos, a.out_cap,
                                  reinterpret_cast<uint64_t*>(ws), reinterpret_cast<uint32_t*>(ws + 8),
                                  stream);
    }
    sample_kernel<<<a.k <= kSpSmallK ? kSpBlocksSmallK : kSpBlocksLargeK, kSpThreads, 0, stream>>>(a);
    return hipGetLastError();
}

}  // namespace tiattn
