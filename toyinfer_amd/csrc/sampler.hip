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
// Layout: 32 workgroups of 256 threads.  Workgroup b takes the contiguous
// chunk b of the logits (at most 8192), finds its local k-th largest key by an
// LDS radix select (four 8-bit digit passes), and writes its top k (keys and
// indices) to the workspace in index order.  The last workgroup to finish (an
// agent-scope ticket) runs the same select over the 32*k candidates, sorts
// the k survivors (bitonic, in LDS), and does the softmax, the top-p cut and
// the coin walk with block scans.  Ties at the k-th value keep the lowest
// indices; equal values are ordered by index.
#include <hip/hip_runtime.h>

#include "../../include/toyinfer_attn.h"
#include "common.hpp"
#include "kernels.hpp"

namespace tiattn {
namespace {

constexpr int kSpBlocks = 32, kSpThreads = 256;
constexpr uint32_t kSpChunk = kSampleMaxVocab / kSpBlocks;
static_assert(kSampleMaxK <= kSpThreads, "one thread per kept candidate");
static_assert(kSpBlocks * kSampleMaxK <= kSpChunk, "candidates reuse the chunk buffer");

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
    for (int i = 0; i < kSpThreads / 64; ++i) {
        if (i < w) base += s_w[i];
        total += s_w[i];
    }
    __syncthreads();
    return base + x - v;
}

// The k-th largest of s_key[0..m) (1 <= k <= m): its key, and how many of
// the elements equal to it belong to the top k (the rest of the top k is
// strictly larger).
__device__ void radix_select(const uint32_t* s_key, uint32_t m, uint32_t k, uint32_t* s_hist,
                             uint32_t* s_sel, uint32_t& thr, uint32_t& need) {
    uint32_t prefix = 0, mask = 0;
    need = k;
    for (int shift = 24; shift >= 0; shift -= 8) {
        s_hist[threadIdx.x] = 0;
        __syncthreads();
        for (uint32_t i = threadIdx.x; i < m; i += kSpThreads) {
            const uint32_t key = s_key[i];
            if ((key & mask) == prefix) atomicAdd(&s_hist[(key >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (threadIdx.x < 64) {
            // Lane l holds digits 4l..4l+3; `above` counts the elements with a
            // larger digit.  Exactly one digit has above < need <= above + h.
            const int l = threadIdx.x;
            uint32_t h[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) h[j] = s_hist[4 * l + j];
            const uint32_t t = h[0] + h[1] + h[2] + h[3];
            uint32_t suf = t;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const uint32_t y = __shfl_down(suf, o);
                if (l + o < 64) suf += y;
            }
            uint32_t above = suf - t;
#pragma unroll
            for (int j = 3; j >= 0; --j) {
                if (above < need && need <= above + h[j]) {
                    s_sel[0] = 4 * l + j;
                    s_sel[1] = need - above;
                }
                above += h[j];
            }
        }
        __syncthreads();
        prefix |= s_sel[0] << shift;
        mask |= 255u << shift;
        need = s_sel[1];
        __syncthreads();
    }
    thr = prefix;
}

// Calls emit(slot, i) for the top k of s_key[0..m) given the select's result:
// slots [0, k-need) take the larger keys in index order, slots [k-need, k)
// the first `need` keys equal to thr in index order.
template <typename F>
__device__ void compact_top(const uint32_t* s_key, uint32_t m, uint32_t k, uint32_t thr,
                            uint32_t need, uint32_t* s_w, F&& emit) {
    const uint32_t per = (m + kSpThreads - 1) / kSpThreads;
    const uint32_t b = min(m, threadIdx.x * per), e = min(m, b + per);
    uint32_t ngt = 0, neq = 0;
    for (uint32_t i = b; i < e; ++i) {
        const uint32_t key = s_key[i];
        ngt += key > thr;
        neq += key == thr;
    }
    uint32_t tot;
    uint32_t gt = block_scan_excl(ngt, s_w, tot);
    uint32_t eq = block_scan_excl(neq, s_w, tot);
    for (uint32_t i = b; i < e; ++i) {
        const uint32_t key = s_key[i];
        if (key > thr) {
            emit(gt++, i);
        } else if (key == thr) {
            if (eq < need) emit(k - need + eq, i);
            ++eq;
        }
    }
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

__global__ __launch_bounds__(kSpThreads) void sample_kernel(SampleArgs a) {
    __shared__ uint32_t s_key[kSpChunk];
    __shared__ uint32_t s_hist[256];
    __shared__ uint32_t s_sel[2];
    __shared__ uint32_t s_wu[kSpThreads / 64];
    __shared__ float s_wf[kSpThreads / 64];
    __shared__ uint64_t s_top[kSampleMaxK];
    __shared__ float s_acc[kSampleMaxK];
    __shared__ uint32_t s_res[2];
    __shared__ bool s_last;

    const uint32_t k = a.k, tid = threadIdx.x;
    char* ws = static_cast<char*>(a.workspace);
    uint32_t* ticket = reinterpret_cast<uint32_t*>(ws + 12);
    uint32_t* ws_key = reinterpret_cast<uint32_t*>(ws + kSpCandOff);
    uint32_t* ws_idx = ws_key + kSpBlocks * k;

    // Phase 1: this workgroup's chunk.
    const uint32_t cs = (a.n + kSpBlocks - 1) / kSpBlocks;
    const uint32_t c0 = min(a.n, blockIdx.x * cs), m = min(a.n, c0 + cs) - c0;
    for (uint32_t i = tid; i < m; i += kSpThreads) s_key[i] = sp_key(a.logits[c0 + i] / a.temperature);
    __syncthreads();
    uint32_t* bk = ws_key + blockIdx.x * k;
    uint32_t* bi = ws_idx + blockIdx.x * k;
    if (m <= k) {
        // The whole chunk; key 0 pads (below every key of a non-NaN float).
        for (uint32_t i = tid; i < k; i += kSpThreads) {
            bk[i] = i < m ? s_key[i] : 0u;
            bi[i] = i < m ? c0 + i : 0xffffffffu;
        }
    } else {
        uint32_t thr, need;
        radix_select(s_key, m, k, s_hist, s_sel, thr, need);
        compact_top(s_key, m, k, thr, need, s_wu, [&](uint32_t slot, uint32_t i) {
            bk[slot] = s_key[i];
            bi[slot] = c0 + i;
        });
    }
    __threadfence();
    __syncthreads();
    if (tid == 0) s_last = atomicAdd(ticket, 1u) == kSpBlocks - 1;
    __syncthreads();
    if (!s_last) return;
    __threadfence();

    // Phase 2 (last workgroup): the top k of the 32*k candidates.  Within a
    // block's slots, equal keys sit in index order and blocks ascend, so
    // slot order is index order among equal keys.
    const uint32_t nc = kSpBlocks * k;
    for (uint32_t i = tid; i < nc; i += kSpThreads) s_key[i] = ws_key[i];
    if (tid < kSampleMaxK) s_top[tid] = 0;
    __syncthreads();
    {
        uint32_t thr, need;
        radix_select(s_key, nc, k, s_hist, s_sel, thr, need);
        compact_top(s_key, nc, k, thr, need, s_wu, [&](uint32_t slot, uint32_t i) {
            s_top[slot] = ((uint64_t)s_key[i] << 32) | (uint32_t)~ws_idx[i];
        });
    }
    // Bitonic sort, descending: larger key first, then smaller index.
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

    // Softmax over the sorted top k (the first is the largest), running sums.
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
    uint32_t p_out = 0;
    if (a.pos) p_out = *a.pos;
    const float u = a.coin ? *a.coin : sp_coin(a.seed, p_out);
    const float coin = u * s_acc[kept - 1];
    if (tid < kept && acc > coin && (tid == 0 || !(s_acc[tid - 1] > coin))) s_res[1] = tid;
    __syncthreads();
    if (tid == 0) {
        const uint32_t pick = s_res[1] != 0xffffffffu ? s_res[1] : kept - 1;
        const uint32_t idx = ~(uint32_t)s_top[pick];
        *ticket = 0;
        if (a.pos) {
            if (p_out + 1 < a.out_cap) a.out[p_out + 1] = idx;
            *a.pos = p_out + 1;
        } else {
            a.out[0] = idx;
        }
    }
}

}  // namespace

size_t sample_workspace_bytes() { return kSpCandOff + 2ull * kSpBlocks * kSampleMaxK * 4; }

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
    sample_kernel<<<kSpBlocks, kSpThreads, 0, stream>>>(a);
    return hipGetLastError();
}

}  // namespace tiattn
