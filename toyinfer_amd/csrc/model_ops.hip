// Decoder-layer row and element-wise ops around attention and the
// projections: full-row RMSNorm, residual add, SwiGLU, embedding gather and
// greedy argmax (the rest of a Qwen3 forward).  All are HBM- or
// latency-bound; rounding points follow the reference's kernels (fp32
// arithmetic, one round to bf16 at the store).
#include <initializer_list>

#include "common.hpp"
#include "kernels.hpp"

namespace tiattn {
namespace {

constexpr int kRowThreads = 256;

// Workgroup-wide sum (kRowThreads lanes) in every lane.
__device__ __forceinline__ float block_sum(float x, float* s_red) {
    x = wave_sum(x);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) s_red[wave] = x;
    __syncthreads();
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < kRowThreads / 64; ++w) s += s_red[w];
    return s;
}

// One workgroup per row of `size` values.  sum = sum of squares (fp32 FMA per
// element, then a tree), inv = rsqrt(sum / size + eps), y = bf16(x * inv * w).
// sum_out[row] receives the sum of squares, as the reference's `sum` buffer
// does.  VEC = 8 moves 16-byte chunks (size % 8 == 0, 16-byte aligned rows),
// VEC = 2 bf16 pairs.  y may be x: each lane rewrites only the chunks it
// read.
template <int VEC>
__global__ __launch_bounds__(kRowThreads) void rmsnorm_rows_kernel(
    const uint16_t* x, const uint16_t* __restrict__ w, uint16_t* y, float* __restrict__ sum_out,
    float eps, uint32_t size) {
    __shared__ float s_red[kRowThreads / 64];
    const uint16_t* xr = x + (size_t)blockIdx.x * size;
    uint16_t* yr = y + (size_t)blockIdx.x * size;
    float ss = 0.0f;
    for (uint32_t c = threadIdx.x * VEC; c < size; c += kRowThreads * VEC) {
        if constexpr (VEC == 8) {
            const uint4 v = ldg16(xr + c);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t wd = word_of(v, i);
                ss = fmaf(bf16_lo(wd), bf16_lo(wd), ss);
                ss = fmaf(bf16_hi(wd), bf16_hi(wd), ss);
            }
        } else {
            const uint32_t wd = *reinterpret_cast<const uint32_t*>(xr + c);
            ss = fmaf(bf16_lo(wd), bf16_lo(wd), ss);
            ss = fmaf(bf16_hi(wd), bf16_hi(wd), ss);
        }
    }
    const float sum = block_sum(ss, s_red);
    if (threadIdx.x == 0 && sum_out) sum_out[blockIdx.x] = sum;
    const float inv = rsqrtf(fmaf(sum, 1.0f / (float)size, eps));
    for (uint32_t c = threadIdx.x * VEC; c < size; c += kRowThreads * VEC) {
        if constexpr (VEC == 8) {
            const uint4 v = ldg16(xr + c), g = ldg16(w + c);
            uint4 o;
            uint32_t* ow = reinterpret_cast<uint32_t*>(&o);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t a = word_of(v, i), b = word_of(g, i);
                ow[i] = pack_bf16x2(bf16_lo(a) * inv * bf16_lo(b), bf16_hi(a) * inv * bf16_hi(b));
            }
            *reinterpret_cast<uint4*>(yr + c) = o;
        } else {
            const uint32_t a = *reinterpret_cast<const uint32_t*>(xr + c);
            const uint32_t b = *reinterpret_cast<const uint32_t*>(w + c);
            *reinterpret_cast<uint32_t*>(yr + c) =
                pack_bf16x2(bf16_lo(a) * inv * bf16_lo(b), bf16_hi(a) * inv * bf16_hi(b));
        }
    }
}

// hidden[i] = bf16(hidden[i] + residual[i]); VEC values per lane.
template <int VEC>
__global__ void residual_add_kernel(const uint16_t* __restrict__ residual,
                                    uint16_t* __restrict__ hidden, size_t n) {
    const size_t i = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * VEC;
    if (i >= n) return;
    if constexpr (VEC == 8) {
        const uint4 r = ldg16(residual + i), h = ldg16(hidden + i);
        uint4 o;
        uint32_t* ow = reinterpret_cast<uint32_t*>(&o);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t a = word_of(h, k), b = word_of(r, k);
            ow[k] = pack_bf16x2(bf16_lo(a) + bf16_lo(b), bf16_hi(a) + bf16_hi(b));
        }
        *reinterpret_cast<uint4*>(hidden + i) = o;
    } else {
        const uint32_t a = *reinterpret_cast<const uint32_t*>(hidden + i);
        const uint32_t b = *reinterpret_cast<const uint32_t*>(residual + i);
        *reinterpret_cast<uint32_t*>(hidden + i) =
            pack_bf16x2(bf16_lo(a) + bf16_lo(b), bf16_hi(a) + bf16_hi(b));
    }
}


// out[i] = bf16(up[i] * silu(gate[i])), silu(g) = g / (1 + exp(-g)).
template <int VEC>
__global__ void swiglu_kernel(const uint16_t* __restrict__ gate, const uint16_t* __restrict__ up,
                              uint16_t* __restrict__ out, size_t n) {
    const size_t i = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * VEC;
    if (i >= n) return;
    if constexpr (VEC == 8) {
        const uint4 g = ldg16(gate + i), u = ldg16(up + i);
        uint4 o;
        uint32_t* ow = reinterpret_cast<uint32_t*>(&o);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t a = word_of(g, k), b = word_of(u, k);
            ow[k] = pack_bf16x2(swiglu1(bf16_lo(a), bf16_lo(b)), swiglu1(bf16_hi(a), bf16_hi(b)));
        }
        *reinterpret_cast<uint4*>(out + i) = o;
    } else {
        const uint32_t a = *reinterpret_cast<const uint32_t*>(gate + i);
        const uint32_t b = *reinterpret_cast<const uint32_t*>(up + i);
        *reinterpret_cast<uint32_t*>(out + i) =
            pack_bf16x2(swiglu1(bf16_lo(a), bf16_lo(b)), swiglu1(bf16_hi(a), bf16_hi(b)));
    }
}

// hidden[t] = table[ids[t]] (rows of `size` values).  Ids at or past `vocab`
// read as zeros: the table is read through a buffer resource of exactly
// vocab rows.  VEC as above.
template <int VEC>
__global__ void gather_rows_kernel(const uint16_t* __restrict__ table,
                                   const uint32_t* __restrict__ ids, uint16_t* __restrict__ out,
                                   uint32_t size, uint32_t vocab) {
    const uint32_t t = blockIdx.y;
    const uint32_t c = (blockIdx.x * blockDim.x + threadIdx.x) * VEC;
    if (c >= size) return;
    const uint32_t id = ids[t];
    const uint64_t row_bytes = 2ull * size;
    const uint16_t* row = table + (size_t)min(id, vocab - 1) * size;
    const auto r = make_rsrc(row, id < vocab ? (uint32_t)row_bytes : 0u);
    uint16_t* dst = out + (size_t)t * size + c;
    if constexpr (VEC == 8) {
        *reinterpret_cast<uint4*>(dst) = buf_load16(r, c * 2);
    } else {
        *reinterpret_cast<uint32_t*>(dst) = __builtin_amdgcn_raw_buffer_load_b32(r, c * 2, 0, 0);
    }
}

// Index of the first maximum of logits[0..n) under strict '>' from -FLT_MAX
// (NaN never wins; UINT32_MAX when no value exceeds -FLT_MAX), as the
// reference's host sampler.  One workgroup of 1024 lanes.  If pos_d is given,
// the index goes to out[*pos_d + 1] and *pos_d advances by one (the decode
// loop's next token and position, read on the device); else to out[0].
constexpr int kArgmaxThreads = 1024;

__global__ __launch_bounds__(kArgmaxThreads) void argmax_kernel(const float* __restrict__ logits,
                                                                uint32_t n, uint32_t* out,
                                                                uint32_t* pos_d, uint32_t out_cap) {
    __shared__ float s_v[kArgmaxThreads / 64];
    __shared__ uint32_t s_i[kArgmaxThreads / 64];
    float best = -3.402823466e38f;
    uint32_t bi = 0xffffffffu;
    for (uint32_t i = threadIdx.x; i < n; i += kArgmaxThreads) {
        const float v = logits[i];
        if (v > best) {
            best = v;
            bi = i;
        }
    }
    // Wave: larger value wins, the smaller index on ties.
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float ov = __shfl_xor(best, off);
        const uint32_t oi = __shfl_xor(bi, off);
        if (ov > best || (ov == best && oi < bi)) {
            best = ov;
            bi = oi;
        }
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) {
        s_v[wave] = best;
        s_i[wave] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < kArgmaxThreads / 64; ++w)
            if (s_v[w] > best || (s_v[w] == best && s_i[w] < bi)) {
                best = s_v[w];
                bi = s_i[w];
            }
        if (pos_d) {
            const uint32_t p = *pos_d;
            if (p + 1 < out_cap) out[p + 1] = bi;
            *pos_d = p + 1;
        } else {
            out[0] = bi;
        }
    }
}

// The decode step's first kernel: hidden = table[ids[*pos_d]] (the token
// at the current position), seq_len_d[0] = min(*pos_d, cap - 1) + 1 and,
// when rope_row is given, rope_row = row pos of the rotary table
// (rope_floats floats), so that later kernels of the step read the
// position's angles without waiting for the position first.
template <int VEC>
__global__ void decode_step_setup_kernel(const uint16_t* __restrict__ table,
                                         const uint32_t* __restrict__ ids,
                                         const uint32_t* __restrict__ pos_d,
                                         uint16_t* __restrict__ hidden, uint32_t* seq_len_d,
                                         uint32_t size, uint32_t vocab, uint32_t cap,
                                         const float* __restrict__ rope_table,
                                         float* __restrict__ rope_row, uint32_t rope_floats) {
    const uint32_t pos = min(*pos_d, cap - 1);
    const uint32_t c = (blockIdx.x * blockDim.x + threadIdx.x) * VEC;
    if (blockIdx.x == 0 && threadIdx.x == 0) seq_len_d[0] = pos + 1;
    if (blockIdx.x == 0 && rope_row) {
        for (uint32_t i = threadIdx.x; i < rope_floats; i += blockDim.x)
            rope_row[i] = rope_table[(size_t)pos * rope_floats + i];
    }
    if (c >= size) return;
    const uint32_t id = ids[pos];
    const uint16_t* row = table + (size_t)min(id, vocab - 1) * size;
    const auto r = make_rsrc(row, id < vocab ? 2u * size : 0u);
    if constexpr (VEC == 8) {
        *reinterpret_cast<uint4*>(hidden + c) = buf_load16(r, c * 2);
    } else {
        *reinterpret_cast<uint32_t*>(hidden + c) = __builtin_amdgcn_raw_buffer_load_b32(r, c * 2, 0, 0);
    }
}

__global__ void set_u32_kernel(uint32_t* p, uint32_t v) { *p = v; }

bool vec8_ok(uint32_t size, std::initializer_list<const void*> ptrs) {
    if (size % 8 != 0) return false;
    for (const void* p : ptrs)
        if ((uintptr_t)p % 16 != 0) return false;
    return true;
}

}  // namespace

hipError_t launch_rmsnorm_rows(const uint16_t* x, const uint16_t* w, uint16_t* y, float* sum_out,
                               float eps, uint32_t rows, uint32_t size, hipStream_t stream) {
    if (vec8_ok(size, {x, w, y}))
        rmsnorm_rows_kernel<8><<<rows, kRowThreads, 0, stream>>>(x, w, y, sum_out, eps, size);
    else
        rmsnorm_rows_kernel<2><<<rows, kRowThreads, 0, stream>>>(x, w, y, sum_out, eps, size);
    return hipGetLastError();
}

hipError_t launch_residual_add(const uint16_t* residual, uint16_t* hidden, size_t n,
                               hipStream_t stream) {
    constexpr int kT = 256;
    if (n % 8 == 0 && (((uintptr_t)residual | (uintptr_t)hidden) % 16) == 0)
        residual_add_kernel<8><<<(unsigned)((n / 8 + kT - 1) / kT), kT, 0, stream>>>(residual, hidden, n);
    else
        residual_add_kernel<2><<<(unsigned)((n / 2 + kT - 1) / kT), kT, 0, stream>>>(residual, hidden, n);
    return hipGetLastError();
}

hipError_t launch_swiglu(const uint16_t* gate, const uint16_t* up, uint16_t* out, size_t n,
                         hipStream_t stream) {
    constexpr int kT = 256;
    if (n % 8 == 0 && (((uintptr_t)gate | (uintptr_t)up | (uintptr_t)out) % 16) == 0)
        swiglu_kernel<8><<<(unsigned)((n / 8 + kT - 1) / kT), kT, 0, stream>>>(gate, up, out, n);
    else
        swiglu_kernel<2><<<(unsigned)((n / 2 + kT - 1) / kT), kT, 0, stream>>>(gate, up, out, n);
    return hipGetLastError();
}

hipError_t launch_gather_rows(const uint16_t* table, const uint32_t* ids, uint16_t* out,
                              uint32_t tokens, uint32_t size, uint32_t vocab, hipStream_t stream) {
    constexpr int kT = 128;
    if (vec8_ok(size, {table, out})) {
        const dim3 grid((size / 8 + kT - 1) / kT, tokens);
        gather_rows_kernel<8><<<grid, kT, 0, stream>>>(table, ids, out, size, vocab);
    } else {
        const dim3 grid((size / 2 + kT - 1) / kT, tokens);
        gather_rows_kernel<2><<<grid, kT, 0, stream>>>(table, ids, out, size, vocab);
    }
    return hipGetLastError();
}

hipError_t launch_argmax(const float* logits, uint32_t n, uint32_t* out, uint32_t* pos_d,
                         uint32_t out_cap, hipStream_t stream) {
    argmax_kernel<<<1, kArgmaxThreads, 0, stream>>>(logits, n, out, pos_d, out_cap);
    return hipGetLastError();
}

hipError_t launch_decode_step_setup(const uint16_t* table, const uint32_t* ids,
                                    const uint32_t* pos_d, uint16_t* hidden, uint32_t* seq_len_d,
                                    uint32_t size, uint32_t vocab, uint32_t cap,
                                    hipStream_t stream, const float* rope_table, float* rope_row,
                                    uint32_t rope_floats) {
    constexpr int kT = 128;
    if (vec8_ok(size, {table, hidden}))
        decode_step_setup_kernel<8><<<(size / 8 + kT - 1) / kT, kT, 0, stream>>>(
            table, ids, pos_d, hidden, seq_len_d, size, vocab, cap, rope_table, rope_row,
            rope_floats);
    else
        decode_step_setup_kernel<2><<<(size / 2 + kT - 1) / kT, kT, 0, stream>>>(
            table, ids, pos_d, hidden, seq_len_d, size, vocab, cap, rope_table, rope_row,
            rope_floats);
    return hipGetLastError();
}

hipError_t launch_set_u32(uint32_t* p, uint32_t value, hipStream_t stream) {
    set_u32_kernel<<<1, 1, 0, stream>>>(p, value);
    return hipGetLastError();
}

}  // namespace tiattn
