// Shared device helpers for the gfx950 (CDNA4) attention kernels.
//
// Wave64 throughout: cross-lane work uses DPP row operations (16-lane rows),
// ds_bpermute only for the one lane^32 exchange per tile.  bf16 values move
// as raw 16-bit patterns; bf16 -> f32 is a shift, f32 -> bf16 is the
// hardware round-to-nearest-even v_cvt_pk_bf16_f32.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tiattn {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;

// s_waitcnt immediates (gfx9 encoding: vmcnt[3:0] and [15:14], expcnt[6:4],
// lgkmcnt[11:8]); the fields not named are left at their maximum (no wait).
constexpr int kWaitVmcnt0 = 0x0F70;  // vmcnt(0)

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float(uint32_t(h) << 16); }

// Two floats -> packed bf16x2 (lo = a), round to nearest even.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    f32x2_t v = {a, b};
    bf16x2_t r = __builtin_convertvector(v, bf16x2_t);
    return __builtin_bit_cast(uint32_t, r);
}
__device__ __forceinline__ uint16_t f32_to_bf16(float a) {
    return uint16_t(pack_bf16x2(a, 0.0f) & 0xffffu);
}

// DPP move within 16-lane rows (row_mask = bank_mask = 0xf).
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xf, 0xf, false));
}
constexpr int kDppXor1 = 0xB1;          // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;          // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;  // lane i <-> 7-i within 8
constexpr int kDppRowMirror = 0x140;      // lane i <-> 15-i within 16

// x of lanes l and l ^ 32 combined, in every lane.  v_permlane32_swap (a
// VALU op, no LDS round trip) leaves lane l with r[0] = x(l & 31) and
// r[1] = x(32 + (l & 31)); both lanes of a pair combine in the same order.
__device__ __forceinline__ float xor32_sum(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_max(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// The same over lanes l and l ^ 16 with v_permlane16_swap:
// r[0] = x(l & ~16), r[1] = x(l | 16).
__device__ __forceinline__ float xor16_sum(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor16_max(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Sum over the 64 lanes of a wave, in every lane: DPP row steps, then the
// lane^16 and lane^32 exchanges.
__device__ __forceinline__ float wave_sum(float x) {
    x += dpp_f32<kDppXor1>(x);
    x += dpp_f32<kDppXor2>(x);
    x += dpp_f32<kDppRowHalfMirror>(x);
    x += dpp_f32<kDppRowMirror>(x);
    x = xor16_sum(x);
    return xor32_sum(x);
}

// Barrier for LDS hand-offs only: waits for this wave's LDS operations but
// leaves its global loads in flight (a plain __syncthreads also drains them).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Buffer resource over [base, base + bytes): loads outside return 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                             0x00020000);
}

// The whole byte offset goes in the VGPR operand (soffset = 0), so that the
// hardware range check sees all of it and returns zeros past the end.
__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, 0));
}

// Same with the non-temporal hint (cache-policy bit nt), for data a launch
// streams exactly once (weights of a one-token projection).
__device__ __forceinline__ uint4 buf_load16_nt(__amdgpu_buffer_rsrc_t r, uint32_t voff) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, 2));
}

// up * silu(gate) on bf16 values (as floats), silu(g) = g / (1 + exp(-g)),
// written as the reference's SwiGLU kernel computes it.
__device__ __forceinline__ float swiglu1(float g, float u) {
    const float silu = g * (1.0f / (1.0f + expf(-g)));
    return u * silu;
}

// 16 bytes from global memory into LDS at `lds` (buffer-load DMA: the 64
// lanes' 16-byte chunks land contiguously in lane order from the wave's
// first lane's address).
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint16_t* lds, uint32_t voff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16,
                                             voff, 0, 0, 0);
}

// acc + the sum of the eight bf16 values packed in v (v_dot2_f32_bf16 with ones).
__device__ __forceinline__ float sum_bf16x8(uint4 v, float acc) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    const bf16x2_t one = __builtin_bit_cast(bf16x2_t, 0x3f803f80u);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, v.x), one, acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, v.y), one, acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, v.z), one, acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, v.w), one, acc, false);
    return acc;
}

// Slot i (< 3) of a three-slot kernel-argument array, by selects: an indexed
// access with a run-time i becomes a vector load from the argument block,
// whose wait then holds back every load that depends on the result.
template <typename T>
__device__ __forceinline__ T pick3(const T (&v)[3], int i) {
    return i == 0 ? v[0] : (i == 1 ? v[1] : v[2]);
}

// Segment of unit u among up to three stacked segments of span[s] units
// each; u is made relative to its segment.
__device__ __forceinline__ int segment_of(const uint32_t (&span)[3], int nseg, uint32_t& u) {
    int seg = 0;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        if (seg == s && s + 1 < nseg && u >= span[s]) {
            u -= span[s];
            seg = s + 1;
        }
    }
    return seg;
}

__device__ __forceinline__ uint32_t word_of(const uint4& v, int i) {
    return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}

__device__ __forceinline__ uint4 ldg16(const void* p) {
    return *reinterpret_cast<const uint4*>(p);
}

// 16-byte load with the non-temporal hint, for data read exactly once (a
// decode pass over the KV cache): streaming reads then run at 6.4-6.6 TB/s
// where plain loads of the same pattern reach 5.6-5.9 TB/s.
__device__ __forceinline__ uint4 ldg16_nt(const void* p) {
    typedef unsigned v4u_t __attribute__((ext_vector_type(4)));
    const v4u_t v = __builtin_nontemporal_load(reinterpret_cast<const v4u_t*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// 16-byte store with the non-temporal hint, for output that is not read
// again by the kernel; whole 128-byte lines per instruction keep it from
// being split into partial-line writes.
__device__ __forceinline__ void stg16_nt(void* p, uint4 v) {
    typedef unsigned v4u_t __attribute__((ext_vector_type(4)));
    __builtin_nontemporal_store(v4u_t{v.x, v.y, v.z, v.w}, reinterpret_cast<v4u_t*>(p));
}

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8_t, v); }

__device__ __forceinline__ f32x16_t mfma32x32x16(bf16x8_t a, bf16x8_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4_t mfma16x16x32(bf16x8_t a, bf16x8_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

}  // namespace tiattn
