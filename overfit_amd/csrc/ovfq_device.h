// ovfq_device.h — gfx950 device helpers shared by the ovfq kernels.
//
// All global reads of weights and activations go through buffer resources (V#) built with
// __builtin_amdgcn_make_buffer_rsrc: a read past the resource's byte range returns 0 instead of touching
// memory, so a partial tile at the end of a matrix can never fault. Offsets are 32-bit, so every kernel
// rebases its resources at the rows it owns.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ovfq {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
typedef short s16x2 __attribute__((ext_vector_type(2)));

constexpr int kQK = 256;
constexpr int kQ4KBytes = 144;
constexpr int kQ6KBytes = 210;
constexpr int kWave = 64;

// Word 3 of a gfx9 buffer descriptor: 32-bit dword data format, no swizzle.
constexpr int kRsrcWord3 = 0x00020000;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kRsrcWord3);
}

// Byte count a resource may cover starting at `base_off` into a `total`-byte allocation (clamped to 4 GiB-1).
__host__ __device__ __forceinline__ uint32_t rsrc_bytes(uint64_t total, uint64_t base_off) {
    uint64_t rem = total > base_off ? total - base_off : 0;
    return rem > 0xffffffffull ? 0xffffffffu : (uint32_t)rem;
}

__device__ __forceinline__ u32x4 ld4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
}
__device__ __forceinline__ u32x3 ld3(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b96(r, (int)off, 0, 0);
}
__device__ __forceinline__ u32x2 ld2(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0);
}
__device__ __forceinline__ uint32_t ld1(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0);
}

// Reinterpret a 32-bit word as fp32. Always pass a scalar: __builtin_bit_cast applied directly to an
// ext_vector element (v.y) reads element 0 with this compiler, so vector lanes are copied out first.
__device__ __forceinline__ float as_float(uint32_t u) { return __builtin_bit_cast(float, u); }

// Exact fp16 -> fp32 widening (v_cvt_f32_f16; fp16 denormals are preserved in the default MODE).
__device__ __forceinline__ float half_lo(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xffffu));
}
__device__ __forceinline__ float half_hi(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
}

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}
// Sum of the two signed 16-bit halves of w, times k, plus c (v_dot2_i32_i16 with both halves of b = k).
__device__ __forceinline__ int sdot2_k(uint32_t w, int k, int c) {
    s16x2 b = {(short)k, (short)k};
    return __builtin_amdgcn_sdot2(__builtin_bit_cast(s16x2, w), b, c, false);
}

// Sum over the 4 lanes of a quad; every lane of the quad receives the total (exact: integer adds).
__device__ __forceinline__ int quad_sum(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0xb1, 0xf, 0xf, false);  // quad_perm [1,0,3,2]
    v += __builtin_amdgcn_update_dpp(0, v, 0x4e, 0xf, 0xf, false);  // quad_perm [2,3,0,1]
    return v;
}

// Wave-local ordering point for LDS traffic between lanes of the same wave.
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

// fp32 -> fp16 bits, round to nearest even, overflow to infinity: the (Half)x conversion of .NET, written out
// in integer arithmetic so the encoders do not depend on the MODE register.
__device__ __forceinline__ uint16_t float_to_half_rne(float f) {
    uint32_t x = __builtin_bit_cast(uint32_t, f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xffu;
    uint32_t mant = x & 0x7fffffu;
    if (exp == 0xffu) return (uint16_t)(sign | (mant ? (0x7e00u | (mant >> 13)) : 0x7c00u));
    int e = (int)exp - 112;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        uint32_t m = mant | 0x800000u;
        int shift = 14 - e;
        uint32_t hm = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (hm & 1u))) hm++;
        return (uint16_t)(sign | hm);
    }
    uint32_t h = ((uint32_t)e << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

__device__ __forceinline__ float half_bits_to_float(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

}  // namespace ovfq
