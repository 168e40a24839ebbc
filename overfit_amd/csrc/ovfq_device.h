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

// Q8DotKernel.Quantize (RT/Q8DotKernel.cs:42-91) for one 32-element block held by 8 consecutive lanes (lane & 7 =
// sub holds elements 4 sub .. 4 sub + 3 in `raw`): absmax over the 8 lanes, scale = absmax / 127, quants
// round-half-even(v / scale) clamped to [-127, 127] (0 for an all-zero block), packed in element order. Every lane
// of the wave must take part (the absmax uses cross-lane swaps).
struct Q80Lane {
    uint32_t packed;
    float scale;
};
__device__ __forceinline__ Q80Lane q8_0_quantize_lane(u32x4 raw) {
    const float v0 = as_float(raw.x), v1 = as_float(raw.y);
    const float v2 = as_float(raw.z), v3 = as_float(raw.w);
    float am = fmaxf(fmaxf(fabsf(v0), fabsf(v1)), fmaxf(fabsf(v2), fabsf(v3)));
    am = fmaxf(am, __shfl_xor(am, 1, 64));
    am = fmaxf(am, __shfl_xor(am, 2, 64));
    am = fmaxf(am, __shfl_xor(am, 4, 64));
    const float scale = am / 127.0f;
    const float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
    const int q0 = (int)fminf(fmaxf(rintf(v0 * inv), -127.0f), 127.0f);
    const int q1 = (int)fminf(fmaxf(rintf(v1 * inv), -127.0f), 127.0f);
    const int q2 = (int)fminf(fmaxf(rintf(v2 * inv), -127.0f), 127.0f);
    const int q3 = (int)fminf(fmaxf(rintf(v3 * inv), -127.0f), 127.0f);
    return Q80Lane{(uint32_t)(q0 & 0xff) | ((uint32_t)(q1 & 0xff) << 8) | ((uint32_t)(q2 & 0xff) << 16) |
                       ((uint32_t)(q3 & 0xff) << 24),
                   scale};
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

// Q4KDotKernel.QuantizeActivationQ8K (RT/Q4KDotKernel.cs:71-136) for one 256-element super-block held by a
// whole wave, four consecutive elements per lane: absMax is a max (exact in any order); scale = absMax / 127f;
// inverse = scale > 0 ? 1f / scale : 0f; q = clamp(rint(x * inverse), -127, 127). Returns the four quants
// packed in a dword (element 4*lane in the low byte), the sum of the 16-element group (every lane of the quad
// holds it) and the block scale.
struct Q8KLane {
    uint32_t packed;
    int group_sum;
    float scale;
};

__device__ __forceinline__ Q8KLane q8k_quantize_wave(float v0, float v1, float v2, float v3) {
    float am = fmaxf(fmaxf(fabsf(v0), fabsf(v1)), fmaxf(fabsf(v2), fabsf(v3)));
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) am = fmaxf(am, __shfl_xor(am, off, 64));
    const float scale = am / 127.0f;
    const float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
    const int q0 = (int)fminf(fmaxf(rintf(v0 * inv), -127.0f), 127.0f);
    const int q1 = (int)fminf(fmaxf(rintf(v1 * inv), -127.0f), 127.0f);
    const int q2 = (int)fminf(fmaxf(rintf(v2 * inv), -127.0f), 127.0f);
    const int q3 = (int)fminf(fmaxf(rintf(v3 * inv), -127.0f), 127.0f);
    Q8KLane r;
    r.packed = (uint32_t)(q0 & 0xff) | ((uint32_t)(q1 & 0xff) << 8) | ((uint32_t)(q2 & 0xff) << 16) |
               ((uint32_t)(q3 & 0xff) << 24);
    r.group_sum = quad_sum(q0 + q1 + q2 + q3);
    r.scale = scale;
    return r;
}

// Q8_K block `blk` of x (256 floats) quantised by one wave: quants, bsums and scale written to q, bs, s.
__device__ __forceinline__ void q8k_quantize_block(const float* __restrict__ x, int64_t blk, int8_t* __restrict__ q,
                                                   float* __restrict__ s, int16_t* __restrict__ bs) {
    const int lane = threadIdx.x & 63;
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(x + blk * kQK, kQK * 4);
    const u32x4 raw = ld4(xr, lane * 16);
    const Q8KLane r = q8k_quantize_wave(as_float(raw.x), as_float(raw.y), as_float(raw.z), as_float(raw.w));
    reinterpret_cast<uint32_t*>(q + blk * kQK)[lane] = r.packed;
    if ((lane & 3) == 0) bs[blk * 16 + (lane >> 2)] = (int16_t)r.group_sum;
    if (lane == 0) s[blk] = r.scale;
}

// Max over the 16 lanes of a DPP row; every lane of the row receives it. Used on the bit patterns of
// non-negative floats, whose unsigned integer order is their numeric order.
__device__ __forceinline__ uint32_t row16_max_u32(uint32_t v) {
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xb1, 0xf, 0xf, false));   // quad_perm [1,0,3,2]
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4e, 0xf, 0xf, false));   // quad_perm [2,3,0,1]
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xf, 0xf, false));  // row_half_mirror
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xf, 0xf, false));  // row_mirror
    return v;
}

// The same Q8_K quantisation with one super-block spread over a 16-lane row, sixteen consecutive elements per
// lane (the lane's elements are exactly one bsum group). x holds the lane's 16 values; returns the 16 quants
// in four dwords, the group sum and the block scale.
struct Q8KRow {
    u32x4 packed;
    int group_sum;
    float scale;
};

__device__ __forceinline__ Q8KRow q8k_quantize_row16(const float (&x)[16]) {
    uint32_t am = 0;
#pragma unroll
    for (int i = 0; i < 16; i++) am = max(am, __builtin_bit_cast(uint32_t, fabsf(x[i])));
    const float absmax = __builtin_bit_cast(float, row16_max_u32(am));
    const float scale = absmax / 127.0f;
    const float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
    Q8KRow r;
    int sum = 0;
    uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int qv = (int)fminf(fmaxf(rintf(x[i] * inv), -127.0f), 127.0f);
        sum += qv;
        w[i >> 2] |= (uint32_t)(qv & 0xff) << (8 * (i & 3));
    }
    r.packed = u32x4{w[0], w[1], w[2], w[3]};
    r.group_sum = sum;
    r.scale = scale;
    return r;
}

}  // namespace ovfq
