// kquant_blocks.h — per-super-block arithmetic of the Q4_K and Q6_K projections (shared by the decode GEMV
// and the small-batch kernel).
//
// A quad (4 lanes) owns one 256-element super-block. Each format defines:
//   W            the weight registers one lane holds for one block (loaded with 16-byte buffer loads)
//   A            the activation registers one lane holds for one block (its 64 Q8_K quants, bsums, scale)
//   load_w       global -> W
//   load_a       global Q8_K layout -> A
//   load_a_lds   LDS layout written by stage_q8k -> A
//   lds_pos(e)   where element e (a multiple of 4) of a block lives in the LDS layout (see below)
//   dot          the block's fp32 value exactly as the reference's Dot computes it (valid in all quad lanes)
//
// LDS activation layout: each block's 256 quants occupy a 320-byte slot (64 bytes of padding spread the 16
// quads of a wave over all LDS banks), split in sixteen 16-byte chunks; lane t's i-th chunk sits at chunk
// 4i + t, so for every i the four lanes of a quad read 64 contiguous bytes.
#pragma once

#include "ovfq_device.h"

namespace ovfq {

constexpr int kLdsSlot = 320;

// ------------------------------------------------------------------------------------------ Q4_K block
struct Q4K {
    static constexpr int kBytes = kQ4KBytes;
    struct W {
        u32x4 h, a, b;
    };
    struct A {
        u32x4 q[4];
        u32x2 bs;
        float s;
    };
    // lane t of the quad reads the header and nibble bytes [32t, 32t+32) of the block at byte `off`.
    __device__ __forceinline__ static W load_w(__amdgpu_buffer_rsrc_t r, uint32_t off, int t) {
        W w;
        w.h = ld4(r, off);
        w.a = ld4(r, off + 16 + 32 * t);
        w.b = ld4(r, off + 32 + 32 * t);
        return w;
    }
    // element e (multiple of 4) of a block -> byte offset in its LDS slot: lane t = e/64, chunk i = (e/16)%4.
    __device__ __forceinline__ static int lds_pos(int e) { return ((((e >> 4) & 3) << 2) + (e >> 6)) * 16 + (e & 15); }
    // activation of sub-blocks 2t and 2t+1 of super-block sb of activation row m.
    __device__ __forceinline__ static A load_a(__amdgpu_buffer_rsrc_t qr, __amdgpu_buffer_rsrc_t sr,
                                               __amdgpu_buffer_rsrc_t br, int in, int spr, int m, int sb, int t) {
        A a;
        const uint32_t qo = (uint32_t)m * in + sb * kQK + 64 * t;
#pragma unroll
        for (int i = 0; i < 4; i++) a.q[i] = ld4(qr, qo + 16 * i);
        a.bs = ld2(br, ((uint32_t)m * spr + sb) * 32 + 8 * t);
        a.s = __builtin_bit_cast(float, ld1(sr, ((uint32_t)m * spr + sb) * 4));
        return a;
    }
    __device__ __forceinline__ static A load_a_lds(const uint8_t* lq, const int16_t* lb, const float* ls, int sb, int t) {
        A a;
        const uint8_t* slot = lq + sb * kLdsSlot;
#pragma unroll
        for (int i = 0; i < 4; i++) a.q[i] = *reinterpret_cast<const u32x4*>(slot + (4 * i + t) * 16);
        a.bs = *reinterpret_cast<const u32x2*>(lb + sb * 16 + 4 * t);
        a.s = ls[sb];
        return a;
    }
    // Q4KDotKernel.Dot (RT/Q4KDotKernel.cs:216-256) for one block; valid in every lane of the quad.
    __device__ __forceinline__ static float dot(const W& w, const A& a, int t) {
        // UnpackQ4_KScalesMins (LD/GgmlDequant.cs:49-77) for sub-blocks j = 2t, 2t+1: bytes j&3 of the three
        // packed words, two bytes at a time.
        const uint32_t sh = (t & 1) * 16;
        const uint32_t A16 = (w.h.y >> sh) & 0xffffu, B16 = (w.h.z >> sh) & 0xffffu, C16 = (w.h.w >> sh) & 0xffffu;
        // sub-blocks 4..7 (t >= 2) or 0..3, chosen by a bit mask: a conditional here became a branch per lane group
        const uint32_t upper = 0u - ((uint32_t)t >> 1);
        const uint32_t sc01 = (((C16 & 0x0f0fu) | ((A16 >> 2) & 0x3030u)) & upper) | (A16 & 0x3f3fu & ~upper);
        const uint32_t m01 = ((((C16 >> 4) & 0x0f0fu) | ((B16 >> 2) & 0x3030u)) & upper) | (B16 & 0x3f3fu & ~upper);
        const uint32_t qw[8] = {w.a.x, w.a.y, w.a.z, w.a.w, w.b.x, w.b.y, w.b.z, w.b.w};
        const uint32_t aw[16] = {a.q[0].x, a.q[0].y, a.q[0].z, a.q[0].w, a.q[1].x, a.q[1].y, a.q[1].z, a.q[1].w,
                                 a.q[2].x, a.q[2].y, a.q[2].z, a.q[2].w, a.q[3].x, a.q[3].y, a.q[3].z, a.q[3].w};
        int dlo = 0, dhi = 0;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            dlo = sdot4(qw[k] & 0x0f0f0f0fu, aw[k], dlo);
            dhi = sdot4((qw[k] >> 4) & 0x0f0f0f0fu, aw[8 + k], dhi);
        }
        // |dlo|, |dhi| <= 32 * 15 * 127 and sc <= 63: full-rate 24-bit multiplies are exact
        int main_acc = __mul24((int)(sc01 & 0xffu), dlo) + __mul24((int)(sc01 >> 8), dhi);
        int min_acc = sdot2_k(a.bs.x, (int)(m01 & 0xffu), 0);
        min_acc = sdot2_k(a.bs.y, (int)(m01 >> 8), min_acc);
        main_acc = quad_sum(main_acc);
        min_acc = quad_sum(min_acc);
        const float d = half_lo(w.h.x), dmin = half_hi(w.h.x);
        // q8Scale * (d * mainAcc - dmin * minAcc)
        return a.s * (d * (float)main_acc - dmin * (float)min_acc);
    }
    // The same Dot split in two for several activation rows against one block: prep() unpacks the lane's scales,
    // mins and nibbles once; dot_p() is the per-row remainder (identical arithmetic to dot()).
    struct P {
        uint32_t lo[8], hi[8];
        uint32_t sc01, m01;
        uint32_t dd;  // fp16 d | fp16 dmin << 16
    };
    __device__ __forceinline__ static P prep(const W& w, int t) {
        P p;
        const uint32_t sh = (t & 1) * 16;
        const uint32_t A16 = (w.h.y >> sh) & 0xffffu, B16 = (w.h.z >> sh) & 0xffffu, C16 = (w.h.w >> sh) & 0xffffu;
        const uint32_t upper = 0u - ((uint32_t)t >> 1);  // as in dot()
        p.sc01 = (((C16 & 0x0f0fu) | ((A16 >> 2) & 0x3030u)) & upper) | (A16 & 0x3f3fu & ~upper);
        p.m01 = ((((C16 >> 4) & 0x0f0fu) | ((B16 >> 2) & 0x3030u)) & upper) | (B16 & 0x3f3fu & ~upper);
        const uint32_t qw[8] = {w.a.x, w.a.y, w.a.z, w.a.w, w.b.x, w.b.y, w.b.z, w.b.w};
#pragma unroll
        for (int k = 0; k < 8; k++) {
            p.lo[k] = qw[k] & 0x0f0f0f0fu;
            p.hi[k] = (qw[k] >> 4) & 0x0f0f0f0fu;
        }
        p.dd = w.h.x;
        return p;
    }
    __device__ __forceinline__ static float dot_p(const P& p, const A& a) {
        const uint32_t aw[16] = {a.q[0].x, a.q[0].y, a.q[0].z, a.q[0].w, a.q[1].x, a.q[1].y, a.q[1].z, a.q[1].w,
                                 a.q[2].x, a.q[2].y, a.q[2].z, a.q[2].w, a.q[3].x, a.q[3].y, a.q[3].z, a.q[3].w};
        int dlo = 0, dhi = 0;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            dlo = sdot4(p.lo[k], aw[k], dlo);
            dhi = sdot4(p.hi[k], aw[8 + k], dhi);
        }
        int main_acc = __mul24((int)(p.sc01 & 0xffu), dlo) + __mul24((int)(p.sc01 >> 8), dhi);
        int min_acc = sdot2_k(a.bs.x, (int)(p.m01 & 0xffu), 0);
        min_acc = sdot2_k(a.bs.y, (int)(p.m01 >> 8), min_acc);
        main_acc = quad_sum(main_acc);
        min_acc = quad_sum(min_acc);
        const float d = half_lo(p.dd), dmin = half_hi(p.dd);
        return a.s * (d * (float)main_acc - dmin * (float)min_acc);
    }
};

// ------------------------------------------------------------------------------------------ Q6_K block
struct Q6K {
    static constexpr int kBytes = kQ6KBytes;
    struct W {
        uint32_t a[4], b[4], h[4], s0, s1, d;
    };
    struct A {
        u32x4 q[4];
        u32x4 bs;
        float s;
    };
    // 210-byte blocks are only 2-byte aligned inside a row: every run is read as aligned dwords and shifted
    // into place with v_alignbyte_b32 (the resource base is 4-byte aligned, so `off & 3` is the misalignment).
    __device__ __forceinline__ static void run16(__amdgpu_buffer_rsrc_t r, uint32_t o, uint32_t out[4]) {
        const uint32_t o4 = o & ~3u, sh = o & 3u;
        const u32x4 v = ld4(r, o4);
        const uint32_t v4 = ld1(r, o4 + 16);
        out[0] = __builtin_amdgcn_alignbyte(v.y, v.x, sh);
        out[1] = __builtin_amdgcn_alignbyte(v.z, v.y, sh);
        out[2] = __builtin_amdgcn_alignbyte(v.w, v.z, sh);
        out[3] = __builtin_amdgcn_alignbyte(v4, v.w, sh);
    }
    // lane t = (half h = t >> 1, l-range lh = t & 1): ql[64h+16lh..+16), ql[64h+32+16lh..+16), qh[32h+16lh..+16),
    // scales sc[8h..8h+8) and d.
    __device__ __forceinline__ static W load_w(__amdgpu_buffer_rsrc_t r, uint32_t off, int t) {
        W w;
        const int h = t >> 1, lh = t & 1;
        run16(r, off + 64 * h + 16 * lh, w.a);
        run16(r, off + 64 * h + 32 + 16 * lh, w.b);
        run16(r, off + 128 + 32 * h + 16 * lh, w.h);
        const uint32_t so = off + 192 + 8 * h, sh = so & 3u;
        const u32x3 sv = ld3(r, so & ~3u);
        w.s0 = __builtin_amdgcn_alignbyte(sv.y, sv.x, sh);
        w.s1 = __builtin_amdgcn_alignbyte(sv.z, sv.y, sh);
        // d (bytes 208-209) with a 16-bit load: a dword read would run past the last block of the matrix.
        w.d = __builtin_amdgcn_raw_buffer_load_b16(r, (int)(off + 208), 0, 0);
        return w;
    }
    // element e (multiple of 4) -> LDS slot offset: half h = e/128, run i = (e/32)%4, l-range lh = (e/16)%2,
    // lane t = 2h + lh.
    __device__ __forceinline__ static int lds_pos(int e) {
        return ((((e >> 5) & 3) << 2) + ((e >> 7) << 1) + ((e >> 4) & 1)) * 16 + (e & 15);
    }
    __device__ __forceinline__ static A load_a(__amdgpu_buffer_rsrc_t qr, __amdgpu_buffer_rsrc_t sr,
                                               __amdgpu_buffer_rsrc_t br, int in, int spr, int m, int sb, int t) {
        A a;
        const int h = t >> 1, lh = t & 1;
        const uint32_t qo = (uint32_t)m * in + sb * kQK + 128 * h + 16 * lh;
#pragma unroll
        for (int i = 0; i < 4; i++) a.q[i] = ld4(qr, qo + 32 * i);
        a.bs = ld4(br, ((uint32_t)m * spr + sb) * 32 + 16 * h);
        a.s = __builtin_bit_cast(float, ld1(sr, ((uint32_t)m * spr + sb) * 4));
        return a;
    }
    __device__ __forceinline__ static A load_a_lds(const uint8_t* lq, const int16_t* lb, const float* ls, int sb, int t) {
        A a;
        const uint8_t* slot = lq + sb * kLdsSlot;
#pragma unroll
        for (int i = 0; i < 4; i++) a.q[i] = *reinterpret_cast<const u32x4*>(slot + (4 * i + t) * 16);
        a.bs = *reinterpret_cast<const u32x4*>(lb + sb * 16 + 8 * (t >> 1));
        a.s = ls[sb];
        return a;
    }
    // Q6KDotKernel.Dot (RT/Q6KDotKernel.cs:77-116). Lane t covers sub-blocks 8h+lh+2i (i = 0..3), i.e. the
    // 16-element runs q1..q4 of DecodeQ6_KBlock at l in [16lh, 16lh+16).
    __device__ __forceinline__ static float dot(const W& w, const A& a, int t) {
        const int lh = t & 1;
        const uint32_t m4 = 0x0f0f0f0fu, m3 = 0x30303030u;
        const uint32_t aw[16] = {a.q[0].x, a.q[0].y, a.q[0].z, a.q[0].w, a.q[1].x, a.q[1].y, a.q[1].z, a.q[1].w,
                                 a.q[2].x, a.q[2].y, a.q[2].z, a.q[2].w, a.q[3].x, a.q[3].y, a.q[3].z, a.q[3].w};
        int d1 = 0, d2 = 0, d3 = 0, d4 = 0;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t q1 = (w.a[k] & m4) | ((w.h[k] << 4) & m3);
            const uint32_t q2 = (w.b[k] & m4) | ((w.h[k] << 2) & m3);
            const uint32_t q3 = ((w.a[k] >> 4) & m4) | (w.h[k] & m3);
            const uint32_t q4 = ((w.b[k] >> 4) & m4) | ((w.h[k] >> 2) & m3);
            d1 = sdot4(q1, aw[k], d1);
            d2 = sdot4(q2, aw[4 + k], d2);
            d3 = sdot4(q3, aw[8 + k], d3);
            d4 = sdot4(q4, aw[12 + k], d4);
        }
        const uint32_t bo = 8 * lh;
        const int s1 = __builtin_amdgcn_sbfe((int)w.s0, bo, 8);
        const int s2 = __builtin_amdgcn_sbfe((int)w.s0, bo + 16, 8);
        const int s3 = __builtin_amdgcn_sbfe((int)w.s1, bo, 8);
        const int s4 = __builtin_amdgcn_sbfe((int)w.s1, bo + 16, 8);
        const uint32_t hs = 16 * lh;
        const int b1 = __builtin_amdgcn_sbfe((int)a.bs.x, hs, 16);
        const int b2 = __builtin_amdgcn_sbfe((int)a.bs.y, hs, 16);
        const int b3 = __builtin_amdgcn_sbfe((int)a.bs.z, hs, 16);
        const int b4 = __builtin_amdgcn_sbfe((int)a.bs.w, hs, 16);
        // unsignedDot - 32 * bsumTerm, exact in int32 (|.| < 2^28). Each factor fits 24 bits (|s| <= 128; |d - 32 b|
        // <= 16 * 63 * 127 + 32 * 2032 < 2^18), so the products are full-rate 24-bit multiplies.
        int part = __mul24(s1, d1 - 32 * b1) + __mul24(s2, d2 - 32 * b2) + __mul24(s3, d3 - 32 * b3) +
                   __mul24(s4, d4 - 32 * b4);
        part = quad_sum(part);
        const float d = half_lo(w.d);
        // d * q8Scale * mainAcc
        return d * a.s * (float)part;
    }
    // prep() / dot_p(): dot() split for several activation rows against one block (see Q4K).
    struct P {
        uint32_t q[4][4];  // q1..q4 runs, 6-bit values
        int s[4];
        uint32_t d;
        int lh;
    };
    __device__ __forceinline__ static P prep(const W& w, int t) {
        P p;
        const uint32_t m4 = 0x0f0f0f0fu, m3 = 0x30303030u;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            p.q[0][k] = (w.a[k] & m4) | ((w.h[k] << 4) & m3);
            p.q[1][k] = (w.b[k] & m4) | ((w.h[k] << 2) & m3);
            p.q[2][k] = ((w.a[k] >> 4) & m4) | (w.h[k] & m3);
            p.q[3][k] = ((w.b[k] >> 4) & m4) | ((w.h[k] >> 2) & m3);
        }
        p.lh = t & 1;
        const uint32_t bo = 8 * p.lh;
        p.s[0] = __builtin_amdgcn_sbfe((int)w.s0, bo, 8);
        p.s[1] = __builtin_amdgcn_sbfe((int)w.s0, bo + 16, 8);
        p.s[2] = __builtin_amdgcn_sbfe((int)w.s1, bo, 8);
        p.s[3] = __builtin_amdgcn_sbfe((int)w.s1, bo + 16, 8);
        p.d = w.d;
        return p;
    }
    __device__ __forceinline__ static float dot_p(const P& p, const A& a) {
        const uint32_t aw[16] = {a.q[0].x, a.q[0].y, a.q[0].z, a.q[0].w, a.q[1].x, a.q[1].y, a.q[1].z, a.q[1].w,
                                 a.q[2].x, a.q[2].y, a.q[2].z, a.q[2].w, a.q[3].x, a.q[3].y, a.q[3].z, a.q[3].w};
        int d1 = 0, d2 = 0, d3 = 0, d4 = 0;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            d1 = sdot4(p.q[0][k], aw[k], d1);
            d2 = sdot4(p.q[1][k], aw[4 + k], d2);
            d3 = sdot4(p.q[2][k], aw[8 + k], d3);
            d4 = sdot4(p.q[3][k], aw[12 + k], d4);
        }
        const uint32_t hs = 16 * p.lh;
        const int b1 = __builtin_amdgcn_sbfe((int)a.bs.x, hs, 16);
        const int b2 = __builtin_amdgcn_sbfe((int)a.bs.y, hs, 16);
        const int b3 = __builtin_amdgcn_sbfe((int)a.bs.z, hs, 16);
        const int b4 = __builtin_amdgcn_sbfe((int)a.bs.w, hs, 16);
        int part = __mul24(p.s[0], d1 - 32 * b1) + __mul24(p.s[1], d2 - 32 * b2) + __mul24(p.s[2], d3 - 32 * b3) +
                   __mul24(p.s[3], d4 - 32 * b4);
        part = quad_sum(part);
        const float d = half_lo(p.d);
        return d * a.s * (float)part;
    }
};

}  // namespace ovfq
