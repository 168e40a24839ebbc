/*
 * ovfq_oracle.c — CPU restatement of Overfit's GGUF quantized-linear arithmetic (test infrastructure only;
 * see ovfq_oracle.h). Build with -O2 -ffp-contract=off -fno-fast-math: each float expression below is one
 * IEEE binary32 operation per C# operator, evaluated left to right as the reference's C# does.
 */
#include "ovfq_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- fp16 */

/* (float)BitConverter.UInt16BitsToHalf(bits): exact widening (RT/Q4KDotKernel.cs:235-238). */
float orc_half_to_float(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t exp = ((uint32_t)h >> 10) & 0x1fu;
    uint32_t mant = (uint32_t)h & 0x3ffu;
    uint32_t bits;
    if (exp == 0) {
        if (mant == 0) {
            bits = sign;
        } else {
            int e = -14;
            while ((mant & 0x400u) == 0) {
                mant <<= 1;
                e--;
            }
            mant &= 0x3ffu;
            bits = sign | ((uint32_t)(e + 127) << 23) | (mant << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (mant << 13);
    } else {
        bits = sign | ((exp - 15u + 127u) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* (Half)f: round to nearest, ties to even; overflow to infinity (LD/GgmlQuant.cs:105-106). */
uint16_t orc_float_to_half(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xffu;
    uint32_t mant = x & 0x7fffffu;
    if (exp == 0xffu) {
        if (mant != 0) {
            return (uint16_t)(sign | 0x7e00u | (mant >> 13));
        }
        return (uint16_t)(sign | 0x7c00u);
    }
    int e = (int)exp - 112; /* exp - 127 + 15 */
    if (e >= 31) {
        return (uint16_t)(sign | 0x7c00u);
    }
    if (e <= 0) {
        if (e < -10) {
            return (uint16_t)sign;
        }
        uint32_t m = mant | 0x800000u;
        int shift = 14 - e;
        uint32_t hm = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (hm & 1u))) {
            hm++;
        }
        return (uint16_t)(sign | hm);
    }
    uint32_t h = ((uint32_t)e << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) {
        h++;
    }
    return (uint16_t)(sign | h);
}

static inline uint16_t rd_u16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline void wr_u16(uint8_t* p, uint16_t v) {
    p[0] = (uint8_t)(v & 0xff);
    p[1] = (uint8_t)(v >> 8);
}

/* ---------------------------------------------------------------- a1 / a18 packing */

void orc_unpack_q4k_scales_mins(const uint8_t* q, uint8_t* sc, uint8_t* m) {
    /* LD/GgmlDequant.cs:67-76 */
    for (int j = 0; j < 4; j++) {
        sc[j] = (uint8_t)(q[j] & 0x3f);
        m[j] = (uint8_t)(q[j + 4] & 0x3f);
    }
    for (int j = 4; j < 8; j++) {
        sc[j] = (uint8_t)((q[j + 4] & 0x0f) | ((q[j - 4] >> 6) << 4));
        m[j] = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

void orc_pack_q4k_scales_mins(const uint8_t* sc, const uint8_t* m, uint8_t* p) {
    /* LD/GgmlQuant.cs:164-172 */
    for (int j = 0; j < 4; j++) {
        p[j] = (uint8_t)((sc[j] & 0x3f) | ((sc[j + 4] >> 4) << 6));
        p[j + 4] = (uint8_t)((m[j] & 0x3f) | ((m[j + 4] >> 4) << 6));
        p[j + 8] = (uint8_t)((sc[j + 4] & 0x0f) | ((m[j + 4] & 0x0f) << 4));
    }
}

/* ---------------------------------------------------------------- a19 decode */

void orc_decode_q4k_block(const uint8_t* b, float* dst) {
    /* LD/GgmlDequant.cs:95-141 */
    float d = orc_half_to_float(rd_u16(b));
    float dmin = orc_half_to_float(rd_u16(b + 2));
    uint8_t sc[8], m[8];
    orc_unpack_q4k_scales_mins(b + 4, sc, m);
    const uint8_t* qs = b + 16;
    for (int p = 0; p < 4; p++) {
        float scale1 = d * (float)sc[2 * p];
        float min1 = dmin * (float)m[2 * p];
        float scale2 = d * (float)sc[2 * p + 1];
        float min2 = dmin * (float)m[2 * p + 1];
        for (int i = 0; i < 32; i++) {
            dst[64 * p + i] = scale1 * (float)(qs[32 * p + i] & 0x0f) - min1;
        }
        for (int i = 0; i < 32; i++) {
            dst[64 * p + 32 + i] = scale2 * (float)(qs[32 * p + i] >> 4) - min2;
        }
    }
}

void orc_decode_q5_0_block(const uint8_t* b, float* dst) {
    /* LD/GgmlDequant.cs:222-248: d fp16 @0, qh u32 LE @2 (the 5th bit of each quant), qs @6; element j takes the low
     * nibble of qs[j] and qh bit j, element j + 16 the high nibble and bit j + 16; dst = (q - 16) * d. */
    float d = orc_half_to_float(rd_u16(b));
    uint32_t qh = (uint32_t)b[2] | ((uint32_t)b[3] << 8) | ((uint32_t)b[4] << 16) | ((uint32_t)b[5] << 24);
    const uint8_t* qs = b + 6;
    for (int j = 0; j < 16; j++) {
        int xh0 = (int)((qh >> j) << 4) & 0x10;
        int xh1 = (int)(qh >> (j + 12)) & 0x10;
        int x0 = ((qs[j] & 0x0f) | xh0) - 16;
        int x1 = ((qs[j] >> 4) | xh1) - 16;
        dst[j] = (float)x0 * d;
        dst[j + 16] = (float)x1 * d;
    }
}

void orc_decode_q5k_block(const uint8_t* b, float* dst) {
    /* LD/GgmlDequant.cs:262-320: the Q4_K layout (d, dmin, 12 packed scale/min bytes) with 32 bytes of 5th bits
     * (qh @16) before the 128 nibble bytes (qs @48); group g's low nibbles take qh bit 2g, its high nibbles bit
     * 2g + 1. */
    float d = orc_half_to_float(rd_u16(b));
    float dmin = orc_half_to_float(rd_u16(b + 2));
    uint8_t sc[8], m[8];
    orc_unpack_q4k_scales_mins(b + 4, sc, m);
    const uint8_t* qh = b + 16;
    const uint8_t* qs = b + 48;
    for (int g = 0; g < 4; g++) {
        float scale1 = d * (float)sc[2 * g];
        float min1 = dmin * (float)m[2 * g];
        float scale2 = d * (float)sc[2 * g + 1];
        float min2 = dmin * (float)m[2 * g + 1];
        int u1 = 1 << (2 * g), u2 = 2 << (2 * g);
        for (int l = 0; l < 32; l++) {
            int hi = (qh[l] & u1) ? 16 : 0;
            dst[64 * g + l] = scale1 * (float)((qs[32 * g + l] & 0x0f) + hi) - min1;
        }
        for (int l = 0; l < 32; l++) {
            int hi = (qh[l] & u2) ? 16 : 0;
            dst[64 * g + 32 + l] = scale2 * (float)((qs[32 * g + l] >> 4) + hi) - min2;
        }
    }
}

void orc_decode_q6k_block(const uint8_t* b, float* dst) {
    /* LD/GgmlDequant.cs:143-209 */
    const uint8_t* ql = b;
    const uint8_t* qh = b + 128;
    const uint8_t* sc = b + 192;
    float d = orc_half_to_float(rd_u16(b + 208));
    for (int h = 0; h < 2; h++) {
        int qlb = 64 * h, qhb = 32 * h, scb = 8 * h, db = 128 * h;
        for (int l = 0; l < 32; l++) {
            int qhbyte = qh[qhb + l];
            int is = l / 16;
            int q1 = (ql[qlb + l] & 0x0f) | (((qhbyte >> 0) & 3) << 4);
            int q2 = (ql[qlb + l + 32] & 0x0f) | (((qhbyte >> 2) & 3) << 4);
            int q3 = (ql[qlb + l] >> 4) | (((qhbyte >> 4) & 3) << 4);
            int q4 = (ql[qlb + l + 32] >> 4) | (((qhbyte >> 6) & 3) << 4);
            int s1 = (int8_t)sc[scb + is + 0];
            int s2 = (int8_t)sc[scb + is + 2];
            int s3 = (int8_t)sc[scb + is + 4];
            int s4 = (int8_t)sc[scb + is + 6];
            /* d * s1 * (q1 - 32) == (d * (float)s1) * (float)(q1 - 32) */
            dst[db + l] = d * (float)s1 * (float)(q1 - 32);
            dst[db + l + 32] = d * (float)s2 * (float)(q2 - 32);
            dst[db + l + 64] = d * (float)s3 * (float)(q3 - 32);
            dst[db + l + 96] = d * (float)s4 * (float)(q4 - 32);
        }
    }
}

int orc_q4k_decode_row(const uint8_t* blocks, int in, int out, int row, float* dst) {
    /* RT/Q4KWeight.cs:121-138 */
    if (!blocks || !dst) return ORC_ERR_NULL;
    if (row < 0 || row >= out) return ORC_ERR_RANGE;
    if (in <= 0 || in % ORC_QK) return ORC_ERR_SIZE;
    int spr = in / ORC_QK;
    for (int sb = 0; sb < spr; sb++) {
        orc_decode_q4k_block(blocks + ((size_t)row * spr + sb) * ORC_Q4K_BYTES, dst + sb * ORC_QK);
    }
    return ORC_OK;
}

int orc_q6k_decode_row(const uint8_t* blocks, int in, int out, int row, float* dst) {
    /* RT/Q6KWeight.cs DecodeRow (same shape as RT/Q4KWeight.cs:121-138) */
    if (!blocks || !dst) return ORC_ERR_NULL;
    if (row < 0 || row >= out) return ORC_ERR_RANGE;
    if (in <= 0 || in % ORC_QK) return ORC_ERR_SIZE;
    int spr = in / ORC_QK;
    for (int sb = 0; sb < spr; sb++) {
        orc_decode_q6k_block(blocks + ((size_t)row * spr + sb) * ORC_Q6K_BYTES, dst + sb * ORC_QK);
    }
    return ORC_OK;
}

int orc_q8_decode_row(const int8_t* quants, const float* scales, int in, int out, int row, float* dst) {
    /* RT/Q8Weight.cs:81-106: dst[i] = scale * quant[i] */
    if (!quants || !scales || !dst) return ORC_ERR_NULL;
    if (row < 0 || row >= out) return ORC_ERR_RANGE;
    if (in <= 0 || in % ORC_Q8_BLOCK) return ORC_ERR_SIZE;
    int bpr = in / ORC_Q8_BLOCK;
    for (int b = 0; b < bpr; b++) {
        float s = scales[(size_t)row * bpr + b];
        for (int i = 0; i < ORC_Q8_BLOCK; i++) {
            dst[b * ORC_Q8_BLOCK + i] = s * (float)quants[(size_t)row * in + b * ORC_Q8_BLOCK + i];
        }
    }
    return ORC_OK;
}

/* ---------------------------------------------------------------- a3 / a11 activation quantize */

static inline float clampf(float v, float lo, float hi) { return v < lo ? lo : (v > hi ? hi : v); }

int orc_quantize_q8k(const float* src, int n, int8_t* quants, float* scales, int16_t* bsums) {
    /* RT/Q4KDotKernel.cs:71-136 (scalar path; the AVX2 path :148-209 is bit-identical for finite input) */
    if (!src || !quants || !scales || !bsums) return ORC_ERR_NULL;
    if (n < 0 || n % ORC_QK) return ORC_ERR_SIZE;
    int blocks = n / ORC_QK;
    for (int b = 0; b < blocks; b++) {
        const float* blk = src + (size_t)b * ORC_QK;
        float absmax = 0.0f;
        for (int i = 0; i < ORC_QK; i++) {
            float a = fabsf(blk[i]);
            if (a > absmax) absmax = a;
        }
        float scale = absmax / 127.0f;
        scales[b] = scale;
        float inverse = scale > 0.0f ? 1.0f / scale : 0.0f;
        for (int g = 0; g < ORC_QK / ORC_GROUP; g++) {
            int sum = 0;
            for (int k = 0; k < ORC_GROUP; k++) {
                int idx = g * ORC_GROUP + k;
                int q = (int)clampf(rintf(blk[idx] * inverse), -127.0f, 127.0f);
                quants[(size_t)b * ORC_QK + idx] = (int8_t)q;
                sum += q;
            }
            bsums[(size_t)b * (ORC_QK / ORC_GROUP) + g] = (int16_t)sum;
        }
    }
    return ORC_OK;
}

int orc_quantize_q8_0(const float* src, int n, int8_t* quants, float* scales) {
    /* RT/Q8DotKernel.cs:42-91 */
    if (!src || !quants || !scales) return ORC_ERR_NULL;
    if (n < 0 || n % ORC_Q8_BLOCK) return ORC_ERR_SIZE;
    int blocks = n / ORC_Q8_BLOCK;
    for (int blk = 0; blk < blocks; blk++) {
        const float* s = src + (size_t)blk * ORC_Q8_BLOCK;
        float absmax = 0.0f;
        for (int i = 0; i < ORC_Q8_BLOCK; i++) {
            float a = fabsf(s[i]);
            if (a > absmax) absmax = a;
        }
        float scale = absmax / 127.0f;
        scales[blk] = scale;
        float inverse = scale > 0.0f ? 1.0f / scale : 0.0f;
        for (int i = 0; i < ORC_Q8_BLOCK; i++) {
            float q = clampf(rintf(s[i] * inverse), -127.0f, 127.0f);
            quants[(size_t)blk * ORC_Q8_BLOCK + i] = (int8_t)(int)q;
        }
    }
    return ORC_OK;
}

/* ---------------------------------------------------------------- a4 / a5 / a9 / a12 dots */

int32_t orc_q4k_main_dot(const uint8_t* qs, const int8_t* q8, const uint8_t* scales) {
    /* RT/Q4KDotKernel.cs:366-387 */
    int32_t sum = 0;
    for (int s = 0; s < 8; s++) {
        int qsb = 32 * (s >> 1);
        int high = (s & 1) == 1;
        int q8b = 32 * s;
        int32_t dot = 0;
        for (int e = 0; e < 32; e++) {
            int packed = qs[qsb + e];
            int nib = high ? (packed >> 4) : (packed & 0x0f);
            dot += nib * q8[q8b + e];
        }
        sum += scales[s] * dot;
    }
    return sum;
}

int32_t orc_q4k_min_acc(const uint8_t* mins, const int16_t* bsums) {
    /* RT/Q4KDotKernel.cs:249-253 */
    int32_t acc = 0;
    for (int s = 0; s < 8; s++) {
        acc += mins[s] * (bsums[2 * s] + bsums[2 * s + 1]);
    }
    return acc;
}

float orc_q4k_dot(const uint8_t* b, const int8_t* q8, float q8s, const int16_t* bsums) {
    /* RT/Q4KDotKernel.cs:216-256 */
    float d = orc_half_to_float(rd_u16(b));
    float dmin = orc_half_to_float(rd_u16(b + 2));
    uint8_t sc[8], m[8];
    orc_unpack_q4k_scales_mins(b + 4, sc, m);
    int32_t main_acc = orc_q4k_main_dot(b + 16, q8, sc);
    int32_t min_acc = orc_q4k_min_acc(m, bsums);
    /* q8Scale * (d * mainAcc - dmin * minAcc) */
    return q8s * (d * (float)main_acc - dmin * (float)min_acc);
}

int32_t orc_q6k_unsigned_dot(const uint8_t* b, const int8_t* q8) {
    /* RT/Q6KDotKernel.cs:186-216 (scalar fallback; same INT32 sum as the AVX2 path) */
    const uint8_t* ql = b;
    const uint8_t* qh = b + 128;
    const uint8_t* sc = b + 192;
    int32_t sum = 0;
    for (int h = 0; h < 2; h++) {
        int qlb = 64 * h, qhb = 32 * h, scb = 8 * h, q8b = 128 * h;
        for (int l = 0; l < 32; l++) {
            int qhbyte = qh[qhb + l];
            int off = l >> 4;
            int q1 = (ql[qlb + l] & 0x0f) | (((qhbyte >> 0) & 3) << 4);
            int q2 = (ql[qlb + l + 32] & 0x0f) | (((qhbyte >> 2) & 3) << 4);
            int q3 = (ql[qlb + l] >> 4) | (((qhbyte >> 4) & 3) << 4);
            int q4 = (ql[qlb + l + 32] >> 4) | (((qhbyte >> 6) & 3) << 4);
            int s1 = (int8_t)sc[scb + off];
            int s2 = (int8_t)sc[scb + off + 2];
            int s3 = (int8_t)sc[scb + off + 4];
            int s4 = (int8_t)sc[scb + off + 6];
            sum += s1 * q1 * q8[q8b + l] + s2 * q2 * q8[q8b + l + 32] + s3 * q3 * q8[q8b + l + 64] +
                   s4 * q4 * q8[q8b + l + 96];
        }
    }
    return sum;
}

int32_t orc_q6k_bsum_term(const uint8_t* b, const int16_t* bsums) {
    /* RT/Q6KDotKernel.cs:108-113 */
    const uint8_t* sc = b + 192;
    int32_t t = 0;
    for (int s = 0; s < 16; s++) {
        t += (int8_t)sc[s] * bsums[s];
    }
    return t;
}

float orc_q6k_dot(const uint8_t* b, const int8_t* q8, float q8s, const int16_t* bsums) {
    /* RT/Q6KDotKernel.cs:77-116: return d * q8Scale * mainAcc == (d * q8Scale) * (float)mainAcc */
    float d = orc_half_to_float(rd_u16(b + 208));
    int32_t u = orc_q6k_unsigned_dot(b, q8);
    int32_t bt = orc_q6k_bsum_term(b, bsums);
    int32_t main_acc = u - 32 * bt;
    return d * q8s * (float)main_acc;
}

int32_t orc_q8_block_int_dot(const int8_t* a, const int8_t* b) {
    /* RT/Q8DotKernel.cs:469-487 */
    int32_t s = 0;
    for (int i = 0; i < ORC_Q8_BLOCK; i++) s += a[i] * b[i];
    return s;
}

float orc_q8_dot(const int8_t* aq, const float* as, const int8_t* bq, const float* bs, int length) {
    /* RT/Q8DotKernel.cs:99-140: result += aScales[b] * bScales[b] * blockDot */
    int blocks = length / ORC_Q8_BLOCK;
    float result = 0.0f;
    for (int blk = 0; blk < blocks; blk++) {
        int32_t dot = orc_q8_block_int_dot(aq + blk * ORC_Q8_BLOCK, bq + blk * ORC_Q8_BLOCK);
        result += as[blk] * bs[blk] * (float)dot;
    }
    return result;
}

/* ---------------------------------------------------------------- a6 / a7 / a8 Q4_K projections */

static int check_q4k_dims(int in, int out) {
    if (in <= 0 || out <= 0) return ORC_ERR_RANGE;
    if (in % ORC_QK) return ORC_ERR_SIZE;
    return ORC_OK;
}

static float q4k_row_sum(const uint8_t* row, int spr, const int8_t* q, const float* s, const int16_t* b) {
    /* RT/Q4KDotKernel.cs:460-473: sum += Dot(...) over super-blocks ascending */
    float sum = 0.0f;
    for (int sb = 0; sb < spr; sb++) {
        sum += orc_q4k_dot(row + (size_t)sb * ORC_Q4K_BYTES, q + sb * ORC_QK, s[sb], b + sb * 16);
    }
    return sum;
}

int orc_q4k_project_prequantized(const uint8_t* blocks, int in, int out, const float* bias, float* output,
                                 const int8_t* q, const float* s, const int16_t* b) {
    /* RT/Q4KDotKernel.cs:445-476 */
    if (!blocks || !output || !q || !s || !b) return ORC_ERR_NULL;
    int rc = check_q4k_dims(in, out);
    if (rc) return rc;
    int spr = in / ORC_QK;
    for (int o = 0; o < out; o++) {
        float sum = q4k_row_sum(blocks + (size_t)o * spr * ORC_Q4K_BYTES, spr, q, s, b);
        output[o] = bias == NULL ? sum : bias[o] + sum;
    }
    return ORC_OK;
}

int orc_q4k_project(const float* input, const uint8_t* blocks, int in, int out, const float* bias,
                    float* output, int8_t* q, float* s, int16_t* b) {
    /* RT/Q4KDotKernel.cs:414-435 */
    if (!input) return ORC_ERR_NULL;
    int rc = check_q4k_dims(in, out);
    if (rc) return rc;
    rc = orc_quantize_q8k(input, in, q, s, b);
    if (rc) return rc;
    return orc_q4k_project_prequantized(blocks, in, out, bias, output, q, s, b);
}

int orc_q4k_project_gate_up(const float* input, const uint8_t* gate, const uint8_t* up, int in, int out_dim,
                            float* gate_out, float* up_out, int8_t* q, float* s, int16_t* b) {
    /* RT/Q4KDotKernel.cs:563-645: one quantize; rows [0,outDim) gate, [outDim, 2outDim) up; no bias */
    if (!input || !gate || !up || !gate_out || !up_out) return ORC_ERR_NULL;
    int rc = check_q4k_dims(in, out_dim);
    if (rc) return rc;
    rc = orc_quantize_q8k(input, in, q, s, b);
    if (rc) return rc;
    int spr = in / ORC_QK;
    for (int g = 0; g < 2 * out_dim; g++) {
        int is_up = g >= out_dim;
        int row = is_up ? g - out_dim : g;
        const uint8_t* w = is_up ? up : gate;
        float sum = q4k_row_sum(w + (size_t)row * spr * ORC_Q4K_BYTES, spr, q, s, b);
        if (is_up) up_out[row] = sum;
        else gate_out[row] = sum;
    }
    return ORC_OK;
}

static int quantize_rows_q8k(const float* input, int rows, int in, int8_t* q, float* s, int16_t* b) {
    /* the per-row quantize loop of RT/Q4KDotKernel.cs:731-738 / RT/Q6KDotKernel.cs:439-446 */
    int spr = in / ORC_QK;
    for (int n = 0; n < rows; n++) {
        int rc = orc_quantize_q8k(input + (size_t)n * in, in, q + (size_t)n * in, s + (size_t)n * spr,
                                  b + (size_t)n * spr * 16);
        if (rc) return rc;
    }
    return ORC_OK;
}

int orc_q4k_project_batched_prequantized(int rows, const uint8_t* blocks, int in, int out, const float* bias,
                                         float* output, const int8_t* q, const float* s, const int16_t* b) {
    /* RT/Q4KDotKernel.cs:765-786 (ProjectBatchedChunk: rows innermost, output = biasO + sum) */
    if (!blocks || !output || !q || !s || !b) return ORC_ERR_NULL;
    if (rows <= 0) return ORC_ERR_RANGE;
    int rc = check_q4k_dims(in, out);
    if (rc) return rc;
    int spr = in / ORC_QK;
    for (int o = 0; o < out; o++) {
        float bias_o = bias == NULL ? 0.0f : bias[o];
        const uint8_t* row = blocks + (size_t)o * spr * ORC_Q4K_BYTES;
        for (int n = 0; n < rows; n++) {
            float sum = q4k_row_sum(row, spr, q + (size_t)n * in, s + (size_t)n * spr, b + (size_t)n * spr * 16);
            output[(size_t)n * out + o] = bias_o + sum;
        }
    }
    return ORC_OK;
}

int orc_q4k_project_batched(const float* input, int rows, const uint8_t* blocks, int in, int out,
                            const float* bias, float* output, int8_t* q, float* s, int16_t* b) {
    /* RT/Q4KDotKernel.cs:681-763 */
    if (!input) return ORC_ERR_NULL;
    if (rows <= 0) return ORC_ERR_RANGE;
    int rc = check_q4k_dims(in, out);
    if (rc) return rc;
    rc = quantize_rows_q8k(input, rows, in, q, s, b);
    if (rc) return rc;
    return orc_q4k_project_batched_prequantized(rows, blocks, in, out, bias, output, q, s, b);
}

int orc_q4k_project_batched_ws(const float* input, int rows, const uint8_t* blocks, int in, int out,
                               const float* bias, float* output, int8_t* q, float* s, int16_t* b) {
    /* RT/Q4KDotKernel.cs:819-955: decode each super-block once per 64-row tile; same per-row order */
    if (!input || !blocks || !output) return ORC_ERR_NULL;
    if (rows <= 0) return ORC_ERR_RANGE;
    int rc = check_q4k_dims(in, out);
    if (rc) return rc;
    rc = quantize_rows_q8k(input, rows, in, q, s, b);
    if (rc) return rc;
    int spr = in / ORC_QK;
    float acc[64];
    uint8_t sc[8], mn[8];
    for (int o = 0; o < out; o++) {
        const uint8_t* rowp = blocks + (size_t)o * spr * ORC_Q4K_BYTES;
        float bias_o = bias == NULL ? 0.0f : bias[o];
        for (int t0 = 0; t0 < rows; t0 += 64) {
            int tile = rows - t0 < 64 ? rows - t0 : 64;
            for (int t = 0; t < tile; t++) acc[t] = 0.0f;
            for (int sb = 0; sb < spr; sb++) {
                const uint8_t* blk = rowp + (size_t)sb * ORC_Q4K_BYTES;
                float d = orc_half_to_float(rd_u16(blk));
                float dmin = orc_half_to_float(rd_u16(blk + 2));
                orc_unpack_q4k_scales_mins(blk + 4, sc, mn);
                for (int t = 0; t < tile; t++) {
                    int n = t0 + t;
                    int32_t main_acc = orc_q4k_main_dot(blk + 16, q + (size_t)n * in + sb * ORC_QK, sc);
                    int32_t min_acc = orc_q4k_min_acc(mn, b + (size_t)n * spr * 16 + sb * 16);
                    acc[t] += s[(size_t)n * spr + sb] * (d * (float)main_acc - dmin * (float)min_acc);
                }
            }
            for (int t = 0; t < tile; t++) {
                output[(size_t)(t0 + t) * out + o] = bias_o + acc[t];
            }
        }
    }
    return ORC_OK;
}

/* ---------------------------------------------------------------- a10 Q6_K projections */

static float q6k_row_sum(const uint8_t* row, int spr, const int8_t* q, const float* s, const int16_t* b) {
    /* RT/Q6KDotKernel.cs:290-301 */
    float sum = 0.0f;
    for (int sb = 0; sb < spr; sb++) {
        sum += orc_q6k_dot(row + (size_t)sb * ORC_Q6K_BYTES, q + sb * ORC_QK, s[sb], b + sb * 16);
    }
    return sum;
}

int orc_q6k_project_prequantized(const uint8_t* blocks, int in, int out, const float* bias, float* output,
                                 const int8_t* q, const float* s, const int16_t* b) {
    /* RT/Q6KDotKernel.cs:274-305 */
    if (!blocks || !output || !q || !s || !b) return ORC_ERR_NULL;
    int rc = check_q4k_dims(in, out);
    if (rc) return rc;
    int spr = in / ORC_QK;
    for (int o = 0; o < out; o++) {
        float sum = q6k_row_sum(blocks + (size_t)o * spr * ORC_Q6K_BYTES, spr, q, s, b);
        output[o] = bias == NULL ? sum : bias[o] + sum;
    }
    return ORC_OK;
}

int orc_q6k_project(const float* input, const uint8_t* blocks, int in, int out, const float* bias,
                    float* output, int8_t* q, float* s, int16_t* b) {
    /* RT/Q6KDotKernel.cs:245-266 */
    if (!input) return ORC_ERR_NULL;
    int rc = check_q4k_dims(in, out);
    if (rc) return rc;
    rc = orc_quantize_q8k(input, in, q, s, b);
    if (rc) return rc;
    return orc_q6k_project_prequantized(blocks, in, out, bias, output, q, s, b);
}

int orc_q6k_project_batched_prequantized(int rows, const uint8_t* blocks, int in, int out, const float* bias,
                                         float* output, const int8_t* q, const float* s, const int16_t* b) {
    /* RT/Q6KDotKernel.cs:473-494 */
    if (!blocks || !output || !q || !s || !b) return ORC_ERR_NULL;
    if (rows <= 0) return ORC_ERR_RANGE;
    int rc = check_q4k_dims(in, out);
    if (rc) return rc;
    int spr = in / ORC_QK;
    for (int o = 0; o < out; o++) {
        float bias_o = bias == NULL ? 0.0f : bias[o];
        const uint8_t* row = blocks + (size_t)o * spr * ORC_Q6K_BYTES;
        for (int n = 0; n < rows; n++) {
            float sum = q6k_row_sum(row, spr, q + (size_t)n * in, s + (size_t)n * spr, b + (size_t)n * spr * 16);
            output[(size_t)n * out + o] = bias_o + sum;
        }
    }
    return ORC_OK;
}

int orc_q6k_project_batched(const float* input, int rows, const uint8_t* blocks, int in, int out,
                            const float* bias, float* output, int8_t* q, float* s, int16_t* b) {
    /* RT/Q6KDotKernel.cs:403-471 */
    if (!input) return ORC_ERR_NULL;
    if (rows <= 0) return ORC_ERR_RANGE;
    int rc = check_q4k_dims(in, out);
    if (rc) return rc;
    rc = quantize_rows_q8k(input, rows, in, q, s, b);
    if (rc) return rc;
    return orc_q6k_project_batched_prequantized(rows, blocks, in, out, bias, output, q, s, b);
}

/* ---------------------------------------------------------------- a12 Q8_0 projections */

int orc_q8_project(const float* input, const int8_t* wq, const float* ws, int in, int out, const float* bias,
                   float* output, int8_t* in_q, float* in_s) {
    /* RT/Q8DotKernel.cs:155-215: output[o] = bias? bias[o] + dot : dot, dot = Dot(W row, input) */
    if (!input || !wq || !ws || !output || !in_q || !in_s) return ORC_ERR_NULL;
    if (in <= 0 || out <= 0) return ORC_ERR_RANGE;
    if (in % ORC_Q8_BLOCK) return ORC_ERR_SIZE;
    int bpr = in / ORC_Q8_BLOCK;
    int rc = orc_quantize_q8_0(input, in, in_q, in_s);
    if (rc) return rc;
    for (int o = 0; o < out; o++) {
        float dot = orc_q8_dot(wq + (size_t)o * in, ws + (size_t)o * bpr, in_q, in_s, in);
        output[o] = bias == NULL ? dot : bias[o] + dot;
    }
    return ORC_OK;
}

int orc_q8_project_heads(const float* x, int rows, int n_heads, int head_dim, int d_model,
                         const int8_t* const* wq, const float* const* ws, const float* bias, float* y) {
    if (!x || !wq || !ws || !y) return ORC_ERR_NULL;
    if (rows <= 0 || n_heads <= 0 || head_dim <= 0 || d_model <= 0) return ORC_ERR_RANGE;
    if (head_dim % ORC_Q8_BLOCK) return ORC_ERR_SIZE;
    for (int h = 0; h < n_heads; h++)
        if (!wq[h] || !ws[h]) return ORC_ERR_NULL;
    const int nb = head_dim / ORC_Q8_BLOCK;
    int8_t* q = (int8_t*)malloc((size_t)head_dim);
    float* s = (float*)malloc((size_t)nb * sizeof(float));
    float* band = (float*)malloc((size_t)d_model * sizeof(float));
    if (!q || !s || !band) {
        free(q);
        free(s);
        free(band);
        return ORC_ERR_NULL;
    }
    for (int n = 0; n < rows; n++) {
        float* out = y + (size_t)n * d_model;
        /* output starts as the attention bias, or zero (CachedMultiHeadAttention.cs:185-194) */
        for (int o = 0; o < d_model; o++) out[o] = bias == NULL ? 0.0f : bias[o];
        for (int h = 0; h < n_heads; h++) {
            /* the head's projection: Q8DotKernel.Project of its attention output, empty bias */
            const float* xh = x + (size_t)n * n_heads * head_dim + (size_t)h * head_dim;
            int rc = orc_quantize_q8_0(xh, head_dim, q, s);
            if (rc) {
                free(q);
                free(s);
                free(band);
                return rc;
            }
            for (int o = 0; o < d_model; o++)
                band[o] = orc_q8_dot(wq[h] + (size_t)o * head_dim, ws[h] + (size_t)o * nb, q, s, head_dim);
            /* output += head output, heads ascending (AddInPlace, CachedMultiHeadAttention.cs:292-297, :946-955) */
            for (int o = 0; o < d_model; o++) out[o] += band[o];
        }
    }
    free(q);
    free(s);
    free(band);
    return ORC_OK;
}

int orc_q8_project_batched_prequantized(int rows, const int8_t* wq, const float* ws, int in, int out,
                                        const float* bias, float* output, const int8_t* in_q,
                                        const float* in_s) {
    /* RT/Q8DotKernel.cs:423-445 */
    if (!wq || !ws || !output || !in_q || !in_s) return ORC_ERR_NULL;
    if (rows <= 0 || in <= 0 || out <= 0) return ORC_ERR_RANGE;
    if (in % ORC_Q8_BLOCK) return ORC_ERR_SIZE;
    int bpr = in / ORC_Q8_BLOCK;
    for (int o = 0; o < out; o++) {
        float bias_o = bias == NULL ? 0.0f : bias[o];
        for (int n = 0; n < rows; n++) {
            float dot = orc_q8_dot(wq + (size_t)o * in, ws + (size_t)o * bpr, in_q + (size_t)n * in,
                                   in_s + (size_t)n * bpr, in);
            output[(size_t)n * out + o] = bias_o + dot;
        }
    }
    return ORC_OK;
}

int orc_q8_project_batched(const float* input, int rows, const int8_t* wq, const float* ws, int in, int out,
                           const float* bias, float* output, int8_t* in_q, float* in_s) {
    /* RT/Q8DotKernel.cs:352-421 */
    if (!input) return ORC_ERR_NULL;
    if (rows <= 0 || in <= 0 || out <= 0) return ORC_ERR_RANGE;
    if (in % ORC_Q8_BLOCK) return ORC_ERR_SIZE;
    int bpr = in / ORC_Q8_BLOCK;
    for (int n = 0; n < rows; n++) {
        int rc = orc_quantize_q8_0(input + (size_t)n * in, in, in_q + (size_t)n * in, in_s + (size_t)n * bpr);
        if (rc) return rc;
    }
    return orc_q8_project_batched_prequantized(rows, wq, ws, in, out, bias, output, in_q, in_s);
}

/* ---------------------------------------------------------------- a18 encoders */

void orc_encode_q4k_block(const float* src, uint8_t* block) {
    /* LD/GgmlQuant.cs:31-126 */
    float sub_scale[8], sub_min[8];
    for (int j = 0; j < 8; j++) {
        float lo = INFINITY, hi = -INFINITY;
        for (int e = 0; e < 32; e++) {
            float v = src[j * 32 + e];
            if (v < lo) lo = v;
            if (v > hi) hi = v;
        }
        if (lo > 0.0f) lo = 0.0f;
        sub_scale[j] = (hi - lo) / 15.0f;
        sub_min[j] = -lo;
    }
    float max_scale = 0.0f, max_min = 0.0f;
    for (int j = 0; j < 8; j++) {
        if (sub_scale[j] > max_scale) max_scale = sub_scale[j];
        if (sub_min[j] > max_min) max_min = sub_min[j];
    }
    float inv_scale = max_scale > 0.0f ? 63.0f / max_scale : 0.0f;
    float inv_min = max_min > 0.0f ? 63.0f / max_min : 0.0f;
    uint8_t sc[8], m[8];
    for (int j = 0; j < 8; j++) {
        int a = (int)rintf(inv_scale * sub_scale[j]);
        int c = (int)rintf(inv_min * sub_min[j]);
        sc[j] = (uint8_t)(a < 63 ? a : 63);
        m[j] = (uint8_t)(c < 63 ? c : 63);
    }
    float d = max_scale / 63.0f;
    float dmin = max_min / 63.0f;
    wr_u16(block, orc_float_to_half(d));
    wr_u16(block + 2, orc_float_to_half(dmin));
    orc_pack_q4k_scales_mins(sc, m, block + 4);
    uint8_t q[256];
    for (int j = 0; j < 8; j++) {
        /* the float d / dmin (not the fp16-rounded ones): LD/GgmlQuant.cs:111-116 */
        float es = d * (float)sc[j];
        float em = dmin * (float)m[j];
        for (int e = 0; e < 32; e++) {
            int i = j * 32 + e;
            int l = es > 0.0f ? (int)rintf((src[i] + em) / es) : 0;
            q[i] = (uint8_t)(l < 0 ? 0 : (l > 15 ? 15 : l));
        }
    }
    uint8_t* qs = block + 16;
    for (int p = 0; p < 4; p++) {
        for (int e = 0; e < 32; e++) {
            qs[32 * p + e] = (uint8_t)(q[64 * p + e] | (q[64 * p + 32 + e] << 4));
        }
    }
}

int orc_quantize_q4k(const float* f32, int in, int out, uint8_t* dst) {
    /* LD/GgmlQuant.cs:132-161 */
    if (!f32 || !dst) return ORC_ERR_NULL;
    if (in <= 0 || out <= 0) return ORC_ERR_RANGE;
    if (in % ORC_QK) return ORC_ERR_SIZE;
    int spr = in / ORC_QK;
    for (int o = 0; o < out; o++) {
        for (int sb = 0; sb < spr; sb++) {
            orc_encode_q4k_block(f32 + (size_t)o * in + sb * ORC_QK, dst + ((size_t)o * spr + sb) * ORC_Q4K_BYTES);
        }
    }
    return ORC_OK;
}

void orc_encode_q6k_block(const float* src, uint8_t* block) {
    /* Build's own encoder (no reference counterpart). Per 16-element sub-block s: the signed value of
     * largest magnitude v_s maps to q = -32, so scale_s = v_s / -32. One fp16 super-scale d carries the
     * 16 int8 sub-scales: iscale = -128 / (scale of largest magnitude), d = 1 / iscale,
     * sc[s] = min(127, rint(iscale * scale_s)). Quants use the fp16-rounded d:
     * l = clamp(rint(x / (dH * sc[s])), -32, 31), q = l + 32. Packing is the exact inverse of the
     * decode layout of LD/GgmlDequant.cs:184-206. */
    float sub_scale[16];
    float max_abs_scale = 0.0f, max_scale = 0.0f;
    for (int s = 0; s < 16; s++) {
        float amax = 0.0f, vmax = 0.0f;
        for (int e = 0; e < 16; e++) {
            float v = src[s * 16 + e];
            float a = fabsf(v);
            if (a > amax) {
                amax = a;
                vmax = v;
            }
        }
        sub_scale[s] = amax > 0.0f ? vmax / -32.0f : 0.0f;
        float as = fabsf(sub_scale[s]);
        if (as > max_abs_scale) {
            max_abs_scale = as;
            max_scale = sub_scale[s];
        }
    }
    memset(block, 0, ORC_Q6K_BYTES);
    if (max_abs_scale == 0.0f) {
        return; /* all-zero block: d = 0, every byte 0 */
    }
    float iscale = -128.0f / max_scale;
    float d = 1.0f / iscale;
    uint16_t dh = orc_float_to_half(d);
    wr_u16(block + 208, dh);
    float dd = orc_half_to_float(dh);
    int8_t sc[16];
    for (int s = 0; s < 16; s++) {
        int v = (int)rintf(iscale * sub_scale[s]);
        sc[s] = (int8_t)(v < 127 ? v : 127);
        block[192 + s] = (uint8_t)sc[s];
    }
    uint8_t q[256];
    for (int s = 0; s < 16; s++) {
        float ds = dd * (float)sc[s];
        for (int e = 0; e < 16; e++) {
            int i = s * 16 + e;
            int l = 0;
            if (ds != 0.0f) {
                l = (int)rintf(src[i] / ds);
                l = l < -32 ? -32 : (l > 31 ? 31 : l);
            }
            q[i] = (uint8_t)(l + 32);
        }
    }
    uint8_t* ql = block;
    uint8_t* qh = block + 128;
    for (int h = 0; h < 2; h++) {
        for (int l = 0; l < 32; l++) {
            int q1 = q[128 * h + l], q2 = q[128 * h + 32 + l], q3 = q[128 * h + 64 + l], q4 = q[128 * h + 96 + l];
            ql[64 * h + l] = (uint8_t)((q1 & 0x0f) | ((q3 & 0x0f) << 4));
            ql[64 * h + 32 + l] = (uint8_t)((q2 & 0x0f) | ((q4 & 0x0f) << 4));
            qh[32 * h + l] = (uint8_t)((q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6));
        }
    }
}

int orc_quantize_q6k(const float* f32, int in, int out, uint8_t* dst) {
    if (!f32 || !dst) return ORC_ERR_NULL;
    if (in <= 0 || out <= 0) return ORC_ERR_RANGE;
    if (in % ORC_QK) return ORC_ERR_SIZE;
    int spr = in / ORC_QK;
    for (int o = 0; o < out; o++) {
        for (int sb = 0; sb < spr; sb++) {
            orc_encode_q6k_block(f32 + (size_t)o * in + sb * ORC_QK, dst + ((size_t)o * spr + sb) * ORC_Q6K_BYTES);
        }
    }
    return ORC_OK;
}

int orc_q8_quantize_rows(const float* rm, int rows, int len, int8_t* quants, float* scales) {
    /* RT/Q8Weight.cs:115-175 */
    if (!rm || !quants || !scales) return ORC_ERR_NULL;
    if (rows <= 0 || len <= 0) return ORC_ERR_RANGE;
    if (len % ORC_Q8_BLOCK) return ORC_ERR_SIZE;
    int bpr = len / ORC_Q8_BLOCK;
    for (int r = 0; r < rows; r++) {
        orc_quantize_q8_0(rm + (size_t)r * len, len, quants + (size_t)r * len, scales + (size_t)r * bpr);
    }
    return ORC_OK;
}

/* ---------------------------------------------------------------- MoE router */

int orc_q5_requantize_q8_0(int type, const uint8_t* src, int rows, int len, int8_t* quants, float* scales) {
    /* A Q5_0 (ggml type 6) or Q5_K (13) tensor of `rows` rows of `len` elements -> the resident Q8_0 planes, as the
     * loader makes them: every block decoded to F32 (GgufReader.LoadQ5RegionAsF32, LD/GgufReader.cs:677-732, and the
     * F32 fallback, LD/GgufLlamaLoader.cs:665-680), then Q8Weight.QuantizeRows (RT/Q8Weight.cs:115-175). */
    if (!src || !quants || !scales) return ORC_ERR_NULL;
    if (rows <= 0 || len <= 0) return ORC_ERR_RANGE;
    const int blk = type == 6 ? 32 : type == 13 ? 256 : 0;
    if (!blk) return ORC_ERR_SIZE;
    if (len % blk) return ORC_ERR_SIZE;
    const int bb = type == 6 ? 22 : 176;
    float* row = (float*)malloc(sizeof(float) * (size_t)len);
    if (!row) return ORC_ERR_NULL;
    for (int r = 0; r < rows; r++) {
        const uint8_t* rb = src + (size_t)r * (len / blk) * bb;
        for (int b = 0; b < len / blk; b++) {
            if (type == 6)
                orc_decode_q5_0_block(rb + (size_t)b * bb, row + (size_t)b * blk);
            else
                orc_decode_q5k_block(rb + (size_t)b * bb, row + (size_t)b * blk);
        }
        orc_q8_quantize_rows(row, 1, len, quants + (size_t)r * len, scales + (size_t)r * (len / ORC_Q8_BLOCK));
    }
    free(row);
    return ORC_OK;
}

int orc_q8_0_deinterleave(const uint8_t* gguf, long n_blocks, int8_t* quants, float* scales) {
    /* LD/GgufReader.cs:250-260: scale = (float)Half(bits), quants copied */
    if (!gguf || !quants || !scales) return ORC_ERR_NULL;
    for (long b = 0; b < n_blocks; b++) {
        const uint8_t* p = gguf + b * 34;
        scales[b] = orc_half_to_float((uint16_t)(p[0] | (p[1] << 8)));
        memcpy(quants + b * 32, p + 2, 32);
    }
    return ORC_OK;
}

int orc_moe_select_topk(const float* logits, int n, int top_k, int* idx, float* w, int normalize) {
    /* RT/MoeRouter.cs:40-128 */
    if (!logits || !idx || !w) return ORC_ERR_NULL;
    if (n <= 0) return ORC_ERR_SIZE;
    if (top_k <= 0) return ORC_ERR_RANGE;
    int k = top_k < n ? top_k : n;
    for (int i = 0; i < k; i++) {
        idx[i] = -1;
        w[i] = -INFINITY;
    }
    int filled = 0;
    for (int e = 0; e < n; e++) {
        float l = logits[e];
        if (filled == k && l <= w[k - 1]) continue;
        int pos = filled < k ? filled : k - 1;
        while (pos > 0 && w[pos - 1] < l) {
            w[pos] = w[pos - 1];
            idx[pos] = idx[pos - 1];
            pos--;
        }
        w[pos] = l;
        idx[pos] = e;
        if (filled < k) filled++;
    }
    float max = w[0];
    if (normalize) {
        float sum = 0.0f;
        for (int i = 0; i < k; i++) {
            float v = expf(w[i] - max);
            w[i] = v;
            sum += v;
        }
        float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
        for (int i = 0; i < k; i++) w[i] *= inv;
    } else {
        float total = 0.0f;
        for (int e = 0; e < n; e++) total += expf(logits[e] - max);
        float inv = total > 0.0f ? 1.0f / total : 0.0f;
        for (int i = 0; i < k; i++) w[i] = expf(w[i] - max) * inv;
    }
    return k;
}

/* ------------------------------------------------------------------------------------------ routed MoE FFN */

static int batched_kq(int type, const float* x, int rows, const uint8_t* blocks, int in, int out, float* y,
                      int8_t* q, float* s, int16_t* b) {
    if (type == 12) return orc_q4k_project_batched(x, rows, blocks, in, out, NULL, y, q, s, b);
    if (type == 14) return orc_q6k_project_batched(x, rows, blocks, in, out, NULL, y, q, s, b);
    return ORC_ERR_RANGE;
}

/* ApplyGeLU (RT/CachedFeedForwardBlock.cs:498-517): x3 = x*x*x; inner = sqrt(2/pi) * (x + 0.044715 * x3);
 * 0.5f * x * (1 + tanh(inner)), in that operation order. */
static float gelu_tanh(float x) {
    const float sqrt_two_over_pi = 0.7978845608028654f;
    const float coeff = 0.044715f;
    const float x3 = x * x * x;
    const float inner = sqrt_two_over_pi * (x + coeff * x3);
    return 0.5f * x * (1.0f + tanhf(inner));
}

int orc_gated_ffn_batched(const float* x, int rows, const uint8_t* gate, const uint8_t* up, const uint8_t* down,
                          int gate_type, int down_type, int d_model, int d_ff, int activation, float* y) {
    /* RT/CachedFeedForwardBlock.cs:328-348 (DecodeSwiGluBatchedDispatched): gate = ProjectBatched(x); ApplyGate
     * (SiLU: gate *= sigmoid(gate), ApplySiLU :464-472; GELU(tanh): ApplyGeLU :498-517); up = ProjectBatched(x);
     * up = gate * up; y = ProjectBatched(up). */
    if (!x || !gate || !up || !down || !y) return ORC_ERR_NULL;
    if (rows <= 0 || d_model % 256 || d_ff % 256) return ORC_ERR_SIZE;
    if (activation != 3 && activation != 4) return ORC_ERR_RANGE;
    const int kmax = d_model > d_ff ? d_model : d_ff;
    float* g = (float*)malloc(sizeof(float) * (size_t)rows * d_ff);
    float* u = (float*)malloc(sizeof(float) * (size_t)rows * d_ff);
    int8_t* q = (int8_t*)malloc((size_t)rows * kmax);
    float* s = (float*)malloc(sizeof(float) * (size_t)rows * (kmax / 256));
    int16_t* b = (int16_t*)malloc(sizeof(int16_t) * (size_t)rows * (kmax / 16));
    int rc = (g && u && q && s && b) ? ORC_OK : ORC_ERR_SIZE;
    if (!rc) rc = batched_kq(gate_type, x, rows, gate, d_model, d_ff, g, q, s, b);
    if (!rc) {
        for (size_t i = 0; i < (size_t)rows * d_ff; i++) {
            if (activation == 4) {
                g[i] = gelu_tanh(g[i]);
            } else {
                const float sig = 1.0f / (1.0f + expf(-g[i]));
                g[i] = g[i] * sig;
            }
        }
        rc = batched_kq(gate_type, x, rows, up, d_model, d_ff, u, q, s, b);
    }
    if (!rc) {
        for (size_t i = 0; i < (size_t)rows * d_ff; i++) u[i] = g[i] * u[i];
        rc = batched_kq(down_type, u, rows, down, d_ff, d_model, y, q, s, b);
    }
    free(g);
    free(u);
    free(q);
    free(s);
    free(b);
    return rc;
}

int orc_swiglu_batched(const float* x, int rows, const uint8_t* gate, const uint8_t* up, const uint8_t* down,
                       int gate_type, int down_type, int d_model, int d_ff, float* y) {
    return orc_gated_ffn_batched(x, rows, gate, up, down, gate_type, down_type, d_model, d_ff, 3, y);
}

int orc_moe_ffn_batched(int n_experts, const uint8_t* const* gate, const uint8_t* const* up,
                        const uint8_t* const* down, int gate_type, int down_type, const float* x, int rows,
                        int d_model, int d_ff, int top_k, const int* idx, const float* w, float* y) {
    /* RT/MoeFeedForwardBlock.cs:140-241 (DecodeBatched) after routing. */
    if (!gate || !up || !down || !x || !idx || !w || !y) return ORC_ERR_NULL;
    if (n_experts <= 0 || rows <= 0 || top_k <= 0) return ORC_ERR_RANGE;
    const size_t P = (size_t)rows * top_k;
    int* row_buf = (int*)malloc(sizeof(int) * (size_t)rows);
    int* slot_buf = (int*)malloc(sizeof(int) * (size_t)rows);
    int* have = (int*)calloc(P, sizeof(int));
    float* gathered = (float*)malloc(sizeof(float) * (size_t)rows * d_model);
    float* expert_out = (float*)malloc(sizeof(float) * (size_t)rows * d_model);
    float* slot_out = (float*)malloc(sizeof(float) * P * d_model);
    int rc = (row_buf && slot_buf && have && gathered && expert_out && slot_out) ? ORC_OK : ORC_ERR_SIZE;
    /* 2. group rows by expert (first matching slot), gather, batched SwiGLU, stash at (row, slot) */
    for (int e = 0; e < n_experts && !rc; e++) {
        int count = 0;
        for (int n = 0; n < rows; n++)
            for (int j = 0; j < top_k; j++)
                if (idx[n * top_k + j] == e) {
                    row_buf[count] = n;
                    slot_buf[count] = j;
                    count++;
                    break;
                }
        if (count == 0) continue;
        for (int c = 0; c < count; c++)
            memcpy(gathered + (size_t)c * d_model, x + (size_t)row_buf[c] * d_model, sizeof(float) * d_model);
        rc = orc_swiglu_batched(gathered, count, gate[e], up[e], down[e], gate_type, down_type, d_model, d_ff,
                                expert_out);
        for (int c = 0; c < count && !rc; c++) {
            const size_t slot = (size_t)row_buf[c] * top_k + slot_buf[c];
            memcpy(slot_out + slot * d_model, expert_out + (size_t)c * d_model, sizeof(float) * d_model);
            have[slot] = 1;
        }
    }
    /* 3. per-row weighted sum in slot order (a slot no expert claimed contributes nothing) */
    for (int n = 0; n < rows && !rc; n++) {
        float* dst = y + (size_t)n * d_model;
        for (int d = 0; d < d_model; d++) dst[d] = 0.0f;
        for (int j = 0; j < top_k; j++) {
            const size_t slot = (size_t)n * top_k + j;
            if (!have[slot]) continue;
            const float wj = w[slot];
            const float* src = slot_out + slot * d_model;
            for (int d = 0; d < d_model; d++) dst[d] += wj * src[d];
        }
    }
    free(row_buf);
    free(slot_buf);
    free(have);
    free(gathered);
    free(expert_out);
    free(slot_out);
    return rc;
}
