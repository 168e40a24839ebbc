// quant.hip — on-device quantisers: the Q8_K / Q8_0 activation quantisers every projection starts with,
// the Q4_K / Q6_K weight encoders, and the row decoders.
//
// All of them are bit-exact restatements of the reference's scalar code: per-operation IEEE binary32
// (the library is built with -ffp-contract=off, and fp32 division / reciprocal are the correctly rounded
// ones), rintf for MathF.Round (round half to even), integer fp32 -> fp16 conversion with ties to even.
#include "ovfq_device.h"
#include "ovfq_launch.h"

namespace ovfq {

// ------------------------------------------------------------------------------------------ Q8_K activation
// Q4KDotKernel.QuantizeActivationQ8K (RT/Q4KDotKernel.cs:71-136): absMax is a max (exact in any order); scale =
// absMax / 127f; inverse = scale > 0 ? 1f / scale : 0f; q = clamp(rint(x * inverse), -127, 127); bsums[g] = sum
// of the 16 quants of group g. Four super-blocks per wave, one per 16-lane DPP row, sixteen consecutive elements (one
// bsum group) per lane: four 16-byte loads and one 16-byte store of quants per lane, the block's absMax by a 4-step
// DPP row max (a wave per block spent most of its time in the 6 cross-lane exchanges of its max).
__global__ __launch_bounds__(256) void quantize_q8k_kernel(const float* __restrict__ x, int64_t n_blocks,
                                                            int8_t* __restrict__ q, float* __restrict__ s,
                                                            int16_t* __restrict__ bs, uint16_t* __restrict__ bh) {
    // wave_id() is a readfirstlane value, so the buffer resource below is provably wave-uniform (SGPRs).
    const int64_t blk0 = ((int64_t)blockIdx.x * 4 + wave_id()) * 4;
    if (blk0 >= n_blocks) return;
    const int lane = threadIdx.x & 63, row = lane >> 4, l16 = lane & 15;
    const int64_t blk = blk0 + row;
    // blocks past the end read zeros (the resource ends with the last block) and store nothing
    const __amdgpu_buffer_rsrc_t xr =
        make_rsrc(x + blk0 * kQK, rsrc_bytes((uint64_t)n_blocks * kQK * 4, (uint64_t)blk0 * kQK * 4));
    float v[16];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const u32x4 t = ld4(xr, (uint32_t)row * 1024u + (uint32_t)l16 * 64u + (uint32_t)i * 16u);
        v[4 * i] = as_float(t.x);
        v[4 * i + 1] = as_float(t.y);
        v[4 * i + 2] = as_float(t.z);
        v[4 * i + 3] = as_float(t.w);
    }
    const Q8KRow r = q8k_quantize_row16(v);
    if (blk < n_blocks) {
        *reinterpret_cast<u32x4*>(q + blk * kQK + l16 * 16) = r.packed;
        bs[blk * 16 + l16] = (int16_t)r.group_sum;
        if (bh) bh[blk * 16 + l16] = __builtin_bit_cast(uint16_t, (_Float16)r.group_sum);
        if (l16 == 0) s[blk] = r.scale;
    }
}

// ------------------------------------------------------------------------------------------ Q8_0 activation
// Q8DotKernel.Quantize (RT/Q8DotKernel.cs:42-91): 32-element blocks, eight lanes per block.
__global__ __launch_bounds__(256) void quantize_q8_0_kernel(const float* __restrict__ x, int64_t n_blocks,
                                                             int8_t* __restrict__ q, float* __restrict__ s) {
    // One wave covers 8 consecutive blocks; the resource starts at the wave's first block (wave-uniform).
    const int64_t wblk = ((int64_t)blockIdx.x * 4 + wave_id()) * 8;
    const int lane = threadIdx.x & 63;
    const int64_t blk = wblk + (lane >> 3);
    if (wblk >= n_blocks) return;
    const int sub = lane & 7;
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(x + wblk * 32, rsrc_bytes((uint64_t)n_blocks * 128, (uint64_t)wblk * 128));
    const Q80Lane r = q8_0_quantize_lane(ld4(xr, lane * 16));
    if (blk < n_blocks) {
        reinterpret_cast<uint32_t*>(q + blk * 32)[sub] = r.packed;
        if (sub == 0) s[blk] = r.scale;
    }
}

// ------------------------------------------------------------------------------------------ Q4_K encoder
// GgmlQuant.EncodeQ4_KBlock (LD/GgmlQuant.cs:31-126): one thread per 256-element super-block.
__global__ __launch_bounds__(256) void encode_q4k_kernel(const float* __restrict__ w, int64_t n_blocks,
                                                          uint8_t* __restrict__ dst) {
    const int64_t blk = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (blk >= n_blocks) return;
    const float* src = w + blk * kQK;
    float sub_scale[8], sub_min[8];
    for (int j = 0; j < 8; j++) {
        float lo = __builtin_inff(), hi = -__builtin_inff();
        for (int e = 0; e < 32; e++) {
            const float v = src[j * 32 + e];
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
    const float inv_scale = max_scale > 0.0f ? 63.0f / max_scale : 0.0f;
    const float inv_min = max_min > 0.0f ? 63.0f / max_min : 0.0f;
    uint32_t sc[8], m[8];
    for (int j = 0; j < 8; j++) {
        const int a = (int)rintf(inv_scale * sub_scale[j]);
        const int c = (int)rintf(inv_min * sub_min[j]);
        sc[j] = (uint32_t)(a < 63 ? a : 63);
        m[j] = (uint32_t)(c < 63 ? c : 63);
    }
    const float d = max_scale / 63.0f;
    const float dmin = max_min / 63.0f;
    uint32_t* out = reinterpret_cast<uint32_t*>(dst + blk * kQ4KBytes);
    out[0] = (uint32_t)float_to_half_rne(d) | ((uint32_t)float_to_half_rne(dmin) << 16);
    // PackScalesMins (LD/GgmlQuant.cs:164-172), four bytes per 32-bit word.
    uint32_t p0 = 0, p1 = 0, p2 = 0;
    for (int j = 0; j < 4; j++) {
        p0 |= ((sc[j] & 0x3f) | ((sc[j + 4] >> 4) << 6)) << (8 * j);
        p1 |= ((m[j] & 0x3f) | ((m[j + 4] >> 4) << 6)) << (8 * j);
        p2 |= ((sc[j + 4] & 0x0f) | ((m[j + 4] & 0x0f) << 4)) << (8 * j);
    }
    out[1] = p0;
    out[2] = p1;
    out[3] = p2;
    // Nibbles from the float d / dmin (LD/GgmlQuant.cs:108-116): qs[32p+e] = q[64p+e] | q[64p+32+e] << 4.
    for (int p = 0; p < 4; p++) {
        const float es_lo = d * (float)sc[2 * p], em_lo = dmin * (float)m[2 * p];
        const float es_hi = d * (float)sc[2 * p + 1], em_hi = dmin * (float)m[2 * p + 1];
        for (int e4 = 0; e4 < 32; e4 += 4) {
            uint32_t word = 0;
            for (int k = 0; k < 4; k++) {
                const int e = e4 + k;
                int l0 = es_lo > 0.0f ? (int)rintf((src[64 * p + e] + em_lo) / es_lo) : 0;
                int l1 = es_hi > 0.0f ? (int)rintf((src[64 * p + 32 + e] + em_hi) / es_hi) : 0;
                l0 = l0 < 0 ? 0 : (l0 > 15 ? 15 : l0);
                l1 = l1 < 0 ? 0 : (l1 > 15 ? 15 : l1);
                word |= (uint32_t)(l0 | (l1 << 4)) << (8 * k);
            }
            out[4 + (32 * p + e4) / 4] = word;
        }
    }
}

// ------------------------------------------------------------------------------------------ Q6_K encoder
// The build's own Q6_K encoder (the reference has none): the signed value of largest magnitude in each
// 16-element sub-block maps to q = -32; one fp16 super-scale d = 1 / (-128 / largest sub-scale) carries 16
// int8 sub-scales; quants are rint(x / (fp16(d) * sc)) clamped to [-32, 31], stored +32. The byte layout is
// the inverse of GgmlDequant.DecodeQ6_KBlock (LD/GgmlDequant.cs:143-209).
__global__ __launch_bounds__(256) void encode_q6k_kernel(const float* __restrict__ w, int64_t n_blocks,
                                                          uint8_t* __restrict__ dst) {
    const int64_t blk = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (blk >= n_blocks) return;
    const float* src = w + blk * kQK;
    uint8_t* out = dst + blk * kQ6KBytes;  // 210-byte stride: 2-byte aligned, so store 16-bit halves
    float sub_scale[16];
    float max_abs_scale = 0.0f, max_scale = 0.0f;
    for (int s = 0; s < 16; s++) {
        float amax = 0.0f, vmax = 0.0f;
        for (int e = 0; e < 16; e++) {
            const float v = src[s * 16 + e];
            const float a = fabsf(v);
            if (a > amax) {
                amax = a;
                vmax = v;
            }
        }
        sub_scale[s] = amax > 0.0f ? vmax / -32.0f : 0.0f;
        const float as = fabsf(sub_scale[s]);
        if (as > max_abs_scale) {
            max_abs_scale = as;
            max_scale = sub_scale[s];
        }
    }
    uint16_t* o16 = reinterpret_cast<uint16_t*>(out);
    if (max_abs_scale == 0.0f) {
        for (int i = 0; i < kQ6KBytes / 2; i++) o16[i] = 0;
        return;
    }
    const float iscale = -128.0f / max_scale;
    const float d = 1.0f / iscale;
    const uint16_t dh = float_to_half_rne(d);
    const float dd = half_bits_to_float(dh);
    int sc[16];
    for (int s = 0; s < 16; s++) {
        const int v = (int)rintf(iscale * sub_scale[s]);
        sc[s] = v < 127 ? v : 127;
    }
    for (int i = 0; i < 8; i++) {
        o16[96 + i] = (uint16_t)((uint32_t)(sc[2 * i] & 0xff) | ((uint32_t)(sc[2 * i + 1] & 0xff) << 8));
    }
    o16[104] = dh;
    auto quant = [&](int i) -> int {
        const float ds = dd * (float)sc[i >> 4];
        int l = 0;
        if (ds != 0.0f) {
            l = (int)rintf(src[i] / ds);
            l = l < -32 ? -32 : (l > 31 ? 31 : l);
        }
        return l + 32;
    };
    for (int h = 0; h < 2; h++) {
        for (int l = 0; l < 32; l += 2) {
            uint32_t qlA = 0, qlB = 0, qh = 0;
            for (int k = 0; k < 2; k++) {
                const int q1 = quant(128 * h + l + k), q2 = quant(128 * h + 32 + l + k);
                const int q3 = quant(128 * h + 64 + l + k), q4 = quant(128 * h + 96 + l + k);
                qlA |= (uint32_t)((q1 & 0x0f) | ((q3 & 0x0f) << 4)) << (8 * k);
                qlB |= (uint32_t)((q2 & 0x0f) | ((q4 & 0x0f) << 4)) << (8 * k);
                qh |= (uint32_t)((q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6)) << (8 * k);
            }
            o16[(64 * h + l) / 2] = (uint16_t)qlA;
            o16[(64 * h + 32 + l) / 2] = (uint16_t)qlB;
            o16[(128 + 32 * h + l) / 2] = (uint16_t)qh;
        }
    }
}

// ------------------------------------------------------------------------------------------ row decode
// GgmlDequant.DecodeQ4_KBlock (LD/GgmlDequant.cs:95-141) over one output row: one thread per element.
__global__ __launch_bounds__(256) void decode_row_q4k_kernel(const uint8_t* __restrict__ row, float* __restrict__ dst) {
    const uint8_t* b = row + (size_t)blockIdx.x * kQ4KBytes;
    const int i = threadIdx.x;
    const int p = i >> 6, hi = (i >> 5) & 1, e = i & 31;
    const float d = half_bits_to_float((uint16_t)(b[0] | (b[1] << 8)));
    const float dmin = half_bits_to_float((uint16_t)(b[2] | (b[3] << 8)));
    const uint8_t* q = b + 4;
    const int j = 2 * p + hi;
    int sc, m;
    if (j < 4) {
        sc = q[j] & 63;
        m = q[j + 4] & 63;
    } else {
        sc = (q[j + 4] & 0x0f) | ((q[j - 4] >> 6) << 4);
        m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
    const int packed = b[16 + 32 * p + e];
    const int nib = hi ? (packed >> 4) : (packed & 0x0f);
    const float scale = d * (float)sc;
    const float mn = dmin * (float)m;
    dst[(size_t)blockIdx.x * kQK + i] = scale * (float)nib - mn;
}

// GgmlDequant.DecodeQ6_KBlock (LD/GgmlDequant.cs:143-209): dst = d * s * (q - 32).
__global__ __launch_bounds__(256) void decode_row_q6k_kernel(const uint8_t* __restrict__ row, float* __restrict__ dst) {
    const uint8_t* b = row + (size_t)blockIdx.x * kQ6KBytes;
    const int i = threadIdx.x;
    const int h = i >> 7, r = i & 127, grp = r >> 5, l = r & 31;
    const int qlb = b[64 * h + l + ((grp & 1) ? 32 : 0)];
    const int nib = (grp >= 2) ? (qlb >> 4) : (qlb & 0x0f);
    const int hb = (b[128 + 32 * h + l] >> (2 * grp)) & 3;
    const int q = nib | (hb << 4);
    const int s = (int8_t)b[192 + 8 * h + (l >> 4) + 2 * grp];
    const float d = half_bits_to_float((uint16_t)(b[208] | (b[209] << 8)));
    dst[(size_t)blockIdx.x * kQK + i] = d * (float)s * (float)(q - 32);
}

// Q8Weight.DecodeRow (RT/Q8Weight.cs:81-106): dst[i] = scale[block] * quant[i].
__global__ __launch_bounds__(256) void decode_row_q8_0_kernel(const int8_t* __restrict__ q, const float* __restrict__ s,
                                                              int n, float* __restrict__ dst) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    dst[i] = s[i >> 5] * (float)q[i];
}

// ------------------------------------------------------------------------------------------ launchers

// ------------------------------------------------------------------------------------------ GGUF Q8_0 upload
// GgufReader.LoadTensorQ8_0Raw (LD/GgufReader.cs:198-266): the file's 34-byte blocks (fp16 d, 32 int8) become the
// resident planes — quants copied, d widened exactly to f32. One thread per block; blocks are 2-byte aligned, so
// the block is read as 17 halfwords.
__global__ __launch_bounds__(256) void q8_0_deinterleave_kernel(const uint16_t* __restrict__ src, int64_t n_blocks,
                                                                uint32_t* __restrict__ q, float* __restrict__ s) {
    const int64_t blk = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (blk >= n_blocks) return;
    const uint16_t* b = src + blk * 17;
    s[blk] = half_bits_to_float(b[0]);
#pragma unroll
    for (int i = 0; i < 8; i++) q[blk * 8 + i] = (uint32_t)b[1 + 2 * i] | ((uint32_t)b[2 + 2 * i] << 16);
}

// ------------------------------------------------------------------------------------------ GGUF Q5_0 / Q5_K upload
// The loader keeps 5-bit tensors as Q8_0 (LD/GgufLlamaLoader.cs:665-680 for experts, the F32 fallback of the
// per-layer tensors): every block decoded to F32 as GgmlDequant.DecodeQ5_0Block / DecodeQ5_KBlock do
// (LD/GgmlDequant.cs:222-320), then requantised with Q8Weight.QuantizeRows (RT/Q8Weight.cs:115-175). Here both
// happen in registers: eight lanes per 32-element Q8_0 block, four elements per lane, the block's absmax by three
// lane exchanges. Rows are whole numbers of blocks, so the flat 32-element block index of the tensor is also the
// block index of the resident planes. Source blocks are 2-byte aligned (22 bytes) or 16-byte aligned (176 bytes);
// they are read byte by byte (load time only).
__global__ __launch_bounds__(256) void q5_to_q8_0_kernel(const uint8_t* __restrict__ src, int kquant, int64_t n_blocks,
                                                         int8_t* __restrict__ q, float* __restrict__ s) {
    const int64_t wblk = ((int64_t)blockIdx.x * 4 + wave_id()) * 8;
    if (wblk >= n_blocks) return;
    const int lane = threadIdx.x & 63;
    const int64_t blk = wblk + (lane >> 3);
    const int sub = lane & 7;
    const bool live = blk < n_blocks;
    float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (live && !kquant) {
        // Q5_0: d fp16 @0, qh @2 (bit i = the 5th bit of element i), qs @6 (element i < 16: low nibble of qs[i],
        // element i >= 16: high nibble of qs[i - 16]); value (q - 16) * d.
        const uint8_t* b = src + blk * 22;
        const float d = half_bits_to_float((uint16_t)(b[0] | (b[1] << 8)));
        const uint32_t qh = (uint32_t)b[2] | ((uint32_t)b[3] << 8) | ((uint32_t)b[4] << 16) | ((uint32_t)b[5] << 24);
        for (int k = 0; k < 4; k++) {
            const int i = 4 * sub + k;
            const int packed = b[6 + (i & 15)];
            const int nib = i < 16 ? (packed & 0x0f) : (packed >> 4);
            const int x = (nib | (int)(((qh >> i) & 1u) << 4)) - 16;
            v[k] = (float)x * d;
        }
    } else if (live) {
        // Q5_K: the Q4_K header (d, dmin, 12 packed scale/min bytes), qh @16, qs @48. Sub-block j = 2g + h of the
        // super-block takes the low (h = 0) or high (h = 1) nibbles of qs[32g ..] and qh bit 2g + h of qh[l].
        const uint8_t* b = src + (blk >> 3) * 176;
        const int j = (int)(blk & 7), g = j >> 1, h = j & 1;
        const float d = half_bits_to_float((uint16_t)(b[0] | (b[1] << 8)));
        const float dmin = half_bits_to_float((uint16_t)(b[2] | (b[3] << 8)));
        const uint8_t* pk = b + 4;
        int sc, m;
        if (j < 4) {
            sc = pk[j] & 63;
            m = pk[j + 4] & 63;
        } else {
            sc = (pk[j + 4] & 0x0f) | ((pk[j - 4] >> 6) << 4);
            m = (pk[j + 4] >> 4) | ((pk[j] >> 6) << 4);
        }
        const float scale = d * (float)sc;
        const float mn = dmin * (float)m;
        for (int k = 0; k < 4; k++) {
            const int l = 4 * sub + k;
            const int packed = b[48 + 32 * g + l];
            const int nib = h ? (packed >> 4) : (packed & 0x0f);
            const int hi = ((b[16 + l] >> (2 * g + h)) & 1) ? 16 : 0;
            v[k] = scale * (float)(nib + hi) - mn;
        }
    }
    u32x4 raw;
    raw.x = __builtin_bit_cast(uint32_t, v[0]);
    raw.y = __builtin_bit_cast(uint32_t, v[1]);
    raw.z = __builtin_bit_cast(uint32_t, v[2]);
    raw.w = __builtin_bit_cast(uint32_t, v[3]);
    const Q80Lane r = q8_0_quantize_lane(raw);  // every lane of the block takes part in the exchanges
    if (live) {
        reinterpret_cast<uint32_t*>(q + blk * 32)[sub] = r.packed;
        if (sub == 0) s[blk] = r.scale;
    }
}

hipError_t launch_q5_to_q8_0(const void* gguf, bool q5k, int64_t n_blocks, int8_t* q, float* s, hipStream_t st) {
    if (n_blocks <= 0) return hipSuccess;
    const int64_t grid = (n_blocks * 8 + 255) / 256;
    hipLaunchKernelGGL(q5_to_q8_0_kernel, dim3((unsigned)grid), dim3(256), 0, st, static_cast<const uint8_t*>(gguf),
                       q5k ? 1 : 0, n_blocks, q, s);
    return hipGetLastError();
}

hipError_t launch_quantize_q8k(const float* x, int64_t n_blocks, int8_t* q, float* s, int16_t* b, hipStream_t st,
                               uint16_t* bh) {
    if (n_blocks <= 0) return hipSuccess;
    const int64_t grid = (n_blocks + 15) / 16;
    hipLaunchKernelGGL(quantize_q8k_kernel, dim3((unsigned)grid), dim3(256), 0, st, x, n_blocks, q, s, b, bh);
    return hipGetLastError();
}

hipError_t launch_quantize_q8_0(const float* x, int64_t n_blocks, int8_t* q, float* s, hipStream_t st) {
    if (n_blocks <= 0) return hipSuccess;
    const int64_t grid = (n_blocks * 8 + 255) / 256;
    hipLaunchKernelGGL(quantize_q8_0_kernel, dim3((unsigned)grid), dim3(256), 0, st, x, n_blocks, q, s);
    return hipGetLastError();
}

hipError_t launch_q8_0_deinterleave(const void* gguf, int64_t n_blocks, int8_t* q, float* s, hipStream_t st) {
    if (n_blocks <= 0) return hipSuccess;
    hipLaunchKernelGGL(q8_0_deinterleave_kernel, dim3((unsigned)((n_blocks + 255) / 256)), dim3(256), 0, st,
                       static_cast<const uint16_t*>(gguf), n_blocks, reinterpret_cast<uint32_t*>(q), s);
    return hipGetLastError();
}

hipError_t launch_encode_q4k(const float* w, int64_t n_blocks, uint8_t* dst, hipStream_t st) {
    if (n_blocks <= 0) return hipSuccess;
    hipLaunchKernelGGL(encode_q4k_kernel, dim3((unsigned)((n_blocks + 255) / 256)), dim3(256), 0, st, w, n_blocks, dst);
    return hipGetLastError();
}

hipError_t launch_encode_q6k(const float* w, int64_t n_blocks, uint8_t* dst, hipStream_t st) {
    if (n_blocks <= 0) return hipSuccess;
    hipLaunchKernelGGL(encode_q6k_kernel, dim3((unsigned)((n_blocks + 255) / 256)), dim3(256), 0, st, w, n_blocks, dst);
    return hipGetLastError();
}

hipError_t launch_decode_row(int type, const void* blocks, const float* scales, int in, int row, float* dst,
                             hipStream_t st) {
    if (type == 12) {
        const uint8_t* r = static_cast<const uint8_t*>(blocks) + (size_t)row * (in / kQK) * kQ4KBytes;
        hipLaunchKernelGGL(decode_row_q4k_kernel, dim3(in / kQK), dim3(256), 0, st, r, dst);
    } else if (type == 14) {
        const uint8_t* r = static_cast<const uint8_t*>(blocks) + (size_t)row * (in / kQK) * kQ6KBytes;
        hipLaunchKernelGGL(decode_row_q6k_kernel, dim3(in / kQK), dim3(256), 0, st, r, dst);
    } else {
        const int8_t* q = static_cast<const int8_t*>(blocks) + (size_t)row * in;
        const float* s = scales + (size_t)row * (in / 32);
        hipLaunchKernelGGL(decode_row_q8_0_kernel, dim3((in + 255) / 256), dim3(256), 0, st, q, s, in, dst);
    }
    return hipGetLastError();
}

}  // namespace ovfq
