// mfma.hip — batched (prefill) Q4_K / Q6_K projection on CDNA4 int8 MFMA (v_mfma_i32_16x16x64_i8).
//
// ProjectBatched / ProjectBatchedWeightStationary (RT/Q4KDotKernel.cs:681-955, RT/Q6KDotKernel.cs:403-510):
// y[n][o] = biasO + sum over super-blocks (ascending) of the block's fp32 value, for every activation row n.
//
// Exactness. Everything before the per-super-block fp32 tail is integer arithmetic, so it can be regrouped:
//  Q4_K  mainAcc = sum_e (sc*nib)_e * q8_e. sc*nib <= 945 does not fit int8, so the scale is split as
//        sc = 8*sc_hi + sc_lo (both in [0,7]); the operands sc_lo*nib and sc_hi*nib are <= 105, two MFMAs give
//        sum lo*q8 and sum hi*q8, mainAcc = acc_lo + (acc_hi << 3).
//        minAcc = sum_s m_s * (bsums[2s] + bsums[2s+1]) = sum_e m_{s(e)} * q8_e: in the small-M kernel a third MFMA
//        whose weight operand is the sub-block min broadcast over its 32 elements; in the tiled kernel one
//        v_mfma_f32_16x16x16_f16 per 16-row sub-tile over the 16 bsums of each row (|bsums| <= 2032 and m <= 63
//        are exact in fp16, every partial sum is an integer below 2^24, so the fp32 result is minAcc exactly).
//  Q6_K  unsignedTerm - 32*bsumTerm = sum_e sc_{s(e)} * (q_e - 32) * q8_e. W = sc*(q-32) lies in [-4064, 4096]
//        (sc = -128 is a legal scale), split as 256*hi + lo with lo the signed low byte of W (in [-128,127]) and
//        hi = (W + 128) >> 8 (in [-16,16]); two MFMAs, mainAcc = acc_lo + (acc_hi << 8).
// The regroupings use the Q8_K definition bsums[j] = sum of quants 16j..16j+15 (the quantiser's output); only the
// tiled Q4_K kernel reads the bsums plane. The fp32 tail of each super-block — q8Scale * (d*mainAcc - dmin*minAcc) and
// d*q8Scale*mainAcc (RT/Q4KDotKernel.cs:944, RT/Q6KDotKernel.cs:114-115) — is evaluated per (n, o) in the
// reference's operation order and accumulated over super-blocks in ascending order from +0, then biasO + sum.
//
// Tiling. A workgroup (4 waves) owns 64 weight rows (16 per wave) x NT activation rows. MFMA operand A is the
// activation (row n = lane % 16 of a 16-row sub-tile, staged in LDS), operand B the weights (column o = lane % 16:
// the lane's own weight row, built in registers straight from the GGUF bytes), so the 4 results a lane holds,
// D[4*(lane/16) + i][lane % 16], all belong to its own weight row: d, dmin and the bias stay lane-local. In both
// operands byte j of lane-group g = lane / 16 carries K index 16*g + j of a 64-element chunk.
// Per super-block the workgroup stages NT rows x 256 quants (+ scales, and for Q4_K the rows' bsums) in LDS by DMA
// (double-buffered; 256-byte rows whose 16-byte slots are XOR-swizzled by row, so the 16 lanes reading one K slice
// hit distinct banks) while the next super-block's weights and activation are in flight. Workgroups are numbered XCD-aware: the workgroups of one weight tile run consecutively on the
// same XCD (blockIdx % 8), so its bytes come from HBM once and from that XCD's L2 for the other activation tiles.
#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <type_traits>
#include <utility>

#include "kquant_blocks.h"
#include "ovfq_device.h"
#include "ovfq_launch.h"

namespace ovfq {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));

struct MJob {
    const uint8_t* w;
    const uint8_t* pre;  // MFMA-ready copy (used when the launch is the prepared variant)
    const float* bias;
    float* y;
    int n_out;  // output size of this weight
    int tile0;  // first 64-row tile index of this job in the launch
};

// Grouped (MoE) launch: tile list entry t = expert e | (tile i << 8) covers pairs expert_off[e] + [64 i, 64 i + 64);
// gate/up pairs (w1 set) share the launch, the first o_tiles1 weight tiles being gate's.
struct MGroup {
    const uint8_t* w0[kMaxExperts];
    const uint8_t* w1[kMaxExperts];
    const int* expert_off;
    const int* pair_row;  // activation row of each pair (NULL: pair p reads row p)
    const int* tiles;
    const int* tile_count;
    float* y0;
    float* y1;
    int n_rows;    // outputs per matrix
    int o_tiles1;  // 64-row weight tiles of one matrix
};

struct MArgs {
    MJob job[kMaxJobs];
    int njobs;
    int o_tiles;  // 64-row weight tiles over all jobs
    int n_tiles;  // ceil(M / NT); grouped: the tile list's bound
    int m_rows;   // M; grouped: activation rows
    int spr;      // K / 256
    const int8_t* q;
    const float* s;
    const int16_t* b;    // Q8_K bsums (Q4_K: the min term's activation operand)
    const uint16_t* bh;  // the same bsums as fp16 (kernels instantiated with BH read these instead)
    MGroup grp;
};


__device__ __forceinline__ i32x4 mfma16(i32x4 a, i32x4 b, i32x4 c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// Two dwords of 16-bit lanes (pe: K bytes 0 and 2, po: K bytes 1 and 3), each holding u = v + 128 for a value v in
// [-4064, 4224) (two's complement): lo = the low byte of v as int8 (v mod 256, signed), hi = u >> 8 (the high byte of
// u), so that v = 256*hi + lo, as packed bytes in K order. v_perm_b32 gathers bytes 0 and 2 of each source (selector
// 0x06020400 = [pe.b0, po.b0, pe.b2, po.b2]) or bytes 1 and 3 (0x07030501); the low byte of v is the low byte of u
// with its top bit flipped.
__device__ __forceinline__ void split_lo_hi(uint32_t pe, uint32_t po, uint32_t& lo, uint32_t& hi) {
    lo = __builtin_amdgcn_perm(po, pe, 0x06020400u) ^ 0x80808080u;
    hi = __builtin_amdgcn_perm(po, pe, 0x07030501u);
}

// K permutation. The four MFMAs t = 0..3 of a super-block each cover 64 of its 256 elements; lane-group g of
// MFMA t holds 16 consecutive elements starting at base(t, g), in both operands. The activation row is staged in
// LDS as 16-byte pieces in (t, g) order (logical slot 4t + g), so a lane reads its A operand with one
// ds_read_b128. The bases are chosen so that every nibble/bit-field shift on the weight side is a compile-time
// constant. Rows are 256 bytes with the slot XOR-swizzled by (row % 16): the 16 lanes of an A read (16 rows, one
// logical slot) then hit 16 distinct 16-byte bank groups.

// ------------------------------------------------------------------------------------------ Q4_K weight operands
struct Q4KMfma {
    static constexpr int kBytes = kQ4KBytes;
    static constexpr int kNumMfma = 3;  // lo, hi, min
    // MFMA t: nibble (t >> 1) of qs[64(t & 1) + 16g + j]  ->  element 128(t&1) + 64(g>>1) + 32(t>>1) + 16(g&1) + j
    // (qs byte b holds elements 64(b/32) + b%32 in its low nibble and +32 in its high nibble).
    // LDS slot 4t + g holds source piece (element / 16) s with bits [t&1, g>>1, t>>1, g&1].
    __device__ __forceinline__ static uint32_t src_piece(uint32_t slot) {
        const uint32_t t = slot >> 2, g = slot & 3u;
        return 8u * (t & 1u) + 4u * (g >> 1) + 2u * (t >> 1) + (g & 1u);
    }
    struct W {
        u32x4 h;      // d, dmin, 12 packed scale/min bytes
        u32x4 q[2];   // qs[16g .. +16], qs[64 + 16g .. +16]
    };
    __device__ __forceinline__ static W load(__amdgpu_buffer_rsrc_t r, uint32_t off, int g) {
        W w;
        w.h = ld4(r, off);
        w.q[0] = ld4(r, off + 16 + 16 * g);
        w.q[1] = ld4(r, off + 16 + 64 + 16 * g);
        return w;
    }
    // The min MFMA's B operand for lane group g: m_{2g}, m_{2g}, m_{2g+1}, m_{2g+1} in fp16, from the eight 6-bit
    // mins (LD/GgmlDequant.cs:64-79 unpacking; lane group g takes sub-blocks 2g and 2g + 1).
    __device__ __forceinline__ static u32x2 min_operand(const W& w, int g) {
        const uint32_t m_lo = w.h.z & 0x3f3f3f3fu;
        const uint32_t m_hi = ((w.h.w >> 4) & 0x0f0f0f0fu) | ((w.h.z >> 2) & 0x30303030u);
        const uint32_t mg = (g < 2 ? m_lo : m_hi) >> (16 * (g & 1));
        const uint32_t m0 = __builtin_bit_cast(uint16_t, (_Float16)(mg & 0xffu));
        const uint32_t m1 = __builtin_bit_cast(uint16_t, (_Float16)((mg >> 8) & 0xffu));
        return u32x2{m0 * 0x00010001u, m1 * 0x00010001u};
    }
    // Sub-block of MFMA t, lane-group g: js = 4(t&1) + 2(g>>1) + (t>>1) (LD/GgmlDequant.cs:64-79 unpacking).
    template <int T>
    __device__ __forceinline__ static void operands(const W& w, int g, i32x4 (&op)[kNumMfma]) {
        const uint32_t jj = (uint32_t)(2 * (g >> 1) + (T >> 1)) * 8;  // byte index js & 3
        uint32_t sc, m;
        if ((T & 1) == 0) {  // js < 4
            sc = (w.h.y >> jj) & 63u;
            m = (w.h.z >> jj) & 63u;
        } else {
            const uint32_t A = w.h.y >> jj, B = w.h.z >> jj, C = (w.h.w >> jj) & 0xffu;
            sc = (C & 0x0fu) | ((A >> 2) & 0x30u);
            m = (C >> 4) | ((B >> 2) & 0x30u);
        }
        const u32x4 src = w.q[T & 1];
        const uint32_t qv[4] = {src.x, src.y, src.z, src.w};
        constexpr uint32_t kShift = (T >> 1) * 4;
        // sc = 8*sc_hi + sc_lo with both parts in [0, 7]: sc_lo*nib and sc_hi*nib are <= 105, so one packed 16-bit
        // multiply of the four nibble bytes gives the four byte products with no carry between bytes.
        const unsigned short sl = (unsigned short)(sc & 7u), sh = (unsigned short)(sc >> 3);
        const u16x2 sl2 = {sl, sl}, sh2 = {sh, sh};
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const u16x2 nib = __builtin_bit_cast(u16x2, (qv[k] >> kShift) & 0x0f0f0f0fu);
            lo[k] = __builtin_bit_cast(uint32_t, nib * sl2);
            hi[k] = __builtin_bit_cast(uint32_t, nib * sh2);
        }
        op[0] = i32x4{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3]};
        op[1] = i32x4{(int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
        const int mm = (int)__builtin_amdgcn_perm(0u, m, 0u);  // m in all four bytes
        op[2] = i32x4{mm, mm, mm, mm};
    }
    __device__ __forceinline__ static float d_of(const W& w) { return half_lo(w.h.x); }
    __device__ __forceinline__ static float dmin_of(const W& w) { return half_hi(w.h.x); }
    __device__ __forceinline__ static uint32_t raw_scales(const W& w) { return w.h.x; }  // fp16 d | fp16 dmin << 16
    // q8Scale * (d * mainAcc - dmin * minAcc)   (RT/Q4KDotKernel.cs:944)
    __device__ __forceinline__ static float tail(const i32x4 (&acc)[kNumMfma], int i, float d, float dmin,
                                                 float q8s) {
        const int main_acc = acc[0][i] + (acc[1][i] << 3);
        return q8s * (d * (float)main_acc - dmin * (float)acc[2][i]);
    }
};

// ------------------------------------------------------------------------------------------ Q6_K weight operands
struct Q6KMfma {
    static constexpr int kBytes = kQ6KBytes;
    static constexpr int kNumMfma = 2;  // lo, hi
    // MFMA t = qh bit pair p: element 128h + 32p + l with h = g >> 1, l = 16(g&1) + j: nibble (p >> 1) of
    // ql[64h + 32(p&1) + l], bits 2p of qh[32h + l], scale sc[8h + 2p + (g&1)] (RT/Q6KDotKernel.cs:189-213).
    // LDS slot 4p + g holds source piece s with bits [g>>1, p, p, g&1].
    __device__ __forceinline__ static uint32_t src_piece(uint32_t slot) {
        const uint32_t p = slot >> 2, g = slot & 3u;
        return 8u * (g >> 1) + 2u * p + (g & 1u);
    }
    struct W {
        uint32_t ql[2][4];  // ql[64h + 16(g&1) .. +16], ql[64h + 32 + 16(g&1) .. +16]
        uint32_t qh[4];     // qh[32h + 16(g&1) .. +16]
        uint32_t sc;        // byte p = sc[8h + 2p + (g&1)]
        uint32_t d;
    };
    __device__ __forceinline__ static W load(__amdgpu_buffer_rsrc_t r, uint32_t off, int g) {
        W w;
        const uint32_t h = (uint32_t)g >> 1, l0 = 16u * (uint32_t)(g & 1);
        Q6K::run16(r, off + 64 * h + l0, w.ql[0]);
        Q6K::run16(r, off + 64 * h + 32 + l0, w.ql[1]);
        Q6K::run16(r, off + 128 + 32 * h + l0, w.qh);
        const uint32_t so = off + 192 + 8 * h, sh = so & 3u;
        const u32x3 sv = ld3(r, so & ~3u);
        const uint32_t s0 = __builtin_amdgcn_alignbyte(sv.y, sv.x, sh), s1 = __builtin_amdgcn_alignbyte(sv.z, sv.y, sh);
        w.sc = __builtin_amdgcn_perm(s1, s0, (g & 1) ? 0x07050301u : 0x06040200u);
        w.d = __builtin_amdgcn_raw_buffer_load_b16(r, (int)(off + 208), 0, 0);
        return w;
    }
    __device__ __forceinline__ static u32x2 min_operand(const W&, int) { return u32x2{0u, 0u}; }
    template <int P>
    __device__ __forceinline__ static void operands(const W& w, int, i32x4 (&op)[kNumMfma]) {
        // W + 128 = sc * q - 32 * sc + 128 (W = sc * (q - 32) in [-4064, 4096]), computed per 16-bit lane modulo
        // 2^16 (two's complement).
        const uint32_t scp = (uint32_t)(int)(int8_t)((w.sc >> (8 * P)) & 0xffu);
        const uint32_t sc16 = scp & 0xffffu, bias16 = (128u - 32u * scp) & 0xffffu;
        const u16x2 sc2 = {(unsigned short)sc16, (unsigned short)sc16};
        const u16x2 bias2 = {(unsigned short)bias16, (unsigned short)bias16};
        constexpr uint32_t kNib = (P >> 1) * 4, kBits = 2 * P;
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t qhb = kBits <= 4 ? (w.qh[k] << (4 - kBits)) : (w.qh[k] >> (kBits - 4));
            const uint32_t q = ((w.ql[P & 1][k] >> kNib) & 0x0f0f0f0fu) | (qhb & 0x30303030u);
            const uint32_t qe = __builtin_amdgcn_perm(0u, q, 0x0c020c00u);  // K bytes 0, 2 as 16-bit lanes
            const uint32_t qo = __builtin_amdgcn_perm(0u, q, 0x0c030c01u);  // K bytes 1, 3
            const u16x2 we = __builtin_bit_cast(u16x2, qe) * sc2 + bias2;
            const u16x2 wo = __builtin_bit_cast(u16x2, qo) * sc2 + bias2;
            split_lo_hi(__builtin_bit_cast(uint32_t, we), __builtin_bit_cast(uint32_t, wo), lo[k], hi[k]);
        }
        op[0] = i32x4{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3]};
        op[1] = i32x4{(int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
    }
    __device__ __forceinline__ static float d_of(const W& w) { return half_lo(w.d); }
    __device__ __forceinline__ static float dmin_of(const W&) { return 0.0f; }
    __device__ __forceinline__ static uint32_t raw_scales(const W& w) { return w.d; }  // fp16 d
    // d * q8Scale * mainAcc   (RT/Q6KDotKernel.cs:114-115)
    __device__ __forceinline__ static float tail(const i32x4 (&acc)[kNumMfma], int i, float d, float, float q8s) {
        const int main_acc = acc[0][i] + (acc[1][i] << 8);
        return d * q8s * (float)main_acc;
    }
};

// ------------------------------------------------------------------------------------------ MFMA-ready weights
// An optional second resident copy of a Q6_K weight holding, for every 16-row tile and super-block, exactly the B
// operands the kernels below build from the GGUF bytes: the lo and hi operand of each of the four 64-element
// chunks (1 KiB each, lane-major, so a wave loads one with a single coalesced dwordx4 per lane), then 8 bytes per
// lane: a word left for per-chunk bytes (the Q4_K mins, were a Q4_K copy kept) and the block's raw fp16 d (| dmin
// << 16 for Q4_K). The copy is written by the same operand functions, so a prepared weight's MFMA inputs - and
// outputs - are bit-identical; the batched kernel then skips the per-block operand build (for Q6_K, 12 VALU per
// 4 weights). Q4_K keeps building its operands: after the split-scale form they cost less than streaming 3.7x the
// bytes (measured: the Q4_K gate/up launch at M = 512 was 10 % slower prepared, the Q6_K down 23 % faster).
constexpr int kPreOps = 8 * 1024;
constexpr int kPreHdr = 64 * 8;
constexpr int kPreBlock = kPreOps + kPreHdr;

size_t mfma_prepared_bytes(int in, int out) { return (size_t)((out + 63) / 64) * 4 * (size_t)(in / kQK) * kPreBlock; }

// One wave per (16-row tile, super-block); rows past the matrix read zero bytes (their outputs are never stored).
template <class F>
__global__ __launch_bounds__(256) void mfma_prepare_kernel(const uint8_t* __restrict__ w, int n_rows, int spr,
                                                           int tiles16, uint8_t* __restrict__ pre) {
    const int item = (int)blockIdx.x * 4 + wave_id();
    if (item >= tiles16 * spr) return;
    const int tile = item / spr, sb = item % spr;
    const int lane = threadIdx.x & 63, g = lane >> 4, r16 = lane & 15;
    const uint32_t row_bytes = (uint32_t)spr * F::kBytes;
    const uint64_t wbase = (uint64_t)tile * 16 * row_bytes;
    const uint64_t wbase4 = wbase & ~3ull;
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(w + wbase4, rsrc_bytes((uint64_t)n_rows * row_bytes, wbase4));
    const typename F::W wv =
        F::load(wr, (uint32_t)(wbase - wbase4) + (uint32_t)r16 * row_bytes + (uint32_t)sb * F::kBytes, g);
    i32x4 op[4][F::kNumMfma];
    F::template operands<0>(wv, g, op[0]);
    F::template operands<1>(wv, g, op[1]);
    F::template operands<2>(wv, g, op[2]);
    F::template operands<3>(wv, g, op[3]);
    uint8_t* dst = pre + ((size_t)tile * spr + sb) * kPreBlock;
    uint32_t mins = 0;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        *reinterpret_cast<i32x4*>(dst + (2 * t) * 1024 + lane * 16) = op[t][0];
        *reinterpret_cast<i32x4*>(dst + (2 * t + 1) * 1024 + lane * 16) = op[t][1];
        if constexpr (F::kNumMfma == 3) mins |= ((uint32_t)op[t][2][0] & 0xffu) << (8 * t);
    }
    *reinterpret_cast<u32x2*>(dst + kPreOps + lane * 8) = u32x2{mins, F::raw_scales(wv)};
}

hipError_t launch_mfma_prepare(int type, const uint8_t* w, int in, int out, uint8_t* pre, hipStream_t st) {
    const int spr = in / kQK, tiles16 = (out + 63) / 64 * 4;
    const int64_t waves = (int64_t)tiles16 * spr;
    const dim3 grid((unsigned)((waves + 3) / 4));
    if (type != 14) return hipErrorInvalidValue;  // Q6_K only (the batched kernel reads no Q4_K copy)
    hipLaunchKernelGGL(mfma_prepare_kernel<Q6KMfma>, grid, dim3(256), 0, st, w, out, spr, tiles16, pre);
    return hipGetLastError();
}

// A prepared super-block of one lane: the eight chunk operands and the header.
struct PreW {
    u32x4 op[8];
    u32x2 hdr;
};

// ------------------------------------------------------------------------------------------ kernel
template <class F, int NT, bool PRE, bool GRP, bool BH = false>
__global__ __launch_bounds__(256, 2) void kquant_mfma_kernel(const MArgs a) {
    static_assert(!(PRE && GRP), "grouped launches read the GGUF operands");
    constexpr int kSub = NT / 16;
    constexpr int kDma = NT / 16;  // 1 KiB (4-row) activation DMA chunks per wave per super-block
    __shared__ __align__(16) uint8_t act[2][NT * 256];
    __shared__ __align__(16) float act_s[2][NT];
    // Q4_K: the min term is one v_mfma_f32_16x16x16_f16 per 16-row sub-tile and super-block, minAcc = sum over the 16
    // groups k of m_{k/2} * bsums[k], from the activation's bsums (int16 in LDS, [row][16], converted to fp16 as
    // read) and the sub-block mins: every product and partial sum is an integer below 2^24 (|bsums| <= 16 * 127,
    // m <= 63), so the fp32 result is minAcc exactly, in place of the third int8 MFMA per 64-element chunk.
    constexpr bool kMinF16 = F::kNumMfma == 3;
    __shared__ __align__(16) int16_t act_b[2][kMinF16 ? NT * 16 : 8];

    const int wave = wave_id();
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4, r16 = lane & 15;
    const int b = blockIdx.x;
    const int local = b >> 3;
    const int o_tile = (b & 7) + 8 * (local / a.n_tiles);
    const int n_tile = local % a.n_tiles;
    if (o_tile >= a.o_tiles) return;  // uniform over the workgroup
    // weight rows, output and activation rows of this tile (all wave-uniform)
    const uint8_t* wptr;
    const uint8_t* preptr = nullptr;
    const float* bias = nullptr;
    float* y;
    int n_out, o0, n0, m_valid;
    int pbeg = 0;  // grouped: the expert's first pair (output row of tile row 0 is pbeg + n0)
    if constexpr (GRP) {
        if (n_tile >= a.grp.tile_count[0]) return;
        const int te = a.grp.tiles[n_tile];
        const int e = te & 0xff;
        const int mat = o_tile >= a.grp.o_tiles1 ? 1 : 0;
        wptr = mat ? a.grp.w1[e] : a.grp.w0[e];
        y = mat ? a.grp.y1 : a.grp.y0;
        n_out = a.grp.n_rows;
        o0 = (o_tile - mat * a.grp.o_tiles1) * 64 + wave * 16;
        pbeg = a.grp.expert_off[e];
        n0 = (te >> 8) * NT;
        m_valid = min(NT, a.grp.expert_off[e + 1] - pbeg - n0);
    } else {
        int j = 0;
#pragma unroll
        for (int t = 1; t < kMaxJobs; t++)
            if (t < a.njobs && o_tile >= a.job[t].tile0) j = t;
        wptr = a.job[j].w;
        preptr = a.job[j].pre;
        bias = a.job[j].bias;
        y = a.job[j].y;
        n_out = a.job[j].n_out;
        o0 = (o_tile - a.job[j].tile0) * 64 + wave * 16;  // this wave's first weight row
        n0 = n_tile * NT;
        m_valid = min(NT, a.m_rows - n0);
    }
    const int spr = a.spr;
    const uint32_t K = (uint32_t)spr * kQK;
    const uint32_t row_bytes = (uint32_t)spr * F::kBytes;

    const uint64_t wbase = (uint64_t)o0 * row_bytes;
    const uint64_t wbase4 = wbase & ~3ull;
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(wptr + wbase4, rsrc_bytes((uint64_t)n_out * row_bytes, wbase4));
    const uint32_t woff = (uint32_t)(wbase - wbase4) + (uint32_t)r16 * row_bytes;
    // prepared copy: this wave's 16-row tile, spr blocks of kPreBlock bytes
    const uint64_t pbase = (uint64_t)(o0 / 16) * (uint64_t)spr * kPreBlock;
    const __amdgpu_buffer_rsrc_t pr =
        make_rsrc(preptr + (PRE ? pbase : 0),
                  PRE ? rsrc_bytes((uint64_t)((n_out + 63) / 64) * 4 * spr * kPreBlock, pbase) : 0u);
    // Activation: the tile's rows from row n0 on; grouped, the whole activation with each row gathered (tile row r
    // is pair pbeg + n0 + r, activation row pair_row[that]); rows past the tile's pairs point past the resource.
    const uint64_t a0 = GRP ? 0 : (uint64_t)n0;
    const __amdgpu_buffer_rsrc_t qr =
        make_rsrc(a.q + a0 * K, rsrc_bytes((uint64_t)a.m_rows * K, a0 * K));
    const __amdgpu_buffer_rsrc_t sr =
        make_rsrc(a.s + a0 * spr, rsrc_bytes((uint64_t)a.m_rows * spr * 4, a0 * spr * 4));
    auto act_row = [&](uint32_t r) -> uint32_t {  // resource-relative activation row of tile row r
        if constexpr (GRP) {
            if ((int)r >= m_valid) return (uint32_t)a.m_rows;
            const int p = pbeg + n0 + (int)r;
            return (uint32_t)(a.grp.pair_row ? a.grp.pair_row[p] : p);
        } else {
            return r;
        }
    };
    // Q4_K bsums, 32 bytes a tile row, by LDS DMA with the quants: waves w < NT / 32 move rows 32w .. 32w + 31, lane L
    // half L % 2 of row 32w + L / 2.
    const int16_t* bsrc = BH ? reinterpret_cast<const int16_t*>(a.bh) : a.b;
    const __amdgpu_buffer_rsrc_t br =
        make_rsrc(bsrc + (kMinF16 ? a0 * spr * 16 : 0),
                  kMinF16 ? rsrc_bytes((uint64_t)a.m_rows * spr * 32, a0 * spr * 32) : 0u);
    const uint32_t b_src =
        kMinF16 && wave < NT / 32 ? act_row(32u * wave + ((uint32_t)lane >> 1)) * (uint32_t)spr * 32u + 16u * (lane & 1)
                                  : 0u;
    // DMA chunk c = wave * kDma + i covers LDS bytes [1024c, 1024c + 1024): lane L writes physical slot L % 16 of
    // row 4c + L / 16, which holds logical slot (L % 16) ^ (row % 16).
    uint32_t dma_src[kDma];
#pragma unroll
    for (int i = 0; i < kDma; i++) {
        const uint32_t row = 4u * (uint32_t)(wave * kDma + i) + ((uint32_t)lane >> 4);
        dma_src[i] = act_row(row) * K + 16u * F::src_piece(((uint32_t)lane & 15u) ^ (row & 15u));
    }
    const uint32_t s_src = wave * 64 < NT ? act_row(threadIdx.x) * (uint32_t)spr * 4u : 0u;
    // Reads past the last super-block of a row land in the next row or past the resource: harmless (not used).
    auto stage = [&](int sb, int buf) {
#pragma unroll
        for (int i = 0; i < kDma; i++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                qr, (__attribute__((address_space(3))) void*)&act[buf][1024 * (wave * kDma + i)], 16,
                (int)(dma_src[i] + (uint32_t)sb * kQK), 0, 0, 0);
        if (wave * 64 < NT)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                sr, (__attribute__((address_space(3))) void*)&act_s[buf][wave * 64], 4,
                (int)(s_src + (uint32_t)sb * 4u), 0, 0, 0);
        if (kMinF16 && wave < NT / 32)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                br, (__attribute__((address_space(3))) void*)&act_b[buf][512 * wave], 16,
                (int)(b_src + (uint32_t)sb * 32u), 0, 0, 0);
    };
    // A-operand byte offset of logical slot 4t + g in row r16 of a sub-tile: ((4t + g) ^ r16) = 4t ^ (g ^ r16).
    uint32_t a_off[4];
#pragma unroll
    for (int t = 0; t < 4; t++) a_off[t] = (uint32_t)r16 * 256u + (((uint32_t)(g ^ r16)) ^ (4u * t)) * 16u;

    float out[kSub][4];
#pragma unroll
    for (int s = 0; s < kSub; s++)
#pragma unroll
        for (int i = 0; i < 4; i++) out[s][i] = 0.0f;

    // MFMAs and fp32 tail of one super-block from the weight operands `op` and the block's d / dmin; Q4_K: mb = the
    // min MFMA's B operand (m_{2g}, m_{2g}, m_{2g+1}, m_{2g+1} in fp16: lane group g holds groups 4g .. 4g + 3).
    auto mma_tail = [&](int buf, const i32x4 (&op)[4][F::kNumMfma], float d, float dmin, u32x2 mb) {
        const uint8_t* tile = act[buf];
        if constexpr (kMinF16) {
            // Sub-tile s's MFMAs, then sub-tile s - 1's tail (its results are ready by then), one stage after another:
            // two sub-tiles' accumulators live, not all four (left to itself the compiler overlaps every sub-tile and
            // needs 132-146 VGPRs, three waves per SIMD). The same staging measured slower for Q6_K.
            i32x4 pacc[2];
            f32x4 pmn;
#pragma unroll
            for (int s = 0; s <= kSub; s++) {
                i32x4 acc[2] = {i32x4{0, 0, 0, 0}, i32x4{0, 0, 0, 0}};
                f32x4 mn = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                if (s < kSub) {
#pragma unroll
                    for (int t = 0; t < 4; t++) {
                        const u32x4 av = *reinterpret_cast<const u32x4*>(tile + s * 4096 + a_off[t]);
                        const i32x4 aop = i32x4{(int)av.x, (int)av.y, (int)av.z, (int)av.w};
                        acc[0] = mfma16(aop, op[t][0], acc[0]);
                        acc[1] = mfma16(aop, op[t][1], acc[1]);
                    }
                    // the row's bsums 4g .. 4g + 3 as fp16 (exact: |b| <= 2048)
                    f16x4 bq;
                    if constexpr (BH) {
                        bq = *reinterpret_cast<const f16x4*>(&act_b[buf][(s * 16 + r16) * 16 + 4 * g]);
                    } else {
                        const s16x4 bi = *reinterpret_cast<const s16x4*>(&act_b[buf][(s * 16 + r16) * 16 + 4 * g]);
                        bq = f16x4{(_Float16)bi.x, (_Float16)bi.y, (_Float16)bi.z, (_Float16)bi.w};
                    }
                    mn = __builtin_amdgcn_mfma_f32_16x16x16f16(bq, __builtin_bit_cast(f16x4, mb), mn, 0, 0, 0);
                }
                if (s > 0) {
                    const f32x4 q8s = *reinterpret_cast<const f32x4*>(&act_s[buf][(s - 1) * 16 + 4 * g]);
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int main_acc = pacc[0][i] + (pacc[1][i] << 3);
                        // q8Scale * (d * mainAcc - dmin * minAcc)   (RT/Q4KDotKernel.cs:944)
                        out[s - 1][i] += q8s[i] * (d * (float)main_acc - dmin * pmn[i]);
                    }
                }
                pacc[0] = acc[0];
                pacc[1] = acc[1];
                pmn = mn;
                __builtin_amdgcn_sched_barrier(0);
            }
            return;
        }
#pragma unroll
        for (int s = 0; s < kSub; s++) {
            i32x4 acc[F::kNumMfma];
#pragma unroll
            for (int k = 0; k < F::kNumMfma; k++) acc[k] = i32x4{0, 0, 0, 0};
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const u32x4 av = *reinterpret_cast<const u32x4*>(tile + s * 4096 + a_off[t]);
                const i32x4 aop = i32x4{(int)av.x, (int)av.y, (int)av.z, (int)av.w};
#pragma unroll
                for (int k = 0; k < F::kNumMfma; k++) acc[k] = mfma16(aop, op[t][k], acc[k]);
            }
            const f32x4 q8s = *reinterpret_cast<const f32x4*>(&act_s[buf][s * 16 + 4 * g]);
#pragma unroll
            for (int i = 0; i < 4; i++) out[s][i] += F::tail(acc, i, d, dmin, q8s[i]);
        }
    };

    if constexpr (!PRE) {
        auto compute = [&](int buf, const typename F::W& w) {
            i32x4 op[4][F::kNumMfma];
            F::template operands<0>(w, g, op[0]);
            F::template operands<1>(w, g, op[1]);
            F::template operands<2>(w, g, op[2]);
            F::template operands<3>(w, g, op[3]);
            mma_tail(buf, op, F::d_of(w), F::dmin_of(w), F::min_operand(w, g));
        };
        typename F::W wcur = F::load(wr, woff, g);
        stage(0, 0);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if constexpr (F::kNumMfma == 3) {
            // Q4_K: two super-blocks per iteration, the weight registers alternating without copies (3-5 % faster
            // on MI355X; the Q6_K build is slower unrolled). Same loads, waits and barriers as the loop below.
            typename F::W walt;
            for (int sb = 0; sb < spr; sb += 2) {
                walt = F::load(wr, woff + (uint32_t)(sb + 1) * F::kBytes, g);  // past the row: unused
                if (sb + 1 < spr) stage(sb + 1, 1);
                compute(0, wcur);
                __builtin_amdgcn_s_waitcnt(0);
                __syncthreads();
                if (sb + 1 >= spr) break;
                wcur = F::load(wr, woff + (uint32_t)(sb + 2) * F::kBytes, g);
                if (sb + 2 < spr) stage(sb + 2, 0);
                compute(1, walt);
                __builtin_amdgcn_s_waitcnt(0);
                __syncthreads();
            }
        } else {
            for (int sb = 0; sb < spr; sb++) {
                // next super-block's weights (registers) and activation (LDS DMA) in flight during this one's compute
                const typename F::W wnxt = F::load(wr, woff + (uint32_t)(sb + 1) * F::kBytes, g);  // past the row: unused
                if (sb + 1 < spr) stage(sb + 1, (sb + 1) & 1);
                compute(sb & 1, wcur);
                wcur = wnxt;
                __builtin_amdgcn_s_waitcnt(0);  // the DMA writes to LDS are complete before the barrier publishes them
                __syncthreads();
            }
        }
    } else {
        auto load_pre = [&](int sb) {
            PreW p;
            const uint32_t base = (uint32_t)sb * kPreBlock + (uint32_t)lane * 16u;
#pragma unroll
            for (int q = 0; q < 8; q++) p.op[q] = ld4(pr, base + (uint32_t)q * 1024u);
            p.hdr = ld2(pr, (uint32_t)sb * kPreBlock + kPreOps + (uint32_t)lane * 8u);
            return p;
        };
        auto compute = [&](int buf, const PreW& p) {
            i32x4 op[4][F::kNumMfma];
#pragma unroll
            for (int t = 0; t < 4; t++) {
                op[t][0] = __builtin_bit_cast(i32x4, p.op[2 * t]);
                op[t][1] = __builtin_bit_cast(i32x4, p.op[2 * t + 1]);
                if constexpr (F::kNumMfma == 3) {
                    const int mm = (int)__builtin_amdgcn_perm(0u, p.hdr.x, 0x01010101u * (uint32_t)t);
                    op[t][2] = i32x4{mm, mm, mm, mm};
                }
            }
            mma_tail(buf, op, half_lo(p.hdr.y), F::kNumMfma == 3 ? half_hi(p.hdr.y) : 0.0f, u32x2{0u, 0u});
        };
        PreW pcur = load_pre(0);
        stage(0, 0);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        for (int sb = 0; sb < spr; sb++) {
            const PreW pnxt = load_pre(sb + 1);  // past the tile's blocks: resource-clamped or unused
            if (sb + 1 < spr) stage(sb + 1, (sb + 1) & 1);
            compute(sb & 1, pcur);
            pcur = pnxt;
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
        }
    }

    // y[n][o] = biasO + sum   (RT/Q4KDotKernel.cs:951, RT/Q6KDotKernel.cs:507); grouped: output row pbeg + n
    const int o = o0 + r16;
    if (o >= n_out) return;
    const float bias_o = bias ? bias[o] : 0.0f;
#pragma unroll
    for (int s = 0; s < kSub; s++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int n = s * 16 + 4 * g + i;
            if (n < m_valid) y[(size_t)(pbeg + n0 + n) * n_out + o] = bias_o + out[s][i];
        }
}

// ------------------------------------------------------------------------------------------ pair kernel
// The dense 64-row kernel with two waves per 16 weight rows: an 8-wave workgroup owns the same 64 x 64 tile, wave w
// and wave w + 4 share weight rows 16(w & 3) .. + 15 and take alternate super-blocks (w < 4 the even ones, w >= 4
// the odd ones), so a launch whose grid gives each CU only one or two tiles (long inputs, few output rows) keeps twice
// the waves per SIMD at the same instruction count. Each super-block pair is staged in two LDS slots (every wave moves
// a quarter of its parity's slot); the odd wave writes its 16 x 64 block values to LDS and the even wave adds them
// after its own, so every (row, output) is still summed in ascending super-block order. Per pair: the weight operands
// are built (the pair's activation DMA in flight), a wait and a barrier publish the slots, the next pair's weights
// are loaded, the MFMAs and tails run, a barrier frees both slots and publishes the odd values, the next pair's DMA is
// issued, and the even wave adds the odd values.
template <class F, bool BH>
__global__ __launch_bounds__(512) void kquant_mfma_pair_kernel(const MArgs a) {
    constexpr int NT = 64;
    constexpr int kSub = NT / 16;
    constexpr bool kMinF16 = F::kNumMfma == 3;
    __shared__ __align__(16) uint8_t act[2][NT * 256];
    __shared__ __align__(16) float act_s[2][NT];
    __shared__ __align__(16) int16_t act_b[2][kMinF16 ? NT * 16 : 8];
    __shared__ __align__(16) f32x4 xch[4][kSub * 64];  // the odd waves' block values, [weight group][sub-tile][lane]

    const int wave = wave_id();
    const int wg = wave & 3, par = wave >> 2;
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4, r16 = lane & 15;
    const int b = blockIdx.x;
    const int local = b >> 3;
    const int o_tile = (b & 7) + 8 * (local / a.n_tiles);
    const int n_tile = local % a.n_tiles;
    if (o_tile >= a.o_tiles) return;  // uniform over the workgroup
    int j = 0;
#pragma unroll
    for (int t = 1; t < kMaxJobs; t++)
        if (t < a.njobs && o_tile >= a.job[t].tile0) j = t;
    const uint8_t* wptr = a.job[j].w;
    const float* bias = a.job[j].bias;
    float* y = a.job[j].y;
    const int n_out = a.job[j].n_out;
    const int o0 = (o_tile - a.job[j].tile0) * 64 + wg * 16;  // this wave's first weight row
    const int n0 = n_tile * NT;
    const int m_valid = min(NT, a.m_rows - n0);
    const int spr = a.spr;
    const uint32_t K = (uint32_t)spr * kQK;
    const uint32_t row_bytes = (uint32_t)spr * F::kBytes;

    const uint64_t wbase = (uint64_t)o0 * row_bytes;
    const uint64_t wbase4 = wbase & ~3ull;
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(wptr + wbase4, rsrc_bytes((uint64_t)n_out * row_bytes, wbase4));
    const uint32_t woff = (uint32_t)(wbase - wbase4) + (uint32_t)r16 * row_bytes;
    const uint64_t a0 = (uint64_t)n0;
    const __amdgpu_buffer_rsrc_t qr = make_rsrc(a.q + a0 * K, rsrc_bytes((uint64_t)a.m_rows * K, a0 * K));
    const __amdgpu_buffer_rsrc_t sr =
        make_rsrc(a.s + a0 * spr, rsrc_bytes((uint64_t)a.m_rows * spr * 4, a0 * spr * 4));
    const int16_t* bsrc = BH ? reinterpret_cast<const int16_t*>(a.bh) : a.b;
    const __amdgpu_buffer_rsrc_t br =
        make_rsrc(bsrc + (kMinF16 ? a0 * spr * 16 : 0),
                  kMinF16 ? rsrc_bytes((uint64_t)a.m_rows * spr * 32, a0 * spr * 32) : 0u);
    // Slot `par` holds super-block 2p + par. Wave (wg, par) moves its slot's 1 KiB chunks 4wg .. 4wg + 3 (lane L:
    // physical 16-byte slot L % 16 of row 4c + L / 16, holding logical slot (L % 16) ^ (row % 16)), the scales (wg 0:
    // lane L row L) and, for Q4_K, half the bsums (wg < 2: lane L half L % 2 of row 32wg + L / 2).
    uint32_t dma_src[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t row = 4u * (uint32_t)(4 * wg + i) + ((uint32_t)lane >> 4);
        dma_src[i] = row * K + 16u * F::src_piece(((uint32_t)lane & 15u) ^ (row & 15u));
    }
    const uint32_t s_src = (uint32_t)lane * (uint32_t)spr * 4u;
    const uint32_t b_src = kMinF16 && wg < 2 ? (32u * wg + ((uint32_t)lane >> 1)) * (uint32_t)spr * 32u + 16u * (lane & 1)
                                             : 0u;
    const int npair = (spr + 1) / 2;
    auto stage = [&](int p) {
        const int sb = 2 * p + par;
        if (sb >= spr) return;  // wave-uniform: an odd tail super-block that does not exist
#pragma unroll
        for (int i = 0; i < 4; i++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                qr, (__attribute__((address_space(3))) void*)&act[par][1024 * (4 * wg + i)], 16,
                (int)(dma_src[i] + (uint32_t)sb * kQK), 0, 0, 0);
        if (wg == 0)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(sr, (__attribute__((address_space(3))) void*)&act_s[par][0], 4,
                                                     (int)(s_src + (uint32_t)sb * 4u), 0, 0, 0);
        if (kMinF16 && wg < 2)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                br, (__attribute__((address_space(3))) void*)&act_b[par][512 * wg], 16,
                (int)(b_src + (uint32_t)sb * 32u), 0, 0, 0);
    };
    uint32_t a_off[4];
#pragma unroll
    for (int t = 0; t < 4; t++) a_off[t] = (uint32_t)r16 * 256u + (((uint32_t)(g ^ r16)) ^ (4u * t)) * 16u;

    float out[kSub][4];
#pragma unroll
    for (int s = 0; s < kSub; s++)
#pragma unroll
        for (int i = 0; i < 4; i++) out[s][i] = 0.0f;

    typename F::W w = F::load(wr, woff + (uint32_t)par * F::kBytes, g);
    stage(0);
    for (int p = 0; p < npair; p++) {
        const bool live = 2 * p + par < spr;  // wave-uniform
        i32x4 op[4][F::kNumMfma];
        F::template operands<0>(w, g, op[0]);
        F::template operands<1>(w, g, op[1]);
        F::template operands<2>(w, g, op[2]);
        F::template operands<3>(w, g, op[3]);
        const float d = F::d_of(w), dmin = F::dmin_of(w);
        const u32x2 mb = F::min_operand(w, g);
        __builtin_amdgcn_s_waitcnt(0);  // this wave's share of the pair's slots has landed
        __syncthreads();
        // the next pair's weights (past the row: resource-clamped or unused)
        w = F::load(wr, woff + (uint32_t)(2 * p + 2 + par) * F::kBytes, g);
        if (live) {
            const uint8_t* tile = act[par];
#pragma unroll
            for (int s = 0; s < kSub; s++) {
                i32x4 acc[F::kNumMfma];
#pragma unroll
                for (int k = 0; k < F::kNumMfma; k++) acc[k] = i32x4{0, 0, 0, 0};
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    const u32x4 av = *reinterpret_cast<const u32x4*>(tile + s * 4096 + a_off[t]);
                    const i32x4 aop = i32x4{(int)av.x, (int)av.y, (int)av.z, (int)av.w};
                    acc[0] = mfma16(aop, op[t][0], acc[0]);
                    acc[1] = mfma16(aop, op[t][1], acc[1]);
                }
                const f32x4 q8s = *reinterpret_cast<const f32x4*>(&act_s[par][s * 16 + 4 * g]);
                f32x4 v;
                if constexpr (kMinF16) {
                    f16x4 bq;
                    if constexpr (BH) {
                        bq = *reinterpret_cast<const f16x4*>(&act_b[par][(s * 16 + r16) * 16 + 4 * g]);
                    } else {
                        const s16x4 bi = *reinterpret_cast<const s16x4*>(&act_b[par][(s * 16 + r16) * 16 + 4 * g]);
                        bq = f16x4{(_Float16)bi.x, (_Float16)bi.y, (_Float16)bi.z, (_Float16)bi.w};
                    }
                    const f32x4 mn = __builtin_amdgcn_mfma_f32_16x16x16f16(bq, __builtin_bit_cast(f16x4, mb),
                                                                          f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int main_acc = acc[0][i] + (acc[1][i] << 3);
                        // q8Scale * (d * mainAcc - dmin * minAcc)   (RT/Q4KDotKernel.cs:944)
                        v[i] = q8s[i] * (d * (float)main_acc - dmin * mn[i]);
                    }
                } else {
#pragma unroll
                    for (int i = 0; i < 4; i++) v[i] = F::tail(acc, i, d, dmin, q8s[i]);
                }
                if (par == 0) {
#pragma unroll
                    for (int i = 0; i < 4; i++) out[s][i] += v[i];
                } else {
                    xch[wg][s * 64 + lane] = v;
                }
            }
        }
        __syncthreads();  // both slots read; the odd values visible
        if (p + 1 < npair) stage(p + 1);
        if (par == 0 && 2 * p + 1 < spr) {
#pragma unroll
            for (int s = 0; s < kSub; s++) {
                const f32x4 v = xch[wg][s * 64 + lane];
#pragma unroll
                for (int i = 0; i < 4; i++) out[s][i] += v[i];
            }
        }
    }

    // y[n][o] = biasO + sum   (RT/Q4KDotKernel.cs:951, RT/Q6KDotKernel.cs:507): the even waves hold the sums
    const int o = o0 + r16;
    if (par != 0 || o >= n_out) return;
    const float bias_o = bias ? bias[o] : 0.0f;
#pragma unroll
    for (int s = 0; s < kSub; s++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int n = s * 16 + 4 * g + i;
            if (n < m_valid) y[(size_t)(n0 + n) * n_out + o] = bias_o + out[s][i];
        }
}

// ------------------------------------------------------------------------------------------ pair-wide kernel
// The pair kernel over 128 activation rows: an 8-wave workgroup owns 64 weight rows x 128 activation rows; waves w
// and w + 4 share weight rows 16(w & 3) .. + 15 and take the even / odd super-blocks, and each covers all 128 rows
// in two 64-row halves (as the wide kernel), so every operand build serves 128 rows while a small grid (long inputs,
// few output rows) still keeps two waves per SIMD. Per super-block pair: the operands are built; a wait and a barrier
// publish the first halves; the second halves' DMA and the next pair's weights are issued; the first half is
// computed (the odd waves write their block values to LDS); a barrier; the next pair's first halves are DMA'd, the
// even waves add the odd values and compute the second half; a barrier; the even waves add the odd second-half
// values. Each (row, output) is summed in ascending super-block order. The code is specialised per parity so that
// every slot a wave reads or DMAs is a fixed LDS object (see the wide kernel).
template <class F, bool BH>
__global__ __launch_bounds__(512) void kquant_mfma_pairwide_kernel(const MArgs a) {
    constexpr int NH = 64;
    constexpr int kSubH = NH / 16;
    constexpr bool kMinF16 = F::kNumMfma == 3;
    constexpr int kB = kMinF16 ? NH * 16 : 8;
    // [parity][half] slots
    __shared__ __align__(16) uint8_t act00[NH * 256], act01[NH * 256], act10[NH * 256], act11[NH * 256];
    __shared__ __align__(16) float act_s00[NH], act_s01[NH], act_s10[NH], act_s11[NH];
    __shared__ __align__(16) int16_t act_b00[kB], act_b01[kB], act_b10[kB], act_b11[kB];
    // the odd waves' block values of the first / second half, [weight group][sub-tile][lane]
    __shared__ __align__(16) f32x4 xch0[4][kSubH * 64], xch1[4][kSubH * 64];

    const int wave = wave_id();
    const int wg = wave & 3, par = wave >> 2;
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4, r16 = lane & 15;
    const int b = blockIdx.x;
    const int local = b >> 3;
    const int o_tile = (b & 7) + 8 * (local / a.n_tiles);
    const int n_tile = local % a.n_tiles;
    if (o_tile >= a.o_tiles) return;  // uniform over the workgroup
    int j = 0;
#pragma unroll
    for (int t = 1; t < kMaxJobs; t++)
        if (t < a.njobs && o_tile >= a.job[t].tile0) j = t;
    const uint8_t* wptr = a.job[j].w;
    const float* bias = a.job[j].bias;
    float* y = a.job[j].y;
    const int n_out = a.job[j].n_out;
    const int o0 = (o_tile - a.job[j].tile0) * 64 + wg * 16;  // this wave's first weight row
    const int n0 = n_tile * 2 * NH;
    const int m_valid = min(2 * NH, a.m_rows - n0);
    const int spr = a.spr;
    const uint32_t K = (uint32_t)spr * kQK;
    const uint32_t row_bytes = (uint32_t)spr * F::kBytes;

    const uint64_t wbase = (uint64_t)o0 * row_bytes;
    const uint64_t wbase4 = wbase & ~3ull;
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(wptr + wbase4, rsrc_bytes((uint64_t)n_out * row_bytes, wbase4));
    const uint32_t woff = (uint32_t)(wbase - wbase4) + (uint32_t)r16 * row_bytes;
    const uint64_t a0 = (uint64_t)n0;
    const __amdgpu_buffer_rsrc_t qr = make_rsrc(a.q + a0 * K, rsrc_bytes((uint64_t)a.m_rows * K, a0 * K));
    const __amdgpu_buffer_rsrc_t sr =
        make_rsrc(a.s + a0 * spr, rsrc_bytes((uint64_t)a.m_rows * spr * 4, a0 * spr * 4));
    const int16_t* bsrc = BH ? reinterpret_cast<const int16_t*>(a.bh) : a.b;
    const __amdgpu_buffer_rsrc_t br =
        make_rsrc(bsrc + (kMinF16 ? a0 * spr * 16 : 0),
                  kMinF16 ? rsrc_bytes((uint64_t)a.m_rows * spr * 32, a0 * spr * 32) : 0u);
    // A half slot of the wave's parity: wave (wg, par) moves its 1 KiB chunks 4wg .. 4wg + 3 (lane L: physical 16-byte
    // slot L % 16 of half-row 4c + L / 16, holding logical slot (L % 16) ^ (row % 16)), the scales (wg 0: lane L
    // half-row L) and, for Q4_K, half the bsums (wg < 2: lane L half L % 2 of half-row 32wg + L / 2).
    uint32_t dma_src[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t row = 4u * (uint32_t)(4 * wg + i) + ((uint32_t)lane >> 4);
        dma_src[i] = row * K + 16u * F::src_piece(((uint32_t)lane & 15u) ^ (row & 15u));
    }
    const uint32_t s_src = (uint32_t)lane * (uint32_t)spr * 4u;
    const uint32_t b_src = kMinF16 && wg < 2 ? (32u * wg + ((uint32_t)lane >> 1)) * (uint32_t)spr * 32u + 16u * (lane & 1)
                                             : 0u;
    const uint32_t half_q = (uint32_t)NH * K, half_s = (uint32_t)NH * spr * 4u, half_b = (uint32_t)NH * spr * 32u;
    uint32_t a_off[4];
#pragma unroll
    for (int t = 0; t < 4; t++) a_off[t] = (uint32_t)r16 * 256u + (((uint32_t)(g ^ r16)) ^ (4u * t)) * 16u;
    const int npair = (spr + 1) / 2;

    float out[2 * kSubH][4];
#pragma unroll
    for (int s = 0; s < 2 * kSubH; s++)
#pragma unroll
        for (int i = 0; i < 4; i++) out[s][i] = 0.0f;

    auto body = [&](auto pc) {
        constexpr int P = decltype(pc)::value;  // this wave's parity
        uint8_t* const act[2] = {P ? act10 : act00, P ? act11 : act01};
        float* const act_s[2] = {P ? act_s10 : act_s00, P ? act_s11 : act_s01};
        int16_t* const act_b[2] = {P ? act_b10 : act_b00, P ? act_b11 : act_b01};
        // half h of super-block pair p (super-block 2p + P; none past the row)
        auto stage = [&](int p, auto hc) {
            constexpr int H = decltype(hc)::value;
            const int sb = 2 * p + P;
            if (sb >= spr) return;
#pragma unroll
            for (int i = 0; i < 4; i++)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    qr, (__attribute__((address_space(3))) void*)&act[H][1024 * (4 * wg + i)], 16,
                    (int)(dma_src[i] + (uint32_t)H * half_q + (uint32_t)sb * kQK), 0, 0, 0);
            if (wg == 0)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(sr, (__attribute__((address_space(3))) void*)&act_s[H][0], 4,
                                                         (int)(s_src + (uint32_t)H * half_s + (uint32_t)sb * 4u), 0, 0,
                                                         0);
            if (kMinF16 && wg < 2)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    br, (__attribute__((address_space(3))) void*)&act_b[H][512 * wg], 16,
                    (int)(b_src + (uint32_t)H * half_b + (uint32_t)sb * 32u), 0, 0, 0);
        };
        // half H of this wave's super-block: the even waves add their block values, the odd ones hand them over
        auto half = [&](auto hc, const i32x4 (&op)[4][F::kNumMfma], float d, float dmin, u32x2 mb) {
            constexpr int H = decltype(hc)::value;
            const uint8_t* tile = act[H];
            f32x4(&xch)[4][kSubH * 64] = H ? xch1 : xch0;
#pragma unroll
            for (int s = 0; s < kSubH; s++) {
                i32x4 acc[F::kNumMfma];
#pragma unroll
                for (int k = 0; k < F::kNumMfma; k++) acc[k] = i32x4{0, 0, 0, 0};
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    const u32x4 av = *reinterpret_cast<const u32x4*>(tile + s * 4096 + a_off[t]);
                    const i32x4 aop = i32x4{(int)av.x, (int)av.y, (int)av.z, (int)av.w};
                    acc[0] = mfma16(aop, op[t][0], acc[0]);
                    acc[1] = mfma16(aop, op[t][1], acc[1]);
                }
                const f32x4 q8s = *reinterpret_cast<const f32x4*>(&act_s[H][s * 16 + 4 * g]);
                f32x4 v;
                if constexpr (kMinF16) {
                    f16x4 bq;
                    if constexpr (BH) {
                        bq = *reinterpret_cast<const f16x4*>(&act_b[H][(s * 16 + r16) * 16 + 4 * g]);
                    } else {
                        const s16x4 bi = *reinterpret_cast<const s16x4*>(&act_b[H][(s * 16 + r16) * 16 + 4 * g]);
                        bq = f16x4{(_Float16)bi.x, (_Float16)bi.y, (_Float16)bi.z, (_Float16)bi.w};
                    }
                    const f32x4 mn = __builtin_amdgcn_mfma_f32_16x16x16f16(bq, __builtin_bit_cast(f16x4, mb),
                                                                          f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int main_acc = acc[0][i] + (acc[1][i] << 3);
                        // q8Scale * (d * mainAcc - dmin * minAcc)   (RT/Q4KDotKernel.cs:944)
                        v[i] = q8s[i] * (d * (float)main_acc - dmin * mn[i]);
                    }
                } else {
#pragma unroll
                    for (int i = 0; i < 4; i++) v[i] = F::tail(acc, i, d, dmin, q8s[i]);
                }
                if constexpr (P == 0) {
#pragma unroll
                    for (int i = 0; i < 4; i++) out[H * kSubH + s][i] += v[i];
                    // the tail stays here (not sunk past the barrier with the accumulators live)
                    float(&o4)[4] = out[H * kSubH + s];
                    asm volatile("" : "+v"(o4[0]), "+v"(o4[1]), "+v"(o4[2]), "+v"(o4[3]));
                } else {
                    xch[wg][s * 64 + lane] = v;
                }
            }
        };
        // the even waves: add the odd waves' values of half H (pair p has an odd super-block)
        auto take = [&](auto hc, int p) {
            constexpr int H = decltype(hc)::value;
            if constexpr (P == 0) {
                if (2 * p + 1 < spr) {
                    f32x4(&xch)[4][kSubH * 64] = H ? xch1 : xch0;
#pragma unroll
                    for (int s = 0; s < kSubH; s++) {
                        const f32x4 v = xch[wg][s * 64 + lane];
#pragma unroll
                        for (int i = 0; i < 4; i++) out[H * kSubH + s][i] += v[i];
                    }
                }
            }
        };
        using H0 = std::integral_constant<int, 0>;
        using H1 = std::integral_constant<int, 1>;
        typename F::W w = F::load(wr, woff + (uint32_t)P * F::kBytes, g);
        stage(0, H0{});
        for (int p = 0; p < npair; p++) {
            const bool live = 2 * p + P < spr;  // wave-uniform
            i32x4 op[4][F::kNumMfma];
            F::template operands<0>(w, g, op[0]);
            F::template operands<1>(w, g, op[1]);
            F::template operands<2>(w, g, op[2]);
            F::template operands<3>(w, g, op[3]);
            const float d = F::d_of(w), dmin = F::dmin_of(w);
            const u32x2 mb = F::min_operand(w, g);
            __builtin_amdgcn_s_waitcnt(0);  // this wave's share of the first halves has landed
            __syncthreads();
            stage(p, H1{});
            __builtin_amdgcn_sched_barrier(0);
            w = F::load(wr, woff + (uint32_t)(2 * p + 2 + P) * F::kBytes, g);  // past the row: unused
            if (live) half(H0{}, op, d, dmin, mb);
            __builtin_amdgcn_s_waitcnt(0);  // the second halves and the next weights have landed
            __syncthreads();              // first halves read; the odd first-half values visible
            if (p + 1 < npair) stage(p + 1, H0{});
            take(H0{}, p);
            if (live) half(H1{}, op, d, dmin, mb);
            __syncthreads();  // second halves read; the odd second-half values visible
            take(H1{}, p);
        }
    };
    if (par == 0)
        body(std::integral_constant<int, 0>{});
    else
        body(std::integral_constant<int, 1>{});

    // y[n][o] = biasO + sum   (RT/Q4KDotKernel.cs:951, RT/Q6KDotKernel.cs:507): the even waves hold the sums
    const int o = o0 + r16;
    if (par != 0 || o >= n_out) return;
    const float bias_o = bias ? bias[o] : 0.0f;
#pragma unroll
    for (int s = 0; s < 2 * kSubH; s++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int n = s * 16 + 4 * g + i;
            if (n < m_valid) y[(size_t)(n0 + n) * n_out + o] = bias_o + out[s][i];
        }
}

// ------------------------------------------------------------------------------------------ wide kernel
// The dense kernel above with 128 activation rows per workgroup, staged through LDS in two 64-row halves: each
// wave builds its weight operands once per super-block and uses them for 8 sub-tiles instead of 4, which halves the
// operand build per output, while the two half slots take the LDS of one 64-row double buffer (36.5 KB), so the
// occupancy stays that of the 64-row kernel. Per super-block: the DMA of the second half is issued, the operands are
// built, the next super-block's weights are loaded into the registers the build has just read, the first half is
// computed; a barrier; the DMA of the next super-block's first half is issued into the slot the first half has left,
// and the second half is computed; a barrier. BH: the activation's bsums are fp16 (the quantiser's second bsum
// plane), read as the min MFMA's A operand without conversion.
template <class F, bool BH>
__global__ __launch_bounds__(256, 4) void kquant_mfma_wide_kernel(const MArgs a) {
    constexpr int NH = 64;          // activation rows per half
    constexpr int kSubH = NH / 16;  // sub-tiles per half
    constexpr int kDma = NH / 16;   // 1 KiB DMA chunks per wave per half
    constexpr bool kMinF16 = F::kNumMfma == 3;
    // Each slot is its own LDS object: the compiler gives every LDS object an alias scope, so its wait counts can
    // tell that the DMA into one slot does not write the other one, being read. With one array of two slots it
    // waited for every DMA in flight before each LDS read, so each half's DMA had landed before the other half was
    // computed (gate/up at M = 512 157 -> 153 us, at 1024 rows 302 -> 288 us). The 64-row and pair kernels measured
    // slower with the same change (their Q6_K launches 4-7 %), and keep one array.
    __shared__ __align__(16) uint8_t act0[NH * 256], act1[NH * 256];
    __shared__ __align__(16) float act_s0[NH], act_s1[NH];
    __shared__ __align__(16) int16_t act_b0[kMinF16 ? NH * 16 : 8], act_b1[kMinF16 ? NH * 16 : 8];
    uint8_t* const act[2] = {act0, act1};
    float* const act_s[2] = {act_s0, act_s1};
    int16_t* const act_b[2] = {act_b0, act_b1};

    const int wave = wave_id();
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4, r16 = lane & 15;
    const int b = blockIdx.x;
    const int local = b >> 3;
    const int o_tile = (b & 7) + 8 * (local / a.n_tiles);
    const int n_tile = local % a.n_tiles;
    if (o_tile >= a.o_tiles) return;  // uniform over the workgroup
    int j = 0;
#pragma unroll
    for (int t = 1; t < kMaxJobs; t++)
        if (t < a.njobs && o_tile >= a.job[t].tile0) j = t;
    const uint8_t* wptr = a.job[j].w;
    const float* bias = a.job[j].bias;
    float* y = a.job[j].y;
    const int n_out = a.job[j].n_out;
    const int o0 = (o_tile - a.job[j].tile0) * 64 + wave * 16;  // this wave's first weight row
    const int n0 = n_tile * 2 * NH;
    const int m_valid = min(2 * NH, a.m_rows - n0);
    const int spr = a.spr;
    const uint32_t K = (uint32_t)spr * kQK;
    const uint32_t row_bytes = (uint32_t)spr * F::kBytes;

    const uint64_t wbase = (uint64_t)o0 * row_bytes;
    const uint64_t wbase4 = wbase & ~3ull;
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(wptr + wbase4, rsrc_bytes((uint64_t)n_out * row_bytes, wbase4));
    const uint32_t woff = (uint32_t)(wbase - wbase4) + (uint32_t)r16 * row_bytes;
    // the tile's activation rows n0 .. n0 + 127; rows past M read zeros (resource-clamped)
    const uint64_t a0 = (uint64_t)n0;
    const __amdgpu_buffer_rsrc_t qr = make_rsrc(a.q + a0 * K, rsrc_bytes((uint64_t)a.m_rows * K, a0 * K));
    const __amdgpu_buffer_rsrc_t sr =
        make_rsrc(a.s + a0 * spr, rsrc_bytes((uint64_t)a.m_rows * spr * 4, a0 * spr * 4));
    const int16_t* bsrc = BH ? reinterpret_cast<const int16_t*>(a.bh) : a.b;
    const __amdgpu_buffer_rsrc_t br =
        make_rsrc(bsrc + (kMinF16 ? a0 * spr * 16 : 0),
                  kMinF16 ? rsrc_bytes((uint64_t)a.m_rows * spr * 32, a0 * spr * 32) : 0u);
    // bsums of half-row r (32 bytes): waves w < 2 move rows 32w .. 32w + 31, lane L half L % 2 of row 32w + L / 2
    const uint32_t b_src =
        kMinF16 && wave < NH / 32 ? (32u * wave + ((uint32_t)lane >> 1)) * (uint32_t)spr * 32u + 16u * (lane & 1) : 0u;
    // DMA chunk c = wave * kDma + i covers LDS bytes [1024c, 1024c + 1024) of a half slot: lane L writes physical slot
    // L % 16 of half-row 4c + L / 16, which holds logical slot (L % 16) ^ (row % 16).
    uint32_t dma_src[kDma];
#pragma unroll
    for (int i = 0; i < kDma; i++) {
        const uint32_t row = 4u * (uint32_t)(wave * kDma + i) + ((uint32_t)lane >> 4);
        dma_src[i] = row * K + 16u * F::src_piece(((uint32_t)lane & 15u) ^ (row & 15u));
    }
    const uint32_t s_src = (uint32_t)lane * (uint32_t)spr * 4u;  // wave 0: scale of half-row `lane`
    const uint32_t half_q = (uint32_t)NH * K, half_s = (uint32_t)NH * spr * 4u, half_b = (uint32_t)NH * spr * 32u;
    // Reads past the last super-block of a row land in the next row or past the resource: harmless (not used).
    auto stage = [&](int sb, int h, int buf) {
#pragma unroll
        for (int i = 0; i < kDma; i++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                qr, (__attribute__((address_space(3))) void*)&act[buf][1024 * (wave * kDma + i)], 16,
                (int)(dma_src[i] + (uint32_t)h * half_q + (uint32_t)sb * kQK), 0, 0, 0);
        if (wave == 0)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(sr, (__attribute__((address_space(3))) void*)&act_s[buf][0], 4,
                                                     (int)(s_src + (uint32_t)h * half_s + (uint32_t)sb * 4u), 0, 0, 0);
        if (kMinF16 && wave < NH / 32)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                br, (__attribute__((address_space(3))) void*)&act_b[buf][512 * wave], 16,
                (int)(b_src + (uint32_t)h * half_b + (uint32_t)sb * 32u), 0, 0, 0);
    };
    uint32_t a_off[4];
#pragma unroll
    for (int t = 0; t < 4; t++) a_off[t] = (uint32_t)r16 * 256u + (((uint32_t)(g ^ r16)) ^ (4u * t)) * 16u;

    float out[2 * kSubH][4];
#pragma unroll
    for (int s = 0; s < 2 * kSubH; s++)
#pragma unroll
        for (int i = 0; i < 4; i++) out[s][i] = 0.0f;

    // MFMAs and fp32 tails of one half (sub-tiles 4H .. 4H + 3 of the tile): each sub-tile's MFMAs, then its tail.
    auto mma_tail = [&](auto half, int buf, const i32x4 (&op)[4][F::kNumMfma], float d, float dmin, u32x2 mb) {
        constexpr int H = decltype(half)::value;
        const uint8_t* tile = act[buf];
#pragma unroll
        for (int s = 0; s < kSubH; s++) {
            i32x4 acc[F::kNumMfma];
#pragma unroll
            for (int k = 0; k < F::kNumMfma; k++) acc[k] = i32x4{0, 0, 0, 0};
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const u32x4 av = *reinterpret_cast<const u32x4*>(tile + s * 4096 + a_off[t]);
                const i32x4 aop = i32x4{(int)av.x, (int)av.y, (int)av.z, (int)av.w};
                acc[0] = mfma16(aop, op[t][0], acc[0]);
                acc[1] = mfma16(aop, op[t][1], acc[1]);
            }
            const f32x4 q8s = *reinterpret_cast<const f32x4*>(&act_s[buf][s * 16 + 4 * g]);
            if constexpr (kMinF16) {
                f16x4 bq;
                if constexpr (BH) {
                    bq = *reinterpret_cast<const f16x4*>(&act_b[buf][(s * 16 + r16) * 16 + 4 * g]);
                } else {
                    const s16x4 bi = *reinterpret_cast<const s16x4*>(&act_b[buf][(s * 16 + r16) * 16 + 4 * g]);
                    bq = f16x4{(_Float16)bi.x, (_Float16)bi.y, (_Float16)bi.z, (_Float16)bi.w};
                }
                const f32x4 mn =
                    __builtin_amdgcn_mfma_f32_16x16x16f16(bq, __builtin_bit_cast(f16x4, mb), f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int main_acc = acc[0][i] + (acc[1][i] << 3);
                    // q8Scale * (d * mainAcc - dmin * minAcc)   (RT/Q4KDotKernel.cs:944)
                    out[H * kSubH + s][i] += q8s[i] * (d * (float)main_acc - dmin * mn[i]);
                }
            } else {
#pragma unroll
                for (int i = 0; i < 4; i++) out[H * kSubH + s][i] += F::tail(acc, i, d, dmin, q8s[i]);
            }
            // the tail stays here: left to itself the compiler sinks the first half's tails past the barrier, with
            // every sub-tile's accumulators live across it
            float(&o4)[4] = out[H * kSubH + s];
            asm volatile("" : "+v"(o4[0]), "+v"(o4[1]), "+v"(o4[2]), "+v"(o4[3]));
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    typename F::W w = F::load(wr, woff, g);
    stage(0, 0, 0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    for (int sb = 0; sb < spr; sb++) {
        stage(sb, 1, 1);
        i32x4 op[4][F::kNumMfma];
        F::template operands<0>(w, g, op[0]);
        F::template operands<1>(w, g, op[1]);
        F::template operands<2>(w, g, op[2]);
        F::template operands<3>(w, g, op[3]);
        const float d = F::d_of(w), dmin = F::dmin_of(w);
        const u32x2 mb = F::min_operand(w, g);
        // the next super-block's weights into the registers just read (past the row: unused)
        __builtin_amdgcn_sched_barrier(0);
        w = F::load(wr, woff + (uint32_t)(sb + 1) * F::kBytes, g);
        mma_tail(std::integral_constant<int, 0>{}, 0, op, d, dmin, mb);
        __builtin_amdgcn_s_waitcnt(0);  // the second half and the weights have landed; every wave is past slot 0
        __syncthreads();
        if (sb + 1 < spr) stage(sb + 1, 0, 0);
        mma_tail(std::integral_constant<int, 1>{}, 1, op, d, dmin, mb);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
    }

    // y[n][o] = biasO + sum   (RT/Q4KDotKernel.cs:951, RT/Q6KDotKernel.cs:507)
    const int o = o0 + r16;
    if (o >= n_out) return;
    const float bias_o = bias ? bias[o] : 0.0f;
#pragma unroll
    for (int s = 0; s < 2 * kSubH; s++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int n = s * 16 + 4 * g + i;
            if (n < m_valid) y[(size_t)(n0 + n) * n_out + o] = bias_o + out[s][i];
        }
}

template <class F, int NT>
static hipError_t launch_mfma(MArgs& ma, bool pre, hipStream_t st) {
    ma.n_tiles = (ma.m_rows + NT - 1) / NT;
    const int grid = (ma.o_tiles + 7) / 8 * 8 * ma.n_tiles;
    if constexpr (F::kNumMfma == 2) {  // only Q6_K weights carry the MFMA-ready copy
        if (pre) {
            hipLaunchKernelGGL((kquant_mfma_kernel<F, NT, true, false>), dim3(grid), dim3(256), 0, st, ma);
            return hipGetLastError();
        }
    } else {
        if (ma.bh) {  // Q4_K with the quantiser's fp16 bsums
            hipLaunchKernelGGL((kquant_mfma_kernel<F, NT, false, false, true>), dim3(grid), dim3(256), 0, st, ma);
            return hipGetLastError();
        }
    }
    hipLaunchKernelGGL((kquant_mfma_kernel<F, NT, false, false>), dim3(grid), dim3(256), 0, st, ma);
    return hipGetLastError();
}

hipError_t launch_mfma_grouped(int type, const GroupLaunch& L, const int* tiles, const int* tile_count,
                               int max_tiles, hipStream_t st) {
    MArgs ma{};
    const int o1 = (L.n_rows + 63) / 64;
    ma.o_tiles = o1 * (L.w1 ? 2 : 1);
    ma.n_tiles = max_tiles;
    ma.m_rows = L.rows;
    ma.spr = L.in / kQK;
    ma.q = L.act.q;
    ma.s = L.act.s;
    ma.b = L.act.b;
    if (type == 12 && !ma.b) return hipErrorInvalidValue;  // the Q4_K kernel reads the bsums
    for (int e = 0; e < L.experts; e++) {
        ma.grp.w0[e] = L.w0[e];
        ma.grp.w1[e] = L.w1 ? L.w1[e] : nullptr;
    }
    ma.grp.expert_off = L.expert_off;
    ma.grp.pair_row = L.pair_row;
    ma.grp.tiles = tiles;
    ma.grp.tile_count = tile_count;
    ma.grp.y0 = L.y0;
    ma.grp.y1 = L.y1;
    ma.grp.n_rows = L.n_rows;
    ma.grp.o_tiles1 = o1;
    const int grid = (ma.o_tiles + 7) / 8 * 8 * max_tiles;
    constexpr int NT = kGroupedTileRows;
    if (type == 12)
        hipLaunchKernelGGL((kquant_mfma_kernel<Q4KMfma, NT, false, true>), dim3(grid), dim3(256), 0, st, ma);
    else
        hipLaunchKernelGGL((kquant_mfma_kernel<Q6KMfma, NT, false, true>), dim3(grid), dim3(256), 0, st, ma);
    return hipGetLastError();
}

// 128 activation rows per workgroup halve the operand-build cost per output but allow only two workgroups per CU;
// 64 rows fit four, which hides more latency. Measured on MI355X (Llama-3-8B layer shapes): 64 is faster up to
// M = 512, 128 from M = 2048. The wide kernel (128 rows staged in 64-row halves, the LDS of the 64-row kernel, so
// four workgroups per CU) takes Q4_K launches whose grid has at least 448 workgroups; below that the 64-row kernel's
// twice-larger grid fills the CUs better. Measured (graph replay with the quantise launch, us, 64-row / 128-row /
// wide): gate/up 2x14336x4096 at 256 rows 98.7 / 110 / 93.1 and at 512 rows 181 / 184 / 161; q/k/v at 512 rows
// (384 wide workgroups) 49.2 / 55.7 / 55.4 and at 1024 rows 84.9 / 86.6 / 77.7; o 4096x4096 at 2048 rows 115 / 111 /
// 99.6. For Q6_K the wide kernel is slower (its operand build is not what bounds the launch: 4096x14336 at 1024
// rows 250 / 181 / 228). OVFQ_MFMA_TILE_ROWS=64 / 128 / wide forces one.
constexpr int kWideTile = 1;
constexpr int kPairTile = 2;
constexpr int kPairWideTile = 3;
static int mfma_tile_rows(int type, int rows, int o_tiles) {
    static const int forced = [] {
        const char* e = getenv("OVFQ_MFMA_TILE_ROWS");
        if (e && !strcmp(e, "wide")) return kWideTile;
        if (e && !strcmp(e, "pair")) return kPairTile;
        if (e && !strcmp(e, "pairwide")) return kPairWideTile;
        return e && *e ? atoi(e) : 0;
    }();
    if (forced == 64 || forced == 128 || forced == kWideTile || forced == kPairTile || forced == kPairWideTile)
        return forced;
    if (type == 12 && (long)o_tiles * ((rows + 127) / 128) >= 448) return kWideTile;
    // The pair kernel (two waves per 16 weight rows on alternate super-blocks) where the 64-row grid leaves each CU
    // one or two tiles: Q6_K 4096x14336 at 128 / 256 rows (128 / 256 workgroups) 116 / 118 -> 92 / 93 us, at 512
    // rows (512, issue-bound at two waves per SIMD already) 131 -> 135; Q4_K q/k/v at 256 rows (384) 36.3 -> 34.7,
    // o 4096x4096 at 512 rows (512) 38.7 -> 37.0, but o at 256 rows (256) 27.4 -> 28.1 and q/k/v at 512 rows (768)
    // 49.4 -> 55.3.
    const long grid64 = (long)o_tiles * ((rows + 63) / 64);
    // The pair-wide kernel (one 8-wave workgroup per CU: 64 weight rows x 128 activation rows, each wave's operands
    // built once per 128 rows) for Q6_K where its grid gives about one workgroup per CU: 4096x14336 at 512 rows (256
    // workgroups) 130.7 -> 112.5 us; at 256 rows (128) 98 -> 105 and at 1024 rows (512, two rounds) 179 -> 210.
    const long grid128 = (long)o_tiles * ((rows + 127) / 128);
    if (type == 14 && grid128 >= 192 && grid128 <= 256) return kPairWideTile;
    if (rows < 1024 && (type == 14 ? grid64 <= 256 : grid64 >= 384 && grid64 <= 512)) return kPairTile;
    return rows >= 1024 ? 128 : 64;
}

bool mfma_supported(int type) { return type == 12 || type == 14; }

// The small-M kernel's time grows with every 16 activation rows (it streams the weights once per 16-row tile);
// the tiled kernel's stays flat while its grid (64-row weight tiles x 64-row activation tiles) leaves CUs idle,
// each workgroup walking the whole input dimension. Measured on MI355X (graph replay, weights rotated past the
// cache, Llama-3-8B shapes, us small-M vs tiled): at 16 rows small-M wins everywhere (gate/up pair 34.6 vs 35.7);
// from 17 rows the tiled kernel wins once its grid reaches 96 workgroups (14336x4096 Q4_K at 24 rows 31.2 vs
// 25.9, fused q/k/v 32.8 vs 25.0) and loses below it (4096x4096 Q4_K at 64 rows 20.9 vs 25.4, at 96 rows and 128
// workgroups 29.4 vs 25.5). Q6_K operands cost the tiled kernel more per workgroup: 4096x14336 stays on small-M
// at 96 rows (109 vs 120) and switches at 128 (144 vs 123), i.e. from rows x out_rows >= 448 Ki.
// Whatever the grid, one wave of tiled workgroups costs about as much as 6 (Q4_K) or 7 (Q6_K) small-M passes at the
// same input size, because both walk the whole input: at 256 / 1024 output rows, us small-M vs tiled, Q4_K K = 4096
// at 80 rows 23.9 vs 23.9 and 96 rows 28.2 vs 23.9, K = 14336 at 80 rows 68.2 vs 73.8 and 96 rows 81.2 vs 73.8;
// Q6_K K = 4096 at 96 rows 33.9 vs 34.5 and 112 rows 39.1 vs 34.8, K = 14336 at 96 rows 105.1 vs 111.5 and 112
// rows 122.3 vs 111.0; at 512 rows and 128 output rows 138 vs 24.
bool mfma_tiled_preferred(int type, int rows, int o_tiles, long out_rows) {
    if (rows <= 16) return false;
    if ((rows + 15) / 16 >= (type == 14 ? 7 : 6)) return true;
    if ((long)o_tiles * ((rows + 63) / 64) < 96) return false;
    return type != 14 || (long)rows * out_rows >= 448L * 1024;
}

hipError_t launch_project_mfma(int type, const ProjJob* jobs, int njobs, int in, int rows, ActQ act,
                               hipStream_t st) {
    MArgs ma{};
    int tiles = 0;
    bool pre = true;  // the prepared variant when every weight of the launch has its MFMA-ready copy
    for (int i = 0; i < njobs; i++) {
        ma.job[i] = MJob{jobs[i].w, jobs[i].pre, jobs[i].bias, jobs[i].y, jobs[i].n_rows, tiles};
        tiles += (jobs[i].n_rows + 63) / 64;
        pre = pre && jobs[i].pre != nullptr;
    }
    ma.njobs = njobs;
    ma.o_tiles = tiles;
    ma.m_rows = rows;
    ma.spr = in / kQK;
    ma.q = act.q;
    ma.s = act.s;
    ma.b = act.b;
    ma.bh = type == 12 ? act.bh : nullptr;
    if (type == 12 && !ma.b) return hipErrorInvalidValue;  // the Q4_K kernel reads the bsums
    const int nt = mfma_tile_rows(type, rows, tiles);
    if (nt == kPairWideTile && !pre) {
        ma.n_tiles = (rows + 127) / 128;
        const int grid = (ma.o_tiles + 7) / 8 * 8 * ma.n_tiles;
        if (type == 12 && ma.bh)
            hipLaunchKernelGGL((kquant_mfma_pairwide_kernel<Q4KMfma, true>), dim3(grid), dim3(512), 0, st, ma);
        else if (type == 12)
            hipLaunchKernelGGL((kquant_mfma_pairwide_kernel<Q4KMfma, false>), dim3(grid), dim3(512), 0, st, ma);
        else
            hipLaunchKernelGGL((kquant_mfma_pairwide_kernel<Q6KMfma, false>), dim3(grid), dim3(512), 0, st, ma);
        return hipGetLastError();
    }
    if (nt == kPairTile && !pre) {
        ma.n_tiles = (rows + 63) / 64;
        const int grid = (ma.o_tiles + 7) / 8 * 8 * ma.n_tiles;
        if (type == 12 && ma.bh)
            hipLaunchKernelGGL((kquant_mfma_pair_kernel<Q4KMfma, true>), dim3(grid), dim3(512), 0, st, ma);
        else if (type == 12)
            hipLaunchKernelGGL((kquant_mfma_pair_kernel<Q4KMfma, false>), dim3(grid), dim3(512), 0, st, ma);
        else
            hipLaunchKernelGGL((kquant_mfma_pair_kernel<Q6KMfma, false>), dim3(grid), dim3(512), 0, st, ma);
        return hipGetLastError();
    }
    if (nt == kWideTile && !pre) {
        ma.n_tiles = (rows + 127) / 128;
        const int grid = (ma.o_tiles + 7) / 8 * 8 * ma.n_tiles;
        if (type == 12 && ma.bh)
            hipLaunchKernelGGL((kquant_mfma_wide_kernel<Q4KMfma, true>), dim3(grid), dim3(256), 0, st, ma);
        else if (type == 12)
            hipLaunchKernelGGL((kquant_mfma_wide_kernel<Q4KMfma, false>), dim3(grid), dim3(256), 0, st, ma);
        else
            hipLaunchKernelGGL((kquant_mfma_wide_kernel<Q6KMfma, false>), dim3(grid), dim3(256), 0, st, ma);
        return hipGetLastError();
    }
    if (type == 12)
        return nt == 128 ? launch_mfma<Q4KMfma, 128>(ma, pre, st) : launch_mfma<Q4KMfma, 64>(ma, pre, st);
    return nt == 128 ? launch_mfma<Q6KMfma, 128>(ma, pre, st) : launch_mfma<Q6KMfma, 64>(ma, pre, st);
}

// The 16 x 16 fp32 values of one super-block for the small-M kernel: MFMAs over the four 64-element chunks (A
// operands av[t] already in the weight operands' K order), then the reference's fp32 tail per (row 4g+j, output
// r16); `q8s` is the q8 scale of activation row lane % 16.
template <class F>
__device__ __forceinline__ void lohi_block_values(const typename F::W& w, const u32x4 (&av)[4], int g, float q8s,
                                                  float (&v)[4]) {
    i32x4 op[4][F::kNumMfma];
    F::template operands<0>(w, g, op[0]);
    F::template operands<1>(w, g, op[1]);
    F::template operands<2>(w, g, op[2]);
    F::template operands<3>(w, g, op[3]);
    i32x4 acc[F::kNumMfma];
#pragma unroll
    for (int k = 0; k < F::kNumMfma; k++) acc[k] = i32x4{0, 0, 0, 0};
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const i32x4 aop = i32x4{(int)av[t].x, (int)av[t].y, (int)av[t].z, (int)av[t].w};
#pragma unroll
        for (int k = 0; k < F::kNumMfma; k++) acc[k] = mfma16(aop, op[t][k], acc[k]);
    }
    const float d = F::d_of(w), dmin = F::dmin_of(w);
#pragma unroll
    for (int j = 0; j < 4; j++) v[j] = F::tail(acc, j, d, dmin, __shfl(q8s, 4 * g + j, 64));
}

// ------------------------------------------------------------------------------------------ small M
// Few activation rows (M <= 16 per tile; MoE experts' token groups): one workgroup owns 16 weight rows and its
// four waves split the row's super-blocks (wave w takes w, w+4, ...), so a 4096-row matrix already gives 1024
// waves. Each wave loads the weights of kBatch super-blocks at once, reads its A operands straight from the
// (L2-resident) Q8_K activation in the same K order the big kernel stages in LDS, runs the super-block's MFMAs and
// fp32 tail, and stores the 16 x 16 block values in LDS; then one lane per (output, row) adds the values in
// ascending super-block order (the reference's sequential sum) and writes biasO + sum.
// grid.x = 16-row tiles over one or two matrices (gate/up), grid.y = expert: expert e owns pairs
// [expert_off[e], expert_off[e+1]) of a pair list; pair p reads activation row pair_row[p] and writes output row p
// (without a pair list: one expert over activation rows 0..rows-1).
struct SArgs {
    const uint8_t* w0[kMaxExperts];
    const uint8_t* w1[kMaxExperts];
    const float* bias0;
    const float* bias1;
    float* y0;
    float* y1;
    int n_rows;
    int spr;
    int tiles;  // 16-row tiles of one matrix
    int rows;      // pairs of the single expert when expert_off == NULL
    int act_rows;  // rows of the Q8_K activation (< 2^31 bytes in total)
    const int* expert_off;
    const int* pair_row;
    const int8_t* q;
    const float* s;
    float* comb;            // if set: add comb_w[pair] * value to comb[comb_tok[pair]] (GroupLaunch)
    const int* comb_tok;
    const float* comb_w;
};

template <class F, int kBatch, bool kPipe>
__global__ __launch_bounds__(256) void kquant_mfma_small_kernel(const SArgs a) {
    extern __shared__ __align__(16) float vals[];  // [spr][16 rows n][16 outputs o]
    const int wave = wave_id();
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4, r16 = lane & 15;
    const int e = blockIdx.y;
    const int pbeg = a.expert_off ? a.expert_off[e] : 0;
    const int cnt = a.expert_off ? a.expert_off[e + 1] - pbeg : a.rows;
    if (cnt <= 0) return;  // uniform over the workgroup
    const int mat = (int)blockIdx.x >= a.tiles ? 1 : 0;
    const int o0 = ((int)blockIdx.x - mat * a.tiles) * 16;
    const uint8_t* wptr = mat ? a.w1[e] : a.w0[e];
    const int spr = a.spr;
    const uint32_t K = (uint32_t)spr * kQK;
    const uint32_t row_bytes = (uint32_t)spr * F::kBytes;
    const uint64_t wbase = (uint64_t)o0 * row_bytes;
    const uint64_t wbase4 = wbase & ~3ull;
    const __amdgpu_buffer_rsrc_t wr =
        make_rsrc(wptr + wbase4, rsrc_bytes((uint64_t)a.n_rows * row_bytes, wbase4));
    const uint32_t woff = (uint32_t)(wbase - wbase4) + (uint32_t)r16 * row_bytes;
    uint32_t a_off[4];  // byte offset inside a super-block of this lane's 16 A-operand bytes for MFMA t
#pragma unroll
    for (int t = 0; t < 4; t++) a_off[t] = 16u * F::src_piece(4u * t + (uint32_t)g);

    // One wave-uniform resource over all activation rows (a per-lane resource would be re-made uniform by a
    // readfirstlane loop around every load); the lane's row goes into the 32-bit offset.
    const __amdgpu_buffer_rsrc_t qr = make_rsrc(a.q, (uint32_t)a.act_rows * K);
    const __amdgpu_buffer_rsrc_t sr = make_rsrc(a.s, (uint32_t)a.act_rows * (uint32_t)spr * 4u);
    for (int n0 = 0; n0 < cnt; n0 += 16) {
        // A operand row r16 of this tile: pair pbeg + n0 + r16; an absent row reads past the resource (zeros)
        const bool have = n0 + r16 < cnt;
        const int p = pbeg + n0 + r16;
        const int arow = have ? (a.pair_row ? a.pair_row[p] : p) : 0;
        const uint32_t qbase = have ? (uint32_t)arow * K : 0x80000000u;
        const uint32_t sbase = have ? (uint32_t)arow * (uint32_t)spr * 4u : 0x80000000u;
        // Batches of kBatch super-blocks (wave w: w, w + 4, ...). With kPipe (long rows) the batches are
        // double-buffered: the next batch's weights and A operands are issued before the current batch is computed
        // (twice the registers, so fewer waves: it pays from about four batches per wave). Loads past the row are
        // harmless (resource-clamped or unused) and keep the instruction stream fixed; a slot past the row only
        // skips its store.
        struct Batch {
            typename F::W w[kBatch];
            u32x4 av[kBatch][4];
            uint32_t sv[kBatch];
        };
        auto load_batch = [&](int sb0, Batch& bt) {
#pragma unroll
            for (int i = 0; i < kBatch; i++) {
                const int sb = sb0 + 4 * i;
                bt.w[i] = F::load(wr, woff + (uint32_t)sb * F::kBytes, g);
#pragma unroll
                for (int t = 0; t < 4; t++) bt.av[i][t] = ld4(qr, qbase + (uint32_t)sb * kQK + a_off[t]);
                bt.sv[i] = ld1(sr, sbase + (uint32_t)sb * 4);
            }
        };
        auto compute_batch = [&](int sb0, const Batch& cur) {
#pragma unroll
            for (int i = 0; i < kBatch; i++) {
                const int sb = sb0 + 4 * i;
                float v[4];
                lohi_block_values<F>(cur.w[i], cur.av[i], g, as_float(cur.sv[i]), v);  // sv: q8 scale of row r16
                if (sb < spr) {
                    float* vrow = vals + sb * 256;
#pragma unroll
                    for (int j = 0; j < 4; j++) vrow[(4 * g + j) * 16 + r16] = v[j];
                }
            }
        };
        if constexpr (kPipe) {
            int sb0 = wave;
            auto step = [&](const Batch& cur, Batch& nxt) -> bool {
                load_batch(sb0 + 4 * kBatch, nxt);
                compute_batch(sb0, cur);
                sb0 += 4 * kBatch;
                return sb0 < spr;
            };
            Batch ba, bb;
            load_batch(sb0, ba);
            if (sb0 < spr) {
                while (step(ba, bb) && step(bb, ba)) {
                }
            }
        } else {
            for (int sb0 = wave; sb0 < spr; sb0 += 4 * kBatch) {
                Batch bt;
                load_batch(sb0, bt);
                compute_batch(sb0, bt);
            }
        }
        __syncthreads();
        // one lane per (row n, output o): ascending super-block sum, then biasO + sum
        {
            const int n = threadIdx.x >> 4, o = threadIdx.x & 15;
            float sum = 0.0f;
            for (int sb = 0; sb < spr; sb++) sum += vals[sb * 256 + threadIdx.x];
            if (n0 + n < cnt && o0 + o < a.n_rows) {
                const float* bias = mat ? a.bias1 : a.bias0;
                const float v = bias ? bias[o0 + o] + sum : sum;
                const int p = pbeg + n0 + n;
                if (a.comb) {
                    const float prod = a.comb_w[p] * v;
                    __hip_atomic_fetch_add(a.comb + (size_t)a.comb_tok[p] * a.n_rows + o0 + o, prod, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
                } else {
                    float* y = mat ? a.y1 : a.y0;
                    y[(size_t)p * a.n_rows + o0 + o] = v;
                }
            }
        }
        __syncthreads();  // the next row tile overwrites vals
    }
}

// ------------------------------------------------------------------------------------------ expert stream
// Grouped (MoE) Q4_K / Q6_K projections with few pairs per expert, on a persistent grid. A unit of work is (expert e,
// matrix, 64-row weight group, 16-pair chunk) and belongs to one workgroup: workgroup b takes units b, b + (workgroups
// in the launch), ... (experts without pairs skipped) and walks each unit's super-blocks in ascending order, one per
// step, its four waves in step (wave w owns weight rows 16w .. 16w + 15 of the group). Per step each wave brings its
// 16 weight rows' super-block (Q4_K: 16 x 144 bytes; Q6_K: 16 aligned 224-byte windows holding the 210-byte blocks)
// into its own LDS ring slot by DMA, and a quarter of the chunk's A operands (4 pairs
// x 256 activation bytes) and scales into the workgroup's shared slot, so the four waves read the activation once
// between them; all of it is issued two steps ahead of use and crosses unit boundaries. The step runs the
// super-block's MFMAs (Q4_K on raw nibbles, Q4KRaw; Q6_K on the lo/hi operands of Q6KMfma) and the reference's fp32
// tail for the results that hold pairs, and adds
// each block value to the lane's running sums: lane
// (g, r16) owns outputs (MFMA rows 4g + j, weight row r16), so its sum is the reference's sequential sum over the
// row, with no exchange between waves. The unit's last step stores biasO + sum.
constexpr int kStreamA = 4096;         // the chunk's A operands per step: 16 pairs x 256 bytes, 1 KiB DMA per wave
constexpr int kStreamS = 64;           // the chunk's activation scales: 4 per wave
constexpr int kStreamMaxPairs = 1024;  // the pair -> activation row map is cached in LDS (dynamic, 4 bytes a pair)
constexpr int kStreamRows = 64;        // weight rows per unit (16 per wave)

// Calls f(slot 0), f(slot 1), ..., f(slot n - 1), f(slot 0), ... with each slot a compile-time constant, until one
// call returns false.
template <typename Fn, int... I>
__device__ __forceinline__ void run_slots(Fn& f, std::integer_sequence<int, I...>) {
    while ((f(std::integral_constant<int, I>{}) && ...)) {
    }
}

// A Q4_K super-block of the expert-stream kernel on raw nibbles. Per sub-block s (32 elements) one
// v_mfma_i32_16x16x32_i8 of the activation bytes and the weight nibbles gives acc_s = sum nib * q8; the 6-bit scales
// are applied to the results that hold pairs, mainAcc = sum_s sc_s * acc_s (24-bit multiply-adds, exact: |acc_s| <=
// 32 * 15 * 127). minAcc = sum_s m_s * (sum of the sub-block's q8) comes from four v_mfma_i32_16x16x64_i8 over the
// sub-block pairs (s, s + 4): the A operand is the two sub-blocks' activation bytes side by side, as read from LDS,
// and the B operand m_s in the first eight bytes of each lane group, m_{s+4} in the last eight. These are the
// integers of Q4KMfma's split-scale form (fewer operand instructions, one fewer MFMA), so the fp32 tail gives the same
// block value. Lane (g, r16) holds: h = the block's d, dmin and 12 scale bytes; q01 / q23 = qs[32 c + 8 g .. + 7]
// for c = 0, 1 / 2, 3 (low nibbles: sub-block 2c, high: 2c + 1; qs byte b holds elements 64 (b / 32) + b % 32 and
// +32); av[t] = its pair's activation bytes 32 s + 8 g .. + 7 of sub-blocks s = t and t + 4; q8s[j] = the q8 scale of
// result j's pair. Both operands of every MFMA hold the same element in the same byte.
struct Q4KRaw {
    __device__ __forceinline__ static i32x4 mfma32(uint32_t a0, uint32_t a1, uint32_t b0, uint32_t b1) {
        const long av = (long)(((uint64_t)a1 << 32) | a0), bv = (long)(((uint64_t)b1 << 32) | b0);
        return __builtin_amdgcn_mfma_i32_16x16x32_i8(av, bv, i32x4{0, 0, 0, 0}, 0, 0, 0);
    }
    __device__ __forceinline__ static void accumulate(const u32x4& h, const u32x4& q01, const u32x4& q23,
                                                      const u32x4 (&av)[4], const f32x4& q8s, int live,
                                                      float (&run)[4]) {
        const uint32_t qw[8] = {q01.x, q01.y, q01.z, q01.w, q23.x, q23.y, q23.z, q23.w};
        i32x4 acc[8];
#pragma unroll
        for (int s = 0; s < 8; s++) {
            const int c = s >> 1, sh = 4 * (s & 1);
            const uint32_t b0 = (qw[2 * c] >> sh) & 0x0f0f0f0fu, b1 = (qw[2 * c + 1] >> sh) & 0x0f0f0f0fu;
            acc[s] = s < 4 ? mfma32(av[s & 3].x, av[s & 3].y, b0, b1) : mfma32(av[s & 3].z, av[s & 3].w, b0, b1);
        }
        // the eight 6-bit scales and mins, one byte each (LD/GgmlDequant.cs:64-79 unpacking)
        const uint32_t sc_lo = h.y & 0x3f3f3f3fu, m_lo = h.z & 0x3f3f3f3fu;
        const uint32_t sc_hi = (h.w & 0x0f0f0f0fu) | ((h.y >> 2) & 0x30303030u);
        const uint32_t m_hi = ((h.w >> 4) & 0x0f0f0f0fu) | ((h.z >> 2) & 0x30303030u);
        i32x4 mn = i32x4{0, 0, 0, 0};
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const int ml = (int)__builtin_amdgcn_perm(0u, m_lo, 0x01010101u * t);  // m_t in all four bytes
            const int mh = (int)__builtin_amdgcn_perm(0u, m_hi, 0x01010101u * t);  // m_{t+4}
            mn = mfma16(i32x4{(int)av[t].x, (int)av[t].y, (int)av[t].z, (int)av[t].w}, i32x4{ml, ml, mh, mh}, mn);
        }
        int sc[8];
#pragma unroll
        for (int s = 0; s < 8; s++) sc[s] = (int)(((s < 4 ? sc_lo : sc_hi) >> (8 * (s & 3))) & 0xffu);
        const float d = half_lo(h.x), dmin = half_hi(h.x);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            if (j < live) {
                int main_acc = __mul24(sc[0], acc[0][j]);
#pragma unroll
                for (int s = 1; s < 8; s++) main_acc += __mul24(sc[s], acc[s][j]);
                // q8Scale * (d * mainAcc - dmin * minAcc)   (RT/Q4KDotKernel.cs:944)
                run[j] += q8s[j] * (d * (float)main_acc - dmin * (float)mn[j]);
            }
        }
    }
};

// The format side of the expert-stream kernel: a wave's weight DMA per step (pieces of 16 bytes: kPieces per weight
// row, kRowLds bytes a row in the LDS slot, kWInstr DMA instructions of which the last moves kLastLanes pieces), the
// swizzle of the shared A slot, and the step's compute from the LDS rings.
// Q4_K: 144-byte blocks, row starts 16-byte aligned, so a row's block is 9 pieces at super-block offset 144 sb.
struct StreamQ4K {
    static constexpr int kPieces = 9;
    static constexpr int kRowLds = 144;
    static constexpr int kWInstr = 3;
    static constexpr int kLastLanes = 16;
    // scalar offset of super-block sb's pieces in a row
    __device__ __forceinline__ static uint32_t soff(int sb) { return (uint32_t)sb * kQ4KBytes; }
    // The MFMA row m of a pair holds its 16-byte pieces XORed with m % 8: rows m and m + 8 then share banks (a two-way
    // conflict on the reads), but logical pieces i and i + 8 stay 128 bytes apart in every row, so one ds_read2_b64
    // fetches a sub-block pair (s, s + 4).
    __device__ __forceinline__ static uint32_t a_swizzle(uint32_t m) { return m & 7u; }
    // Lane (g, r16) takes activation bytes 32 s + 8 g .. + 7 of sub-block s = 0..7 of its pair (MFMA row r16): half
    // g % 2 of logical piece 2 s + g / 2, and for sub-block s + 4 the same half 128 bytes further.
    __device__ __forceinline__ static void a_reads(uint32_t row, int g, int r16, uint32_t (&a_rd)[4]) {
#pragma unroll
        for (int t = 0; t < 4; t++)
            a_rd[t] = row + 16u * ((2u * t + ((uint32_t)g >> 1)) ^ ((uint32_t)r16 & 7u)) + 8u * ((uint32_t)g & 1u);
    }
    // wrow: the LDS address of this lane's weight row in the step's slot; abase + a_rd: its A operand pieces; sadr:
    // its four results' scales. Reads and waits are explicit (see the kernel). Every output is early-clobber: a read's
    // data may land while later reads of the block still use their address registers.
    __device__ __forceinline__ static void step(uint32_t wrow, uint32_t abase, const uint32_t (&a_rd)[4], uint32_t sadr,
                                                int, int g, int live, float (&run)[4]) {
        u32x4 h, q01, q23, av[4];
        f32x4 q8s;
        asm volatile("ds_read_b128 %0, %8\n\t"
                     "ds_read2_b64 %1, %9 offset1:4\n\t"
                     "ds_read2_b64 %2, %9 offset0:8 offset1:12\n\t"
                     "ds_read2_b64 %3, %10 offset1:16\n\t"
                     "ds_read2_b64 %4, %11 offset1:16\n\t"
                     "ds_read2_b64 %5, %12 offset1:16\n\t"
                     "ds_read2_b64 %6, %13 offset1:16\n\t"
                     "ds_read_b128 %7, %14\n\t"
                     "s_waitcnt lgkmcnt(0)"
                     : "=&v"(h), "=&v"(q01), "=&v"(q23), "=&v"(av[0]), "=&v"(av[1]), "=&v"(av[2]), "=&v"(av[3]),
                       "=&v"(q8s)
                     : "v"(wrow), "v"(wrow + 16u + 8u * (uint32_t)g), "v"(abase + a_rd[0]), "v"(abase + a_rd[1]),
                       "v"(abase + a_rd[2]), "v"(abase + a_rd[3]), "v"(sadr)
                     : "memory");
        Q4KRaw::accumulate(h, q01, q23, av, q8s, live, run);
    }
};

// Q6_K: 210-byte blocks, 2-byte aligned inside a row. With rows 16-byte aligned (super-blocks per row a multiple of 8),
// super-block sb starts 2 (sb % 8) bytes past a 16-byte boundary in every row, so each row's block is DMA'd as the
// 14 aligned pieces (224 bytes) from that boundary, and read back from LDS as aligned dwords shifted by 0 or 2 bytes
// (v_alignbyte_b32). The block then runs as in the other batched kernels: Q6KMfma's lo/hi operands, two
// v_mfma_i32_16x16x64_i8 per 64-element chunk, the tail d * q8Scale * mainAcc.
struct StreamQ6K {
    static constexpr int kPieces = 14;
    static constexpr int kRowLds = 224;
    static constexpr int kWInstr = 4;
    static constexpr int kLastLanes = 32;  // 16 x 14 = 224 pieces = 3 x 64 + 32
    __device__ __forceinline__ static uint32_t soff(int sb) { return (uint32_t)sb * kQ6KBytes - 2u * (uint32_t)(sb & 7); }
    // 16-byte reads of one logical piece by the 16 rows of a lane group: XOR with the whole row index, conflict-free.
    __device__ __forceinline__ static uint32_t a_swizzle(uint32_t m) { return m & 15u; }
    // Chunk P of lane group g covers elements 128 (g / 2) + 32 P + 16 (g % 2) .. + 15 (Q6KMfma's K order): logical
    // piece 8 (g / 2) + 2 P + g % 2.
    __device__ __forceinline__ static void a_reads(uint32_t row, int g, int r16, uint32_t (&a_rd)[4]) {
#pragma unroll
        for (int t = 0; t < 4; t++)
            a_rd[t] = row + 16u * ((8u * ((uint32_t)g >> 1) + 2u * t + ((uint32_t)g & 1u)) ^ ((uint32_t)r16 & 15u));
    }
    __device__ __forceinline__ static void step(uint32_t wrow, uint32_t abase, const uint32_t (&a_rd)[4], uint32_t sadr,
                                                int sb, int g, int live, float (&run)[4]) {
        // The block starts at wrow + mis; every run the lane reads starts a multiple of 4 bytes after it.
        const uint32_t mis = 2u * (uint32_t)(sb & 7), sh = mis & 2u;
        const uint32_t hh = (uint32_t)g >> 1, l0 = 16u * ((uint32_t)g & 1u);
        const uint32_t blk = wrow + (mis & ~3u);
        const uint32_t oa = blk + 64u * hh + l0;          // ql[64h + l0 .. +16], then ql[64h + 32 + l0 ..] at + 32
        const uint32_t oh = blk + 128u + 32u * hh + l0;   // qh[32h + l0 .. +16]
        const uint32_t os = blk + 192u + 8u * hh;         // sc[8h .. 8h + 8]
        u32x2 a01, a23, b01, b23, h01, h23, s01;
        uint32_t a4, b4, h4, s2, dw;
        u32x4 av[4];
        f32x4 q8s;
        asm volatile("ds_read2_b32 %0, %17 offset1:1\n\t"
                     "ds_read2_b32 %1, %17 offset0:2 offset1:3\n\t"
                     "ds_read_b32 %2, %17 offset:16\n\t"
                     "ds_read2_b32 %3, %17 offset0:8 offset1:9\n\t"
                     "ds_read2_b32 %4, %17 offset0:10 offset1:11\n\t"
                     "ds_read_b32 %5, %17 offset:48\n\t"
                     "ds_read2_b32 %6, %18 offset1:1\n\t"
                     "ds_read2_b32 %7, %18 offset0:2 offset1:3\n\t"
                     "ds_read_b32 %8, %18 offset:16\n\t"
                     "ds_read2_b32 %9, %19 offset1:1\n\t"
                     "ds_read_b32 %10, %19 offset:8\n\t"
                     "ds_read_b32 %11, %20 offset:208\n\t"
                     "ds_read_b128 %12, %21\n\t"
                     "ds_read_b128 %13, %22\n\t"
                     "ds_read_b128 %14, %23\n\t"
                     "ds_read_b128 %15, %24\n\t"
                     "ds_read_b128 %16, %25\n\t"
                     "s_waitcnt lgkmcnt(0)"
                     : "=&v"(a01), "=&v"(a23), "=&v"(a4), "=&v"(b01), "=&v"(b23), "=&v"(b4), "=&v"(h01), "=&v"(h23),
                       "=&v"(h4), "=&v"(s01), "=&v"(s2), "=&v"(dw), "=&v"(av[0]), "=&v"(av[1]), "=&v"(av[2]),
                       "=&v"(av[3]), "=&v"(q8s)
                     : "v"(oa), "v"(oh), "v"(os), "v"(blk), "v"(abase + a_rd[0]), "v"(abase + a_rd[1]),
                       "v"(abase + a_rd[2]), "v"(abase + a_rd[3]), "v"(sadr)
                     : "memory");
        Q6KMfma::W w;
        const uint32_t ra[5] = {a01.x, a01.y, a23.x, a23.y, a4}, rb[5] = {b01.x, b01.y, b23.x, b23.y, b4};
        const uint32_t rh[5] = {h01.x, h01.y, h23.x, h23.y, h4};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            w.ql[0][i] = __builtin_amdgcn_alignbyte(ra[i + 1], ra[i], sh);
            w.ql[1][i] = __builtin_amdgcn_alignbyte(rb[i + 1], rb[i], sh);
            w.qh[i] = __builtin_amdgcn_alignbyte(rh[i + 1], rh[i], sh);
        }
        const uint32_t sc0 = __builtin_amdgcn_alignbyte(s01.y, s01.x, sh), sc1 = __builtin_amdgcn_alignbyte(s2, s01.y, sh);
        w.sc = __builtin_amdgcn_perm(sc1, sc0, (g & 1) ? 0x07050301u : 0x06040200u);
        w.d = (dw >> (8u * sh)) & 0xffffu;  // d at block byte 208
        i32x4 op[4][Q6KMfma::kNumMfma];
        Q6KMfma::operands<0>(w, g, op[0]);
        Q6KMfma::operands<1>(w, g, op[1]);
        Q6KMfma::operands<2>(w, g, op[2]);
        Q6KMfma::operands<3>(w, g, op[3]);
        i32x4 acc[Q6KMfma::kNumMfma] = {i32x4{0, 0, 0, 0}, i32x4{0, 0, 0, 0}};
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const i32x4 aop = i32x4{(int)av[t].x, (int)av[t].y, (int)av[t].z, (int)av[t].w};
            acc[0] = mfma16(aop, op[t][0], acc[0]);
            acc[1] = mfma16(aop, op[t][1], acc[1]);
        }
        const float d = Q6KMfma::d_of(w);
#pragma unroll
        for (int j = 0; j < 4; j++)
            if (j < live) run[j] += Q6KMfma::tail(acc, j, d, 0.0f, q8s[j]);
    }
};

// D = ring slots: steps q + 1 .. q + D - 1 are in flight while step q is computed.
template <class FS, int D>
__global__ __launch_bounds__(256) void mfma_stream_kernel(const SArgs a, int n_experts, int nmat, int pairs) {
    constexpr int kWait = (FS::kWInstr + 2) * (D - 2) + FS::kWInstr;
    static_assert(D >= 3 && kWait <= 63, "the wait count below must fit the 6-bit vmcnt field");
    constexpr int kSlot = 16 * FS::kRowLds;  // a wave's weights per step
    // The rings are read with explicit LDS instructions after explicit waits (below), so one array serves each.
    __shared__ __align__(16) uint8_t wring[D][4][kSlot];
    __shared__ __align__(16) uint8_t aring[D][kStreamA];
    __shared__ __align__(16) uint8_t sring[D][kStreamS];
    __shared__ int eoff[kMaxExperts + 1];
    extern __shared__ int prow[];  // pairs entries; with comb, then the pairs' tokens and combine weights
    int* ctok = prow + pairs;
    float* cw = reinterpret_cast<float*>(prow + 2 * pairs);
    const int tid = threadIdx.x, wave = wave_id(), lane = tid & 63;
    const int g = lane >> 4, r16 = lane & 15;
    // without a pair list: one expert over activation rows 0 .. rows - 1 (a dense small batch)
    for (int i = tid; i <= n_experts; i += 256) eoff[i] = a.expert_off ? a.expert_off[i] : (i == 0 ? 0 : a.rows);
    for (int i = tid; i < pairs; i += 256) prow[i] = a.pair_row ? a.pair_row[i] : i;
    if (a.comb)
        for (int i = tid; i < pairs; i += 256) {
            ctok[i] = a.comb_tok[i];
            cw[i] = a.comb_w[i];
        }
    __syncthreads();

    const int spr = a.spr;
    const int groups = a.tiles, per_e = groups * nmat, T = n_experts * per_e;
    const int NG = (int)gridDim.x;  // workgroups in the launch
    const uint32_t K = (uint32_t)spr * kQK;
    const uint32_t row_bytes = (uint32_t)spr * (uint32_t)(FS::kRowLds == 144 ? kQ4KBytes : kQ6KBytes);

    // The schedule: step (unit t, pair chunk n0, super-block sb), the same in every wave of the workgroup. A lead
    // cursor walks it once; each step's fields are kept in a descriptor from the issue of its loads until it is
    // computed.
    struct Step {
        int t, n0, sb;  // t >= T: past the end
        int pbeg, cnt;  // the unit's expert: first pair and pair count
        int mat, o0;    // matrix (gate / up) and the wave's first weight row
    };
    // eoff is the same for every lane; reading it through readfirstlane lets the compiler keep every schedule field
    // in scalar registers (a value it must assume per-lane would turn each buffer access into a waterfall loop).
    // The read is an explicit instruction: the compiler's own LDS read would first wait for the ring's DMAs in
    // flight (it cannot tell that they write other LDS), draining the pipeline at every unit change.
    auto eoff_u = [&](int i) {
        const uint32_t addr = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) int*)(eoff + i);
        int v;
        asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(addr) : "memory");
        return __builtin_amdgcn_readfirstlane(v);
    };
    // Weight DMA pieces of a step (16 rows x kPieces pieces of 16 bytes): instruction i moves pieces 64 i + lane (the
    // last one on its first kLastLanes lanes only). The super-block's offset in the row goes in the scalar offset.
    uint32_t lane_off[FS::kWInstr];
#pragma unroll
    for (int i = 0; i < FS::kWInstr; i++) {
        const uint32_t p = 64u * i + (uint32_t)(i == FS::kWInstr - 1 ? (lane & (FS::kLastLanes - 1)) : lane);
        lane_off[i] = (p / (uint32_t)FS::kPieces) * row_bytes + 16u * (p % (uint32_t)FS::kPieces);
    }
    // Shared A slot: pair p of the chunk (p < 16) at 1024 (p / 4) + 256 (p % 4), written by wave p / 4. The MFMA row
    // of pair p is m(p) = 4 (p % 4) + p / 4 (pair p sits in MFMA row m(p)), and its 16-byte pieces are stored XORed
    // with FS::a_swizzle(m(p)). Wave w's A DMA: lane L moves pair 4w + L / 16 (MFMA row 4 (L / 16) + w), physical
    // piece L % 16 = logical piece (L % 16) ^ a_swizzle(that row).
    const int a_pair = 4 * wave + (lane >> 4);                       // the pair this lane's A DMA moves
    const uint32_t a_piece = (uint32_t)(lane & 15) ^ FS::a_swizzle((uint32_t)(4 * (lane >> 4) + wave));
    const int s_pair = 4 * (lane & 3) + wave;                        // lanes 0-3: the pair of this lane's scale DMA
    const __amdgpu_buffer_rsrc_t qr = make_rsrc(a.q, (uint32_t)a.act_rows * K);
    const __amdgpu_buffer_rsrc_t sr = make_rsrc(a.s, (uint32_t)a.act_rows * (uint32_t)spr * 4u);
    constexpr uint32_t kOut = 0x80000000u;  // an offset past every resource (the DMA then writes zeros)

    // What the lead step's loads need, set when the lead enters a unit or a chunk (not per step): this wave's weight
    // resource, and the lane's A and scale offsets at super-block 0.
    __amdgpu_buffer_rsrc_t lead_w = make_rsrc(a.q, 0u);
    uint32_t lead_q = kOut, lead_s = kOut;
    auto prow_at = [&](int i) {  // an explicit read, like eoff_u's
        const uint32_t addr = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) int*)(prow + i);
        int v;
        asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(addr) : "memory");
        return (uint32_t)v;
    };
    auto enter_chunk = [&](const Step& c) {
        lead_q = c.n0 + a_pair < c.cnt ? prow_at(c.pbeg + c.n0 + a_pair) * K + 16u * a_piece : kOut;
        lead_s = lane < 4 && c.n0 + s_pair < c.cnt ? prow_at(c.pbeg + c.n0 + s_pair) * (uint32_t)spr * 4u : kOut;
    };
    auto enter = [&](Step& c) {
        const int e = c.t / per_e;
        const int r = c.t - e * per_e;
        c.mat = r >= groups ? 1 : 0;
        c.o0 = (r - c.mat * groups) * kStreamRows + 16 * wave;
        c.pbeg = eoff_u(e);
        c.cnt = eoff_u(e + 1) - c.pbeg;
        const uint64_t base = (uint64_t)c.o0 * row_bytes;
        // the descriptor from values marked uniform (else the compiler wraps each DMA in a waterfall loop)
        const uint64_t wpi = (uint64_t)(uintptr_t)((c.mat ? a.w1[e] : a.w0[e]) + base);
        const uint64_t wpu = ((uint64_t)__builtin_amdgcn_readfirstlane((uint32_t)(wpi >> 32)) << 32) |
                             (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)wpi);
        const uint32_t nb = __builtin_amdgcn_readfirstlane(rsrc_bytes((uint64_t)a.n_rows * row_bytes, base));
        lead_w = make_rsrc(reinterpret_cast<const void*>((uintptr_t)wpu), nb);
        enter_chunk(c);
    };
    auto seek = [&](Step& c, int t) {  // the first unit from t on (stride NG) whose expert has pairs
        for (; t < T; t += NG) {
            const int e = t / per_e;
            if (eoff_u(e + 1) > eoff_u(e)) break;
        }
        c.t = t;
        c.n0 = 0;
        c.sb = 0;
        if (t < T) {
            enter(c);
        } else {  // past the end: the loads still issue (a fixed count keeps the waits below exact) and write zeros
            lead_w = make_rsrc(a.q, 0u);
            lead_q = lead_s = kOut;
        }
    };
    auto advance = [&](Step& c) {
        if (c.t >= T) return;
        if (++c.sb < spr) return;
        c.sb = 0;
        c.n0 += 16;
        if (c.n0 < c.cnt) {
            enter_chunk(c);
            return;
        }
        seek(c, c.t + NG);
    };

    // The lead step's weights go to this wave's ring slot j, its A operands and scales to the shared slot j.
    auto issue_w = [&](const Step& c, int j) {
        const int soff = (int)FS::soff(c.sb);
        uint8_t* sl = wring[j][wave];
#pragma unroll
        for (int i = 0; i < FS::kWInstr - 1; i++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(lead_w, (__attribute__((address_space(3))) void*)(sl + 1024 * i),
                                                     16, (int)lane_off[i], soff, 0, 0);
        // the last instruction on its first kLastLanes lanes only (the DMA writes only active lanes)
        if (lane < FS::kLastLanes)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                lead_w, (__attribute__((address_space(3))) void*)(sl + 1024 * (FS::kWInstr - 1)), 16,
                (int)lane_off[FS::kWInstr - 1], soff, 0, 0);
    };
    auto issue_a = [&](const Step& c, int j) {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(qr, (__attribute__((address_space(3))) void*)(aring[j] + 1024 * wave),
                                                 16, (int)(lead_q + (uint32_t)c.sb * kQK), 0, 0, 0);
        // lanes 0-3 only: the DMA writes only active lanes, so four scales per wave fill 16 bytes
        if (lane < 4)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(sr, (__attribute__((address_space(3))) void*)(sring[j] + 16 * wave),
                                                     4, (int)(lead_s + (uint32_t)c.sb * 4u), 0, 0, 0);
    };
    // Read side: lane (g, r16) reads pair p with m(p) = r16, i.e. p = 4 (r16 % 4) + r16 / 4, held at
    // 1024 (r16 % 4) + 256 (r16 / 4).
    uint32_t a_rd[4];
    FS::a_reads(1024u * (uint32_t)(r16 & 3) + 256u * (uint32_t)(r16 >> 2), g, r16, a_rd);

    Step lead;  // the next step whose loads go out
    seek(lead, (int)blockIdx.x);
    if (lead.t >= T) {
        // no unit for this workgroup (the same in all its waves)
        return;
    }
    // Issue order: a step's weights, then its A operands and scales; the first D - 1 steps are issued here. Step q
    // issues the weights of step q + D - 1 into this wave's slot that step q - 1 read, then (after its barrier, when
    // every wave is past step q - 1) the A operands and scales of step q + D - 1 into the shared slot step q - 1
    // read.
    Step desc[D];
#pragma unroll
    for (int i = 0; i < D; i++) desc[i] = lead;  // defined from the start (undefined descriptors cost the compiler a wait)
#pragma unroll
    for (int i = 0; i < D - 1; i++) {
        desc[i] = lead;
        issue_w(lead, i);
        issue_a(lead, i);
        advance(lead);
    }

    float run[4] = {0.0f, 0.0f, 0.0f, 0.0f};  // sums of outputs (MFMA row 4g + j, weight row r16) so far
    auto step = [&](auto sc) -> bool {
        constexpr int s = decltype(sc)::value;  // this step's slot
        constexpr int w = (s + D - 1) % D;      // the slot of the step issued now (read by the last step)
        const Step& cur = desc[s];
        desc[w] = lead;
        issue_w(lead, w);
        // This wave's loads of step q have landed: younger are the next D - 2 steps' kWInstr + 2 instructions each and
        // the weights just issued, kWInstr (a unit's output stores only add younger ones). The barrier then makes the
        // other waves' A operands and scales of step q visible, and frees slot w of the shared rings.
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kWait) : "memory");
        __builtin_amdgcn_s_barrier();
        issue_a(lead, w);
        advance(lead);
        const uint32_t wrow = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)(wring[s][wave]) +
                              (uint32_t)r16 * FS::kRowLds;
        const uint32_t abase = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)(aring[s]);
        const uint32_t sadr = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)(sring[s]) + 16u * (uint32_t)g;
        const int live = min(4, (cur.cnt - cur.n0 + 3) >> 2);  // results j < live hold pairs
        FS::step(wrow, abase, a_rd, sadr, cur.sb, g, live, run);
        if (cur.sb == spr - 1) {
            const int o = cur.o0 + r16;
            const float* bias = cur.mat ? a.bias1 : a.bias0;
            float* y = cur.mat ? a.y1 : a.y0;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int pr = cur.n0 + 4 * j + g;
                if (j < live && pr < cur.cnt && o < a.n_rows) {
                    const float v = bias ? bias[o] + run[j] : run[j];
                    const int p = cur.pbeg + pr;
                    if (a.comb) {
                        // explicit LDS reads, like prow_at's (a compiler read would wait for the rings' DMAs)
                        const uint32_t ta = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) int*)(ctok + p);
                        const uint32_t wa = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) float*)(cw + p);
                        int tok;
                        float wt;
                        asm volatile("ds_read_b32 %0, %2\n\tds_read_b32 %1, %3\n\ts_waitcnt lgkmcnt(0)"
                                     : "=&v"(tok), "=&v"(wt)
                                     : "v"(ta), "v"(wa)
                                     : "memory");
                        const float prod = wt * v;
                        __hip_atomic_fetch_add(a.comb + (size_t)tok * a.n_rows + o, prod, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT);
                    } else {
                        y[(size_t)p * a.n_rows + o] = v;
                    }
                }
                run[j] = 0.0f;
            }
        }
        return desc[(s + 1) % D].t < T;
    };
    run_slots(step, std::make_integer_sequence<int, D>{});
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the rings' last DMAs land before the wave ends
}

template <class F, int kBatch>
static hipError_t launch_small(SArgs& sa, int nmat, int experts, hipStream_t st) {
    sa.tiles = (sa.n_rows + 15) / 16;
    const size_t lds = (size_t)sa.spr * 256 * sizeof(float);
    const dim3 grid(sa.tiles * nmat, experts);
    // measured on MI355X: double-buffered batches win for Q6_K from K = 8192 (4 batches per wave: 4096x14336 at
    // M = 4..16 is 10-20 % faster); they lose below, and for Q4_K, whose cheaper batches do not repay the halved
    // occupancy (config-5 MoE step 263 -> 268 us)
    if constexpr (kBatch == 2 && F::kNumMfma == 2) {
        if (sa.spr >= 32) {
            hipLaunchKernelGGL((kquant_mfma_small_kernel<F, kBatch, true>), grid, dim3(256), lds, st, sa);
            return hipGetLastError();
        }
    }
    hipLaunchKernelGGL((kquant_mfma_small_kernel<F, kBatch, false>), grid, dim3(256), lds, st, sa);
    return hipGetLastError();
}

// Static LDS of the expert-stream kernel (its dynamic part is the pair map, 4 bytes a pair).
template <class FS>
static size_t stream_lds_bytes() {
    static const size_t bytes = [] {
        hipFuncAttributes fa{};
        return hipFuncGetAttributes(&fa, reinterpret_cast<const void*>(mfma_stream_kernel<FS, 3>)) == hipSuccess
                   ? fa.sharedSizeBytes
                   : (size_t)(160 * 1024);
    }();
    return bytes;
}

bool mfma_small_supported(int type, int in) { return (type == 12 || type == 14) && in % kQK == 0 && in / kQK <= 64; }

static bool stream_enabled() {
    static const int stream = [] {
        const char* v = getenv("OVFQ_MOE_STREAM");
        return v && *v ? atoi(v) : 1;
    }();
    return stream != 0;
}

// A dense small batch takes the stream kernel only with many 16-row tiles: a few units leave most of the chip idle
// (MI355X, us, stream / super-block-parallel kernel: 14336x4096 at 16 rows 18.9 / 20.2, 32 rows 29.9 / 34.8;
// 4096x4096 at 16 rows 17.9 / 9.4; 4096x14336 at 16 rows 44.7 / 19.0).
static bool stream_dense_ok(int nmat, int n_rows) {
    static const int min_tiles = [] {
        const char* v = getenv("OVFQ_SMALL_STREAM_MIN_TILES");
        return v && *v ? atoi(v) : 768;
    }();
    return (long)nmat * ((n_rows + 15) / 16) >= min_tiles;
}

bool stream_pair_preferred(int type, int in, int n_rows) {
    return stream_enabled() && type == 12 && mfma_small_supported(type, in) && stream_dense_ok(2, n_rows);
}

// Whether launch_mfma_small runs this launch on the expert-stream kernel.
static bool mfma_small_streams(int type, const GroupLaunch& L) {
    const int nmat = L.w1 ? 2 : 1;
    const int pairs = L.expert_off ? L.pairs : L.rows;
    // Q6_K blocks are DMA'd from the 16-byte boundary before them, which is the same in every row when rows are whole
    // multiples of 16 bytes (super-blocks per row a multiple of 8; Mixtral's 14336 and Llama's 4096 inputs are).
    const bool fmt = type == 12 || (type == 14 && (L.in / kQK) % 8 == 0);
    return stream_enabled() && fmt && (L.expert_off || stream_dense_ok(nmat, L.n_rows)) && pairs > 0 &&
           pairs <= kStreamMaxPairs;
}

hipError_t launch_mfma_small(int type, const GroupLaunch& L, hipStream_t st) {
    SArgs sa{};
    for (int i = 0; i < L.experts; i++) {
        sa.w0[i] = L.w0[i];
        sa.w1[i] = L.w1 ? L.w1[i] : nullptr;
    }
    sa.bias0 = L.bias0;
    sa.bias1 = L.bias1;
    sa.y0 = L.y0;
    sa.y1 = L.y1;
    sa.n_rows = L.n_rows;
    sa.spr = L.in / kQK;
    sa.rows = L.rows;
    sa.act_rows = L.rows;
    sa.expert_off = L.expert_off;
    sa.pair_row = L.pair_row;
    sa.q = L.act.q;
    sa.s = L.act.s;
    sa.comb = L.comb;
    sa.comb_tok = L.comb_tok;
    sa.comb_w = L.comb_w;
    const int nmat = L.w1 ? 2 : 1;
    const int pairs = L.expert_off ? L.pairs : L.rows;
    if (L.comb && (nmat != 1 || !L.expert_off || !L.comb_tok || !L.comb_w)) return hipErrorInvalidValue;
    if (mfma_small_streams(type, L)) {
        sa.tiles = (sa.n_rows + kStreamRows - 1) / kStreamRows;  // 64-row groups
        const long units = (long)L.experts * nmat * sa.tiles;
        int dev = 0, cus = 256;
        if (hipGetDevice(&dev) == hipSuccess) (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
        // Workgroups per CU: three (two if the pair map's LDS does not fit three). Measured on MI355X (config-5 MoE
        // step, whose gate/up launch has 3584 units): three per CU, 179.6 us mean of five alternating runs against
        // 181.3 us at four (LDS would allow four up to 140 pairs); two per CU 184.9-186.1 against 180.6-183.9 us, and 896
        // or 640 workgroups 188-190 us, were slower. A
        // 5-slot ring at two per CU leaves the down launch (512 units) unchanged, 64.4 vs 64.6 us, and makes gate/up
        // 11 % slower.
        static const int per_cu_env = [] {
            const char* v = getenv("OVFQ_MOE_STREAM_WG");
            return v && *v ? atoi(v) : 0;
        }();
        const size_t dyn = (size_t)pairs * sizeof(int) * (L.comb ? 3 : 1);
        const size_t lds = type == 12 ? stream_lds_bytes<StreamQ4K>() : stream_lds_bytes<StreamQ6K>();
        const int per_cu = per_cu_env ? per_cu_env : (lds + dyn <= 160 * 1024 / 3 ? 3 : 2);
        const int grid = (int)std::min<long>(units, (long)cus * per_cu);
        if (type == 12)
            hipLaunchKernelGGL((mfma_stream_kernel<StreamQ4K, 3>), dim3(grid), dim3(256), dyn, st, sa, L.experts, nmat,
                               pairs);
        else
            hipLaunchKernelGGL((mfma_stream_kernel<StreamQ6K, 3>), dim3(grid), dim3(256), dyn, st, sa, L.experts, nmat,
                               pairs);
        return hipGetLastError();
    }
    // super-blocks per wave batch (measured on MI355X: 2 beats 4 for every Llama/Mixtral shape)
    static const int forced = [] {
        const char* v = getenv("OVFQ_SMALL_BATCH");
        return v && *v ? atoi(v) : 0;
    }();
    const int batch = forced == 4 ? 4 : 2;
    if (type == 12) return batch == 2 ? launch_small<Q4KMfma, 2>(sa, nmat, L.experts, st)
                                      : launch_small<Q4KMfma, 4>(sa, nmat, L.experts, st);
    return batch == 2 ? launch_small<Q6KMfma, 2>(sa, nmat, L.experts, st)
                      : launch_small<Q6KMfma, 4>(sa, nmat, L.experts, st);
}

}  // namespace ovfq
