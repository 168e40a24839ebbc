// mfma.hip — batched (prefill) Q4_K / Q6_K projection on CDNA4 int8 MFMA (v_mfma_i32_16x16x64_i8).
//
// ProjectBatched / ProjectBatchedWeightStationary (RT/Q4KDotKernel.cs:681-955, RT/Q6KDotKernel.cs:403-510):
// y[n][o] = biasO + sum over super-blocks (ascending) of the block's fp32 value, for every activation row n.
//
// Exactness. Everything before the per-super-block fp32 tail is integer arithmetic, so it can be regrouped:
//  Q4_K  mainAcc = sum_e (sc*nib)_e * q8_e. sc*nib <= 945 does not fit int8, so it is split as 128*hi + lo
//        (lo in [0,127], hi in [0,7]); two MFMAs give sum lo*q8 and sum hi*q8, mainAcc = acc_lo + (acc_hi << 7).
//        minAcc = sum_s m_s * (bsums[2s] + bsums[2s+1]) = sum_e m_{s(e)} * q8_e: a third MFMA whose weight operand
//        is the sub-block min broadcast over its 32 elements.
//  Q6_K  unsignedTerm - 32*bsumTerm = sum_e sc_{s(e)} * (q_e - 32) * q8_e. W = sc*(q-32) lies in [-4064, 4096]
//        (sc = -128 is a legal scale), split as 128*hi + lo (lo in [0,127], hi in [-32,32]); two MFMAs.
// Both regroupings use the Q8_K definition bsums[j] = sum of quants 16j..16j+15 (the quantiser's output), so the
// bsums plane itself is not read. The fp32 tail of each super-block — q8Scale * (d*mainAcc - dmin*minAcc) and
// d*q8Scale*mainAcc (RT/Q4KDotKernel.cs:944, RT/Q6KDotKernel.cs:114-115) — is evaluated per (n, o) in the
// reference's operation order and accumulated over super-blocks in ascending order from +0, then biasO + sum.
//
// Tiling. A workgroup (4 waves) owns 64 weight rows (16 per wave) x NT activation rows. MFMA operand A is the
// activation (row n = lane % 16 of a 16-row sub-tile, staged in LDS), operand B the weights (column o = lane % 16:
// the lane's own weight row, built in registers straight from the GGUF bytes), so the 4 results a lane holds,
// D[4*(lane/16) + i][lane % 16], all belong to its own weight row: d, dmin and the bias stay lane-local. In both
// operands byte j of lane-group g = lane / 16 carries K index 16*g + j of a 64-element chunk.
// Per super-block the workgroup stages NT rows x 256 quants (+ scales) in LDS (double-buffered; 272-byte row stride
// keeps the 16 lanes reading one K slice on distinct banks) while the next super-block's weights and activation
// are in flight. Workgroups are numbered XCD-aware: the workgroups of one weight tile run consecutively on the
// same XCD (blockIdx % 8), so its bytes come from HBM once and from that XCD's L2 for the other activation tiles.
#include "kquant_blocks.h"
#include "ovfq_device.h"
#include "ovfq_launch.h"

namespace ovfq {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct MJob {
    const uint8_t* w;
    const float* bias;
    float* y;
    int n_out;  // output size of this weight
    int tile0;  // first 64-row tile index of this job in the launch
};

struct MArgs {
    MJob job[kMaxJobs];
    int njobs;
    int o_tiles;  // 64-row weight tiles over all jobs
    int n_tiles;  // ceil(M / NT)
    int m_rows;   // M
    int spr;      // K / 256
    const int8_t* q;
    const float* s;
};

constexpr int kActStride = 272;  // LDS bytes per staged activation row: 256 quants + 16 bytes padding

__device__ __forceinline__ i32x4 mfma16(i32x4 a, i32x4 b, i32x4 c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// Four 16-bit values, two per dword (pe: bytes 0 and 2 of the result, po: bytes 1 and 3), each in [0, 2^15):
// lo = v & 127 and h = (v >> 7) & 255 as packed bytes in the original byte order.
__device__ __forceinline__ void split_lo_hi(uint32_t pe, uint32_t po, uint32_t& lo, uint32_t& h) {
    lo = (pe & 0x007f007fu) | ((po & 0x007f007fu) << 8);
    h = ((pe >> 7) & 0x00ff00ffu) | (((po >> 7) & 0x00ff00ffu) << 8);
}

// ------------------------------------------------------------------------------------------ Q4_K weight operands
struct Q4KMfma {
    static constexpr int kBytes = kQ4KBytes;
    static constexpr int kNumMfma = 3;  // lo, hi, min
    struct W {
        u32x4 h;      // d, dmin, 12 packed scale/min bytes
        u32x4 qs[4];  // chunk c: qs[32c + 16*(g & 1) .. +16]
    };
    __device__ __forceinline__ static W load(__amdgpu_buffer_rsrc_t r, uint32_t off, int g) {
        W w;
        w.h = ld4(r, off);
#pragma unroll
        for (int c = 0; c < 4; c++) w.qs[c] = ld4(r, off + 16 + 32 * c + 16 * (g & 1));
        return w;
    }
    // Chunk c = elements 64c..64c+63; lane-group g holds 64c + 16g + j: the low (g < 2) or high nibble of
    // qs[32c + 16(g&1) + j], sub-block 2c + (g >> 1) (LD/GgmlDequant.cs:64-79 for the scale/min unpacking).
    __device__ __forceinline__ static void operands(const W& w, int c, int g, i32x4 (&op)[kNumMfma]) {
        const int js = 2 * c + (g >> 1);
        const uint32_t jj = (uint32_t)(js & 3) * 8;
        const uint32_t A = (w.h.y >> jj) & 0xffu, B = (w.h.z >> jj) & 0xffu, C = (w.h.w >> jj) & 0xffu;
        uint32_t sc, m;
        if (c < 2) {
            sc = A & 63u;
            m = B & 63u;
        } else {
            sc = (C & 0x0fu) | ((A >> 6) << 4);
            m = (C >> 4) | ((B >> 6) << 4);
        }
        const uint32_t shift = (uint32_t)(g >> 1) * 4;
        const uint32_t qv[4] = {w.qs[c].x, w.qs[c].y, w.qs[c].z, w.qs[c].w};
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t nib = (qv[k] >> shift) & 0x0f0f0f0fu;
            const uint32_t pe = __umul24(nib & 0x00ff00ffu, sc);  // two 16-bit products per dword
            const uint32_t po = __umul24((nib >> 8) & 0x00ff00ffu, sc);
            split_lo_hi(pe, po, lo[k], hi[k]);
        }
        op[0] = i32x4{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3]};
        op[1] = i32x4{(int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
        const int mm = (int)(m * 0x01010101u);
        op[2] = i32x4{mm, mm, mm, mm};
    }
    __device__ __forceinline__ static float d_of(const W& w) { return half_lo(w.h.x); }
    __device__ __forceinline__ static float dmin_of(const W& w) { return half_hi(w.h.x); }
    // q8Scale * (d * mainAcc - dmin * minAcc)   (RT/Q4KDotKernel.cs:944)
    __device__ __forceinline__ static float tail(const i32x4 (&acc)[kNumMfma], int i, float d, float dmin,
                                                 float q8s) {
        const int main_acc = acc[0][i] + (acc[1][i] << 7);
        return q8s * (d * (float)main_acc - dmin * (float)acc[2][i]);
    }
};

// ------------------------------------------------------------------------------------------ Q6_K weight operands
struct Q6KMfma {
    static constexpr int kBytes = kQ6KBytes;
    static constexpr int kNumMfma = 2;  // lo, hi
    struct W {
        uint32_t ql[2][4];  // half h: ql[64h + 16g .. +16]
        uint32_t qh[2][4];  // half h: qh[32h + 16(g & 1) .. +16]
        uint32_t sc;        // byte c = scales[4c + g]
        uint32_t d;
    };
    // 16 bytes at any byte offset (Q6_K rows are only 2-byte aligned).
    __device__ __forceinline__ static void run16(__amdgpu_buffer_rsrc_t r, uint32_t o, uint32_t (&out)[4]) {
        const uint32_t o4 = o & ~3u, sh = o & 3u;
        const u32x4 v = ld4(r, o4);
        const uint32_t v4 = ld1(r, o4 + 16);
        const uint32_t x0 = v.x, x1 = v.y, x2 = v.z, x3 = v.w;
        out[0] = __builtin_amdgcn_alignbyte(x1, x0, sh);
        out[1] = __builtin_amdgcn_alignbyte(x2, x1, sh);
        out[2] = __builtin_amdgcn_alignbyte(x3, x2, sh);
        out[3] = __builtin_amdgcn_alignbyte(v4, x3, sh);
    }
    __device__ __forceinline__ static W load(__amdgpu_buffer_rsrc_t r, uint32_t off, int g) {
        W w;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            run16(r, off + 64 * h + 16 * g, w.ql[h]);
            run16(r, off + 128 + 32 * h + 16 * (g & 1), w.qh[h]);
        }
        uint32_t sc = 0;
#pragma unroll
        for (int c = 0; c < 4; c++)
            sc |= (__builtin_amdgcn_raw_buffer_load_b8(r, (int)(off + 192 + 4 * c + g), 0, 0) & 0xffu) << (8 * c);
        w.sc = sc;
        w.d = __builtin_amdgcn_raw_buffer_load_b16(r, (int)(off + 208), 0, 0);
        return w;
    }
    // Chunk c = elements 64c..64c+63 = half h = c/2, quant group grp = 2(c&1) + (g>>1), l = 16(g&1) + j:
    // ql[64h + 16g + j] (low nibble for grp < 2), qh[32h + l] bits 2*grp, scale scales[4c + g]
    // (RT/Q6KDotKernel.cs:189-213).
    __device__ __forceinline__ static void operands(const W& w, int c, int g, i32x4 (&op)[kNumMfma]) {
        const int h = c >> 1;
        const uint32_t nsh = (uint32_t)(c & 1) * 4;
        const uint32_t hsh = (uint32_t)(c & 1) * 4 + (uint32_t)(g >> 1) * 2;
        const int sc = (int)(int8_t)((w.sc >> (8 * c)) & 0xffu);
        const bool neg = sc < 0;
        const uint32_t asc = (uint32_t)(neg ? -sc : sc);
        // Wb = W + 4096 in [0, 8192] per 16-bit half, built without carry or borrow between the halves:
        //   sc >= 0: (4096 - 32*sc) + q*sc        sc < 0: (4096 + 32*|sc|) - q*|sc|
        const uint32_t k16 = neg ? 4096u + 32u * asc : 4096u - 32u * asc;
        const uint32_t kk = k16 | (k16 << 16);
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t q = ((w.ql[h][k] >> nsh) & 0x0f0f0f0fu) | (((w.qh[h][k] >> hsh) & 0x03030303u) << 4);
            const uint32_t pe = __umul24(q & 0x00ff00ffu, asc);
            const uint32_t po = __umul24((q >> 8) & 0x00ff00ffu, asc);
            uint32_t l, hb;
            split_lo_hi(neg ? kk - pe : kk + pe, neg ? kk - po : kk + po, l, hb);
            lo[k] = l;                                                  // W & 127 (Wb and W agree mod 128)
            hi[k] = ((hb | 0x80808080u) - 0x20202020u) ^ 0x80808080u;  // per byte hb - 32 (hb <= 64: no borrow)
        }
        op[0] = i32x4{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3]};
        op[1] = i32x4{(int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
    }
    __device__ __forceinline__ static float d_of(const W& w) { return half_lo(w.d); }
    __device__ __forceinline__ static float dmin_of(const W&) { return 0.0f; }
    // d * q8Scale * mainAcc   (RT/Q6KDotKernel.cs:114-115)
    __device__ __forceinline__ static float tail(const i32x4 (&acc)[kNumMfma], int i, float d, float, float q8s) {
        const int main_acc = acc[0][i] + (acc[1][i] << 7);
        return d * q8s * (float)main_acc;
    }
};

// ------------------------------------------------------------------------------------------ kernel
template <class F, int NT>
__global__ __launch_bounds__(256) void kquant_mfma_kernel(const MArgs a) {
    constexpr int kSub = NT / 16;
    constexpr int kStage = NT / 16;  // 16-byte activation pieces per thread per super-block
    __shared__ __align__(16) uint8_t act[2][NT * kActStride];
    __shared__ __align__(16) float act_s[2][NT];

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
    const int n_out = a.job[j].n_out;
    const int o0 = (o_tile - a.job[j].tile0) * 64 + wave * 16;  // this wave's first weight row
    const int n0 = n_tile * NT;
    const int spr = a.spr;
    const uint32_t K = (uint32_t)spr * kQK;
    const uint32_t row_bytes = (uint32_t)spr * F::kBytes;

    const uint64_t wbase = (uint64_t)o0 * row_bytes;
    const uint64_t wbase4 = wbase & ~3ull;
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(wptr + wbase4, rsrc_bytes((uint64_t)n_out * row_bytes, wbase4));
    const uint32_t woff = (uint32_t)(wbase - wbase4) + (uint32_t)r16 * row_bytes;
    const __amdgpu_buffer_rsrc_t qr =
        make_rsrc(a.q + (uint64_t)n0 * K, rsrc_bytes((uint64_t)a.m_rows * K, (uint64_t)n0 * K));
    const __amdgpu_buffer_rsrc_t sr = make_rsrc(
        a.s + (uint64_t)n0 * spr, rsrc_bytes((uint64_t)a.m_rows * spr * 4, (uint64_t)n0 * spr * 4));

    u32x4 stg[kStage];
    uint32_t stg_s = 0;
    // Reads past the last super-block of a row land in the next row or past the resource: harmless (not stored).
    auto stage_load = [&](int sb) {
#pragma unroll
        for (int i = 0; i < kStage; i++) {
            const uint32_t idx = (uint32_t)(i * 256) + threadIdx.x;
            stg[i] = ld4(qr, (idx >> 4) * K + (uint32_t)sb * kQK + (idx & 15) * 16);
        }
        if (threadIdx.x < NT) stg_s = ld1(sr, threadIdx.x * (uint32_t)spr * 4 + (uint32_t)sb * 4);
    };
    auto stage_store = [&](int buf) {
#pragma unroll
        for (int i = 0; i < kStage; i++) {
            const uint32_t idx = (uint32_t)(i * 256) + threadIdx.x;
            *reinterpret_cast<u32x4*>(&act[buf][(idx >> 4) * kActStride + (idx & 15) * 16]) = stg[i];
        }
        if (threadIdx.x < NT) act_s[buf][threadIdx.x] = as_float(stg_s);
    };

    float out[kSub][4];
#pragma unroll
    for (int s = 0; s < kSub; s++)
#pragma unroll
        for (int i = 0; i < 4; i++) out[s][i] = 0.0f;

    auto compute = [&](int buf, const typename F::W& w) {
        i32x4 op[4][F::kNumMfma];
#pragma unroll
        for (int c = 0; c < 4; c++) F::operands(w, c, g, op[c]);
        const float d = F::d_of(w), dmin = F::dmin_of(w);
#pragma unroll
        for (int s = 0; s < kSub; s++) {
            i32x4 acc[F::kNumMfma];
#pragma unroll
            for (int k = 0; k < F::kNumMfma; k++) acc[k] = i32x4{0, 0, 0, 0};
            const uint8_t* arow = &act[buf][(s * 16 + r16) * kActStride + 16 * g];
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const u32x4 av = *reinterpret_cast<const u32x4*>(arow + 64 * c);
                const i32x4 aop = i32x4{(int)av.x, (int)av.y, (int)av.z, (int)av.w};
#pragma unroll
                for (int k = 0; k < F::kNumMfma; k++) acc[k] = mfma16(aop, op[c][k], acc[k]);
            }
            const f32x4 q8s = *reinterpret_cast<const f32x4*>(&act_s[buf][s * 16 + 4 * g]);
#pragma unroll
            for (int i = 0; i < 4; i++) out[s][i] += F::tail(acc, i, d, dmin, q8s[i]);
        }
    };

    typename F::W wa = F::load(wr, woff, g), wb;
    stage_load(0);
    stage_store(0);
    __syncthreads();
    auto step = [&](int sb, const typename F::W& cur, typename F::W& nxt) {
        stage_load(sb + 1);
        nxt = F::load(wr, woff + (uint32_t)(sb + 1) * F::kBytes, g);
        compute(sb & 1, cur);
        if (sb + 1 < spr) stage_store((sb + 1) & 1);
        __syncthreads();
    };
    int sb = 0;
    for (; sb + 1 < spr; sb += 2) {
        step(sb, wa, wb);
        step(sb + 1, wb, wa);
    }
    if (sb < spr) step(sb, wa, wb);

    // y[n][o] = biasO + sum   (RT/Q4KDotKernel.cs:951, RT/Q6KDotKernel.cs:507)
    const int o = o0 + r16;
    if (o >= n_out) return;
    const float* bias = a.job[j].bias;
    float* y = a.job[j].y;
    const float bias_o = bias ? bias[o] : 0.0f;
#pragma unroll
    for (int s = 0; s < kSub; s++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int n = n0 + s * 16 + 4 * g + i;
            if (n < a.m_rows) y[(size_t)n * n_out + o] = bias_o + out[s][i];
        }
}

template <class F, int NT>
static hipError_t launch_mfma(MArgs& ma, hipStream_t st) {
    ma.n_tiles = (ma.m_rows + NT - 1) / NT;
    const int grid = (ma.o_tiles + 7) / 8 * 8 * ma.n_tiles;
    hipLaunchKernelGGL((kquant_mfma_kernel<F, NT>), dim3(grid), dim3(256), 0, st, ma);
    return hipGetLastError();
}

int mfma_min_rows() {
    static const int v = [] {
        const char* e = getenv("OVFQ_MFMA_MIN_ROWS");
        return e && *e ? atoi(e) : 32;
    }();
    return v;
}

bool mfma_supported(int type, int rows) { return (type == 12 || type == 14) && rows >= mfma_min_rows(); }

hipError_t launch_project_mfma(int type, const ProjJob* jobs, int njobs, int in, int rows, ActQ act,
                               hipStream_t st) {
    MArgs ma{};
    int tiles = 0;
    for (int i = 0; i < njobs; i++) {
        ma.job[i] = MJob{jobs[i].w, jobs[i].bias, jobs[i].y, jobs[i].n_rows, tiles};
        tiles += (jobs[i].n_rows + 63) / 64;
    }
    ma.njobs = njobs;
    ma.o_tiles = tiles;
    ma.m_rows = rows;
    ma.spr = in / kQK;
    ma.q = act.q;
    ma.s = act.s;
    if (type == 12) return launch_mfma<Q4KMfma, 64>(ma, st);
    return launch_mfma<Q6KMfma, 64>(ma, st);
}

}  // namespace ovfq
