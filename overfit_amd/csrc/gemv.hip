// gemv.hip — decode (M = 1) Q4_K / Q6_K projection, one launch per (fused) projection.
//
// The launch covers everything the reference does for one ProjectParallel / ProjectGateUpParallel call
// (RT/Q4KDotKernel.cs:485-645): each workgroup first quantises the fp32 activation to Q8_K into LDS (or copies
// an already-quantised one, the ProjectPreQuantized case), then its waves stream weight rows. The quantiser is
// the same device function as the standalone Q8_K kernel, so the activation is bit-identical to the
// reference's QuantizeActivationQ8K.
//
// Grid: persistent — about `wg_per_cu` workgroups per CU, each wave walking row groups (R consecutive output
// rows) with a stride of the total wave count, so the activation prologue is paid once per workgroup. The
// weight stream is double-buffered in registers: the next (row group, 16-block chunk) item's loads are issued
// before the current item is computed.
//
// Per item, a quad owns one super-block column; its fp32 block value is computed exactly as the reference's
// Dot, and the row's sum over blocks is accumulated in ascending block order by one lane per row, so every
// output is bit-identical to the reference's sequential loop.
#include <cstdlib>
#include <type_traits>

#include "kquant_blocks.h"
#include "ovfq_device.h"
#include "ovfq_launch.h"

namespace ovfq {

typedef float f32x4 __attribute__((ext_vector_type(4)));

struct GJob {
    const uint8_t* w;
    const float* bias;
    float* y;
    int n_rows;
    int g_begin;  // first row group of this job
};

struct GArgs {
    GJob job[kMaxJobs];
    int njobs;
    int total_groups;
    int spr;
    const float* x;  // fp32 activation, quantised in the kernel; NULL -> use q/s/b
    const int8_t* q;
    const float* s;
    const int16_t* b;
};

constexpr int kGemvMaxSpr = 64;  // K <= 16384: the whole Q8_K activation fits in LDS (<= 23 KB)
// Per output row, the 16 block values of an item are written to LDS (one 80-byte row: 16-byte aligned, so the lane
// that sums them reads the row with four 16-byte loads).
constexpr int kRedStride = 20;

// acc + the item's 16 block values of LDS row `row`, in ascending block order (from registers: four 16-byte reads).
// A short last chunk stores +0 for the blocks past the row: the running sum starts at +0 and a sum of IEEE additions
// from +0 is never -0 in round-to-nearest, so each trailing acc + 0 returns acc unchanged (NaN and infinities too).
__device__ __forceinline__ float ordered_item_sum(float acc, const float* row) {
    float v[16];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const f32x4 x = reinterpret_cast<const f32x4*>(row)[i];
        v[4 * i] = x.x;
        v[4 * i + 1] = x.y;
        v[4 * i + 2] = x.z;
        v[4 * i + 3] = x.w;
    }
#pragma unroll
    for (int qq = 0; qq < 16; qq++) acc += v[qq];
    return acc;
}

// Activation prologue: each wave takes four super-blocks at a time, one per 16-lane DPP row; lane l of a row
// owns elements [16l, 16l+16) of its block, i.e. bsum group l, and writes one 16-byte LDS chunk.
// `prefetch` issues the first weight item's loads; it runs after the activation loads so that waiting for the
// activation does not also wait for the weights.
template <class F, int W, class Prefetch>
__device__ __forceinline__ void stage_activation(const GArgs& a, uint8_t* lq, int16_t* lb, float* ls, int wave,
                                                 int lane, Prefetch prefetch) {
    constexpr int kPerPass = 4 * W;  // super-blocks per pass: four per wave
    constexpr int kPasses = (kGemvMaxSpr + kPerPass - 1) / kPerPass;
    const int spr = a.spr;
    const int l16 = lane & 15, row = lane >> 4;
    const int pos = F::lds_pos(16 * l16);
    if (a.x) {
        const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, (uint32_t)spr * kQK * 4);
        u32x4 xv[kPasses][4];
#pragma unroll
        for (int p = 0; p < kPasses; p++) {
            const int sb = p * kPerPass + wave * 4 + row;
            if (p * kPerPass < spr) {
#pragma unroll
                for (int i = 0; i < 4; i++) xv[p][i] = ld4(xr, (uint32_t)sb * 1024 + l16 * 64 + i * 16);
            }
        }
        prefetch();
#pragma unroll
        for (int p = 0; p < kPasses; p++) {
            if (p * kPerPass >= spr) break;
            const int sb = p * kPerPass + wave * 4 + row;
            float v[16];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                v[4 * i + 0] = as_float(xv[p][i].x);
                v[4 * i + 1] = as_float(xv[p][i].y);
                v[4 * i + 2] = as_float(xv[p][i].z);
                v[4 * i + 3] = as_float(xv[p][i].w);
            }
            const Q8KRow r = q8k_quantize_row16(v);
            if (sb < spr) {
                *reinterpret_cast<u32x4*>(lq + sb * kLdsSlot + pos) = r.packed;
                lb[sb * 16 + l16] = (int16_t)r.group_sum;
                if (l16 == 0) ls[sb] = r.scale;
            }
        }
    } else {
        const __amdgpu_buffer_rsrc_t qr = make_rsrc(a.q, (uint32_t)spr * kQK);
        const __amdgpu_buffer_rsrc_t br = make_rsrc(a.b, (uint32_t)spr * 32);
        const __amdgpu_buffer_rsrc_t sr = make_rsrc(a.s, (uint32_t)spr * 4);
        u32x4 qv[kPasses];
        uint32_t bv[kPasses], sv[kPasses];
#pragma unroll
        for (int p = 0; p < kPasses; p++) {
            const int sb = p * kPerPass + wave * 4 + row;
            if (p * kPerPass < spr) {
                qv[p] = ld4(qr, (uint32_t)sb * kQK + l16 * 16);
                bv[p] = __builtin_amdgcn_raw_buffer_load_b16(br, (int)((uint32_t)sb * 32 + l16 * 2), 0, 0);
                sv[p] = ld1(sr, (uint32_t)sb * 4);
            }
        }
        prefetch();
#pragma unroll
        for (int p = 0; p < kPasses; p++) {
            if (p * kPerPass >= spr) break;
            const int sb = p * kPerPass + wave * 4 + row;
            if (sb < spr) {
                *reinterpret_cast<u32x4*>(lq + sb * kLdsSlot + pos) = qv[p];
                lb[sb * 16 + l16] = (int16_t)bv[p];
                if (l16 == 0) ls[sb] = as_float(sv[p]);
            }
        }
    }
}

// kMulti: the launch has several jobs (fused projections); with one, no job lookup is needed. W: waves per
// workgroup (the activation prologue is paid once per workgroup, its quantisation spread over the W waves).
template <class F, int R, bool kMulti, int W>
__global__ __launch_bounds__(64 * W) void kquant_gemv_kernel(const GArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int spr = a.spr;
    uint8_t* lq = smem;
    int16_t* lb = reinterpret_cast<int16_t*>(smem + spr * kLdsSlot);
    float* ls = reinterpret_cast<float*>(smem + spr * (kLdsSlot + 32));
    float* red = reinterpret_cast<float*>(smem + ((spr * (kLdsSlot + 36) + 15) & ~15));
    const int wave = wave_id();
    const int lane = threadIdx.x & 63;
    const int q = lane >> 2, t = lane & 3;
    const int nchunks = (spr + 15) >> 4;
    const int stride = gridDim.x * W;
    const int total = a.total_groups;
    const uint32_t row_bytes = (uint32_t)spr * F::kBytes;
    float* rw = red + wave * R * kRedStride;

    // One work item = (row group g, 16-block chunk c): the weights of R rows plus, on a row group's last chunk,
    // the bias of those rows.
    struct Item {
        typename F::W w[R];
        uint32_t bias;
    };

    // Job fields and first row of row group g (wave-uniform). Every job field is read with a compile-time index
    // and chosen by select, so the table stays in scalar registers: indexing it with a run-time job number would
    // re-read the kernel arguments through scalar memory (a dependent wait) for every item.
    struct Cur {
        const uint8_t* w;
        const float* bias;
        float* y;
        int n_rows;
        int row0;
    };
    auto locate = [&](int g) -> Cur {
        Cur c{a.job[0].w, a.job[0].bias, a.job[0].y, a.job[0].n_rows, 0};
        if constexpr (kMulti) {
#pragma unroll
            for (int i = 1; i < kMaxJobs; i++) {
                const bool take = i < a.njobs && g >= a.job[i].g_begin;
                c.w = take ? a.job[i].w : c.w;
                c.bias = take ? a.job[i].bias : c.bias;
                c.y = take ? a.job[i].y : c.y;
                c.n_rows = take ? a.job[i].n_rows : c.n_rows;
                c.row0 = take ? a.job[i].g_begin : c.row0;
            }
        }
        c.row0 = (g - c.row0) * R;
        return c;
    };
    // The weight resource of a row group, made once per row group (a long row's chunks reuse it) and kept beside the
    // job record, not in it (in the record the compiler stopped treating the record's pointers as wave-uniform). It
    // ends with the row group's last block: quads past the last super-block of a short final chunk then read nothing
    // (instead of the next row's blocks). No block read uses bytes past its block. Past the end (valid false) it has
    // zero length.
    struct WRes {
        __amdgpu_buffer_rsrc_t r;
        uint32_t extra;  // the first row's offset past the resource's 4-byte aligned base
    };
    auto bind = [&](const Cur& c, bool valid) -> WRes {
        const uint64_t base_off = (uint64_t)c.row0 * row_bytes;
        const uint64_t al = base_off & ~3ull;
        const uint32_t extra = (uint32_t)(base_off & 3ull);
        // (the length in 64-bit arithmetic: the same value computed in 32 bits made config 1, a 4096x4096 launch of
        // one item per wave, 5 % slower by a different prologue schedule)
        const uint64_t end = (uint64_t)min(c.row0 + R, c.n_rows) * row_bytes;
        return WRes{make_rsrc(c.w + al, valid ? rsrc_bytes(end, al) : 0u), extra};
    };
    // Issues the loads of item (row group of job record jb, weight resource wr, chunk c). The instruction stream is
    // the same whether or not the item exists (past the end the resources have zero length, so the loads return 0
    // without touching memory): the compiler's wait counts then see a fixed number of younger loads and the prefetch
    // overlaps the current item's math.
    auto load_item = [&](const Cur& jb, const WRes& wr, int c, bool valid, Item& it) {
        const int row0 = jb.row0;
        const uint32_t sb = (uint32_t)(c * 16 + q);
#pragma unroll
        for (int r = 0; r < R; r++) it.w[r] = F::load_w(wr.r, wr.extra + r * row_bytes + sb * F::kBytes, t);
        const float* bias = jb.bias;
        const bool want_bias = valid && bias != nullptr && c == nchunks - 1;
        // (readfirstlane: in the multi-job kernel the compiler kept the job's row count in a vector register and
        // wrapped this load in a loop over distinct resources)
        const uint32_t bbytes = (uint32_t)__builtin_amdgcn_readfirstlane(want_bias ? jb.n_rows * 4 : 0);
        const __amdgpu_buffer_rsrc_t bsr = make_rsrc(bias, bbytes);
        it.bias = ld1(bsr, (uint32_t)(row0 + (lane < R ? lane : 0)) * 4);
    };

    int g = blockIdx.x * W + wave;
    int c = 0;
    Item ia, ib;
    // The first item's lookup runs inside the prefetch, after the activation loads have gone out (they, not the
    // weights, bound the start of the first item).
    stage_activation<F, W>(a, lq, lb, ls, wave, lane, [&] {
        const Cur c0 = locate(g < total ? g : 0);
        load_item(c0, bind(c0, g < total), 0, g < total, ia);
    });
    __syncthreads();
    if (g >= total) return;
    Cur cj = locate(g);  // job record of row group g, looked up once per row group
    WRes cw = bind(cj, true);

    float acc = 0.0f;
    int a_chunk = -1;
    typename F::A av;
    // Computes item (g, c) from `cur` after issuing the loads of the next item into `nxt`.
    auto step = [&](Item& cur, Item& nxt) -> bool {
        int ng = g, nc = c + 1;
        if (nc == nchunks) {
            nc = 0;
            ng += stride;
        }
        const bool more = ng < total;
        Cur nj = cj;  // the same row group (and resource) for its next chunk
        WRes nw = cw;
        if (nc == 0) {
            nj = locate(more ? ng : 0);
            nw = bind(nj, more);
        }
        load_item(nj, nw, nc, more, nxt);
        const int sb = c * 16 + q;
        const bool live = sb < spr;
        if (c != a_chunk) {
            av = F::load_a_lds(lq, lb, ls, live ? sb : 0, t);
            a_chunk = c;
        }
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float v = F::dot(cur.w[r], av, t);
            if (t == 0) rw[r * kRedStride + q] = live ? v : 0.0f;
        }
        wave_sync();
        if (lane < R) acc = ordered_item_sum(acc, rw + lane * kRedStride);
        wave_sync();
        if (c == nchunks - 1) {
            if (lane < R && cj.row0 + lane < cj.n_rows) {
                // bias[o] + sum (RT/Q4KDotKernel.cs:473); no add at all without a bias
                cj.y[cj.row0 + lane] = cj.bias ? as_float(cur.bias) + acc : acc;
            }
            acc = 0.0f;
        }
        g = ng;
        c = nc;
        cj = nj;
        cw = nw;
        return more;
    };
    while (step(ia, ib) && step(ib, ia)) {
    }
}

namespace {

int env_int(const char* name, int dflt) {
    const char* v = getenv(name);
    return v && *v ? atoi(v) : dflt;
}

int cu_count() {
    static int cus[16] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 16) return 256;
    if (!cus[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cus[dev] = n;
    }
    return cus[dev];
}

template <class F, int R, int W>
hipError_t launch_gemv_w(const GArgs& ga, int njobs, int wgs, hipStream_t st) {
    const size_t lds = (size_t)((ga.spr * (kLdsSlot + 36) + 15) & ~15) + W * R * kRedStride * sizeof(float);
    if (njobs > 1)
        hipLaunchKernelGGL((kquant_gemv_kernel<F, R, true, W>), dim3(wgs), dim3(64 * W), lds, st, ga);
    else
        hipLaunchKernelGGL((kquant_gemv_kernel<F, R, false, W>), dim3(wgs), dim3(64 * W), lds, st, ga);
    return hipGetLastError();
}

template <class F, int R>
hipError_t launch_gemv(GArgs& ga, const ProjJob* jobs, int njobs, hipStream_t st) {
    int groups = 0;
    for (int i = 0; i < njobs; i++) {
        ga.job[i].g_begin = groups;
        groups += (jobs[i].n_rows + R - 1) / R;
    }
    ga.total_groups = groups;
    // Waves per workgroup (measured on MI355X, graph replay over weight copies beyond the cache, us, 4 / 8 waves, one
    // eight-wave workgroup per CU): Q4_K rows longer than 16 blocks (one row per wave) 4096x14336 11.4 / 10.5,
    // 8192x8192 9.9 / 9.7; the Q6_K 128256x4096 LM head 83.5 / 80.2. Everything else keeps four-wave workgroups:
    // the Llama-3-8B layer's launches are 1-12 % slower with 8 (also 12 or 16) waves, and so are Q6_K 4096x14336
    // and 8192x8192.
    static const int forced_w = env_int("OVFQ_GEMV_WAVES", 0);
    int W = (std::is_same<F, Q4K>::value && ga.spr > 16) || (std::is_same<F, Q6K>::value && groups >= 65536) ? 8 : 4;
    if (forced_w == 4 || forced_w == 8) W = forced_w;
    if (R == 4) W = 4;
    // Workgroups per CU (measured on MI355X): 2 with two rows per wave (Q4_K rows of up to 16 blocks), else 3;
    // one eight-wave workgroup.
    static const int forced_wg = env_int("OVFQ_GEMV_WG_PER_CU", 0);
    const int wg_per_cu = forced_wg > 0 ? forced_wg : W == 8 ? 1 : (R == 2 ? 2 : 3);
    int wgs = (groups + W - 1) / W;
    const int cap = cu_count() * wg_per_cu;
    if (wgs > cap) wgs = cap;
    if constexpr (R != 4) {
        if (W == 8) return launch_gemv_w<F, R, 8>(ga, njobs, wgs, st);
    }
    return launch_gemv_w<F, R, 4>(ga, njobs, wgs, st);
}

}  // namespace

bool gemv_supported(int in) { return in % kQK == 0 && in / kQK <= kGemvMaxSpr; }

// ------------------------------------------------------------------------------------------ several rows
// 2 .. kRowsMax activation rows (small batches, speculative verification): the decode kernel's persistent,
// double-buffered weight stream, each weight block unpacked once per item (F::prep) and dotted with every
// activation row (F::dot_p) from the rows' Q8_K copy in LDS (quantised in the launch from fp32 rows, or copied
// from a prequantised activation). Per (activation row, output row) one lane adds the block values in ascending
// block order, so outputs stay bit-identical to the reference's loop.
constexpr int kRowsMax = 8;
constexpr int kRowsSlots = 128;  // rows * super-blocks per row staged in LDS (<= 50 KB per workgroup)

struct RArgs {
    GJob job[kMaxJobs];
    int njobs;
    int total_groups;
    int spr;
    int rows;
    const float* x;  // fp32 activation rows, quantised in the kernel; NULL -> use q/s/b
    const int8_t* q;
    const float* s;
    const int16_t* b;
};

template <class F, int R>
__global__ __launch_bounds__(256) void kquant_gemv_rows_kernel(const RArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int spr = a.spr, rows = a.rows, slots = rows * spr;
    uint8_t* lq = smem;                                                      // [rows][spr] activation slots
    int16_t* lb = reinterpret_cast<int16_t*>(smem + slots * kLdsSlot);       // [rows][spr][16] bsums
    float* ls = reinterpret_cast<float*>(smem + slots * (kLdsSlot + 32));    // [rows][spr] scales
    float* red = reinterpret_cast<float*>(smem + ((slots * (kLdsSlot + 36) + 15) & ~15));
    const int wave = wave_id();
    const int lane = threadIdx.x & 63;
    const int q = lane >> 2, t = lane & 3;
    const int nchunks = (spr + 15) >> 4;
    const int stride = gridDim.x * 4;
    const int total = a.total_groups;
    const uint32_t row_bytes = (uint32_t)spr * F::kBytes;
    float* rw = red + wave * (R * kRowsMax * kRedStride);

    struct Item {
        typename F::W w[R];
        uint32_t bias;
    };
    struct Cur {
        const uint8_t* w;
        const float* bias;
        float* y;
        int n_rows;
        int row0;
    };
    // job of row group g, chosen with compile-time indices (the table stays in scalar registers)
    auto locate = [&](int g) -> Cur {
        Cur c{a.job[0].w, a.job[0].bias, a.job[0].y, a.job[0].n_rows, a.job[0].g_begin};
#pragma unroll
        for (int i = 1; i < kMaxJobs; i++) {
            const bool take = i < a.njobs && g >= a.job[i].g_begin;
            c.w = take ? a.job[i].w : c.w;
            c.bias = take ? a.job[i].bias : c.bias;
            c.y = take ? a.job[i].y : c.y;
            c.n_rows = take ? a.job[i].n_rows : c.n_rows;
            c.row0 = take ? a.job[i].g_begin : c.row0;
        }
        c.row0 = (g - c.row0) * R;
        return c;
    };
    // loads of item (g, c); past the end the resources have zero length (the loads return 0)
    auto load_item = [&](int g, int c, bool valid, Item& it) {
        const Cur jb = locate(valid ? g : 0);
        const int row0 = jb.row0;
        const uint64_t base_off = (uint64_t)row0 * row_bytes;
        const uint64_t al = base_off & ~3ull;
        const uint32_t extra = (uint32_t)(base_off & 3ull);
        const uint64_t end = (uint64_t)min(row0 + R, jb.n_rows) * row_bytes;
        const __amdgpu_buffer_rsrc_t wr = make_rsrc(jb.w + al, valid ? rsrc_bytes(end, al) : 0u);
        const uint32_t sb = (uint32_t)(c * 16 + q);
#pragma unroll
        for (int r = 0; r < R; r++) it.w[r] = F::load_w(wr, extra + r * row_bytes + sb * F::kBytes, t);
        const float* bias = jb.bias;
        const bool want_bias = valid && bias != nullptr && c == nchunks - 1;
        const __amdgpu_buffer_rsrc_t bsr = make_rsrc(bias, want_bias ? (uint32_t)jb.n_rows * 4 : 0u);
        it.bias = ld1(bsr, (uint32_t)(row0 + lane % R) * 4);
    };

    int g = blockIdx.x * 4 + wave;
    int c = 0;
    Item ia, ib;
    if (a.x) {
        // The rows' fp32 activation quantised here (the standalone quantiser's arithmetic): slot i = m * spr + sb
        // is 256 consecutive floats; lane l16 of a 16-lane row owns elements [16 l16, 16 l16 + 16), bsum group l16.
        constexpr int kPasses = 4;
        const int l16 = lane & 15, hrow = lane >> 4;
        const int pos = F::lds_pos(16 * l16);
        const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, (uint32_t)slots * kQK * 4);
#pragma unroll 1
        for (int base = 0; base < slots; base += 16 * kPasses) {
            u32x4 xv[kPasses][4];
#pragma unroll
            for (int p = 0; p < kPasses; p++) {
                const uint32_t i = (uint32_t)(base + p * 16 + wave * 4 + hrow);  // past the slots: reads return 0
#pragma unroll
                for (int k = 0; k < 4; k++) xv[p][k] = ld4(xr, i * kQK * 4 + l16 * 64 + k * 16);
            }
            if (base == 0) load_item(g, 0, g < total, ia);
#pragma unroll
            for (int p = 0; p < kPasses; p++) {
                // passes wholly past the slots quantise nothing (their loads above stay: a fixed load count keeps the
                // weight prefetch in flight through the compiler's wait counts)
                if (base + p * 16 >= slots) break;  // wave-uniform
                const int i = base + p * 16 + wave * 4 + hrow;
                float v[16];
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    v[4 * k + 0] = as_float(xv[p][k].x);
                    v[4 * k + 1] = as_float(xv[p][k].y);
                    v[4 * k + 2] = as_float(xv[p][k].z);
                    v[4 * k + 3] = as_float(xv[p][k].w);
                }
                const Q8KRow r = q8k_quantize_row16(v);  // every lane of the 16-lane row takes part
                if (i < slots) {
                    *reinterpret_cast<u32x4*>(lq + i * kLdsSlot + pos) = r.packed;
                    lb[i * 16 + l16] = (int16_t)r.group_sum;
                    if (l16 == 0) ls[i] = r.scale;
                }
            }
        }
    } else {
        // Activation slots i = m * spr + sb (the LDS and the global layout agree): each 16-lane row of a wave takes
        // one slot per pass, lane l16 its 16 quants and bsum group l16; rounds of four passes, each round's loads
        // issued before its stores (the first item's weights go out after the first round's loads).
        constexpr int kPasses = 4;
        const int l16 = lane & 15, hrow = lane >> 4;
        const int pos = F::lds_pos(16 * l16);
        const __amdgpu_buffer_rsrc_t qr = make_rsrc(a.q, (uint32_t)slots * kQK);
        const __amdgpu_buffer_rsrc_t br = make_rsrc(a.b, (uint32_t)slots * 32);
        const __amdgpu_buffer_rsrc_t sr = make_rsrc(a.s, (uint32_t)slots * 4);
#pragma unroll 1
        for (int base = 0; base < slots; base += 16 * kPasses) {
            u32x4 qv[kPasses];
            uint32_t bv[kPasses], sv[kPasses];
#pragma unroll
            for (int p = 0; p < kPasses; p++) {
                const uint32_t i = (uint32_t)(base + p * 16 + wave * 4 + hrow);  // past the slots: reads return 0
                qv[p] = ld4(qr, i * kQK + l16 * 16);
                bv[p] = __builtin_amdgcn_raw_buffer_load_b16(br, (int)(i * 32 + l16 * 2), 0, 0);
                sv[p] = ld1(sr, i * 4);
            }
            if (base == 0) load_item(g, 0, g < total, ia);
#pragma unroll
            for (int p = 0; p < kPasses; p++) {
                const int i = base + p * 16 + wave * 4 + hrow;
                if (i < slots) {
                    *reinterpret_cast<u32x4*>(lq + i * kLdsSlot + pos) = qv[p];
                    lb[i * 16 + l16] = (int16_t)bv[p];
                    if (l16 == 0) ls[i] = as_float(sv[p]);
                }
            }
        }
    }
    __syncthreads();
    if (g >= total) return;

    float acc = 0.0f;
    auto step = [&](Item& cur, Item& nxt) -> bool {
        int ng = g, nc = c + 1;
        if (nc == nchunks) {
            nc = 0;
            ng += stride;
        }
        const bool more = ng < total;
        load_item(ng, nc, more, nxt);
        const int sb = c * 16 + q;
        const bool live = sb < spr;
        const int sbl = live ? sb : 0;
        typename F::P pw[R];
#pragma unroll
        for (int r = 0; r < R; r++) pw[r] = F::prep(cur.w[r], t);
        // one activation row at a time: the rows' operands are not all held in registers at once
#pragma unroll 1
        for (int m = 0; m < rows; m++) {
            const typename F::A av = F::load_a_lds(lq + m * spr * kLdsSlot, lb + m * spr * 16, ls + m * spr, sbl, t);
#pragma unroll
            for (int r = 0; r < R; r++) {
                const float v = F::dot_p(pw[r], av);
                if (t == 0) rw[(m * R + r) * kRedStride + q] = live ? v : 0.0f;
            }
        }
        wave_sync();
        if (lane < rows * R) acc = ordered_item_sum(acc, rw + lane * kRedStride);
        wave_sync();
        if (c == nchunks - 1) {
            const Cur jb = locate(g);
            const int m = lane / R, r = lane % R;
            if (lane < rows * R && jb.row0 + r < jb.n_rows) {
                // bias[o] + sum (RT/Q4KDotKernel.cs:473); no add at all without a bias
                jb.y[(size_t)m * jb.n_rows + jb.row0 + r] = jb.bias ? as_float(cur.bias) + acc : acc;
            }
            acc = 0.0f;
        }
        g = ng;
        c = nc;
        return more;
    };
    while (step(ia, ib) && step(ib, ia)) {
    }
}

bool gemv_rows_supported(int in, int rows) {
    return rows >= 1 && rows <= kRowsMax && in % kQK == 0 && rows * (in / kQK) <= kRowsSlots;
}

// Every workgroup quantises all rows of its activation; up to 64 super-blocks in all (four 4096-element rows) that
// costs no more than a separate quantise launch (MI355X, Llama-3-8B layer at 2 rows 54.4 -> 51.6 us, at 4 rows
// 62.6 -> 62.2 us) and saves the launch.
bool gemv_rows_quantize_inside(int in, int rows) {
    static const int limit = env_int("OVFQ_GEMV_ROWS_QUANT_INSIDE_MAX_SLOTS", 64);
    return gemv_rows_supported(in, rows) && rows * (in / kQK) <= limit;
}

namespace {

template <class F, int R>
hipError_t launch_gemv_rows(RArgs& ra, const ProjJob* jobs, int njobs, hipStream_t st) {
    int groups = 0;
    for (int i = 0; i < njobs; i++) {
        ra.job[i].g_begin = groups;
        groups += (jobs[i].n_rows + R - 1) / R;
    }
    ra.total_groups = groups;
    // Workgroups per CU: 2; one long row (K > 16384, past the one-row decode kernel) takes 3 like that kernel's
    // long rows.
    static const int forced_wg = env_int("OVFQ_GEMV_ROWS_WG_PER_CU", 0);
    const int wg_per_cu = forced_wg > 0 ? forced_wg : (ra.rows == 1 && ra.spr > 16 ? 3 : 2);
    int wgs = (groups + 3) / 4;
    const int cap = cu_count() * wg_per_cu;
    if (wgs > cap) wgs = cap;
    const int slots = ra.rows * ra.spr;
    const size_t lds = (size_t)((slots * (kLdsSlot + 36) + 15) & ~15) + 4 * R * kRowsMax * kRedStride * sizeof(float);
    hipLaunchKernelGGL((kquant_gemv_rows_kernel<F, R>), dim3(wgs), dim3(256), lds, st, ra);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_gemv_rows_kquant(int type, const ProjJob* jobs, int njobs, int in, int rows, const float* x,
                                   ActQ act, hipStream_t st) {
    if (!gemv_rows_supported(in, rows)) return hipErrorInvalidValue;
    RArgs ra{};
    for (int i = 0; i < kMaxJobs; i++) {
        if (i < njobs) {
            ra.job[i] = GJob{jobs[i].w, jobs[i].bias, jobs[i].y, jobs[i].n_rows, 0};
        } else {
            ra.job[i] = GJob{nullptr, nullptr, nullptr, 0, 0x7fffffff};
        }
    }
    ra.njobs = njobs;
    ra.spr = in / kQK;
    ra.rows = rows;
    ra.x = x;
    ra.q = act.q;
    ra.s = act.s;
    ra.b = act.b;
    static const int forced_r = env_int("OVFQ_GEMV_ROWS_R", 0);
    const int R = forced_r == 1 || forced_r == 2 ? forced_r : (ra.spr <= 16 ? 2 : 1);
    if (type == 12) return R == 2 ? launch_gemv_rows<Q4K, 2>(ra, jobs, njobs, st) : launch_gemv_rows<Q4K, 1>(ra, jobs, njobs, st);
    return R == 2 ? launch_gemv_rows<Q6K, 2>(ra, jobs, njobs, st) : launch_gemv_rows<Q6K, 1>(ra, jobs, njobs, st);
}

// Every workgroup of the decode kernel quantises the whole activation, for every input it takes (up to 64
// super-blocks): that prologue costs less than a standalone quantise launch (MI355X, config-2 layer step with the
// 4096x14336 Q6_K down launch quantising its input in-launch 36.97 -> 36.76 us; decode GEMVs at K = 8192-16384
// 1-8 % faster).
bool gemv_quantize_inside(int in) {
    static const int limit = env_int("OVFQ_GEMV_QUANT_INSIDE_MAX_SPR", kGemvMaxSpr);
    return in / kQK <= limit;
}

hipError_t launch_gemv_kquant(int type, const ProjJob* jobs, int njobs, int in, const float* x, ActQ act,
                              hipStream_t st) {
    GArgs ga{};
    for (int i = 0; i < kMaxJobs; i++) {
        if (i < njobs) {
            ga.job[i] = GJob{jobs[i].w, jobs[i].bias, jobs[i].y, jobs[i].n_rows, 0};
        } else {
            ga.job[i] = GJob{nullptr, nullptr, nullptr, 0, 0x7fffffff};
        }
    }
    ga.njobs = njobs;
    ga.spr = in / kQK;
    ga.x = x;
    ga.q = act.q;
    ga.s = act.s;
    ga.b = act.b;
    static const int forced_r = env_int("OVFQ_GEMV_ROWS_PER_WAVE", 0);
    int R = forced_r;
    // Rows per wave (measured on MI355X): 2 for Q4_K rows of up to 16 blocks (K <= 4096), else 1. Q6_K at K = 4096
    // is 7-11 % faster with one row per wave and three workgroups per CU (4096 rows 7.05 -> 6.29 us, 14336 rows
    // 14.3 -> 12.7 us; the 128256-row LM head 85.3 -> 84.3 us).
    if (R != 1 && R != 2 && R != 4) R = type == 12 && ga.spr <= 16 ? 2 : 1;
    if (type == 12) {
        if (R == 4) return launch_gemv<Q4K, 4>(ga, jobs, njobs, st);
        if (R == 2) return launch_gemv<Q4K, 2>(ga, jobs, njobs, st);
        return launch_gemv<Q4K, 1>(ga, jobs, njobs, st);
    }
    if (R == 4) return launch_gemv<Q6K, 4>(ga, jobs, njobs, st);
    if (R == 2) return launch_gemv<Q6K, 2>(ga, jobs, njobs, st);
    return launch_gemv<Q6K, 1>(ga, jobs, njobs, st);
}

}  // namespace ovfq
