// project.hip — Q4_K / Q6_K / Q8_0 projection kernels for decode (M = 1) and small batches.
//
// Layout in HBM: the weights stay in their GGUF super-block form, output-major (row o = output o's
// input_size-long contraction vector as input_size/256 consecutive blocks). The activation arrives already
// quantised (Q8_K: int8 [M][K], f32 scale [M][K/256], int16 bsums [M][K/16]; Q8_0: int8 + f32 per 32).
//
// Work split (K-quants): a wave owns R consecutive output rows. Its 64 lanes form 16 quads; quad q takes
// super-block column (16c + q) of chunk c, so one chunk covers 16 super-blocks (4096 inputs) of all R rows.
// Each lane streams 48 bytes of every row (16-byte loads: the 16-byte block header plus its own 32 bytes of
// Q4_K nibbles, or its 3 runs + scales of a Q6_K block) and 64 bytes of the activation, unpacks the 6-bit
// scales/mins in registers and forms exact int32 partial dots with v_dot4_i32_i8; a 2-step DPP quad
// reduction gives the block's integer sums. The block's fp32 value is then formed exactly as the reference's
// Dot does, and the per-row sum over super-blocks is accumulated in ascending block order by one lane per
// row (through a small LDS transpose), so every output float is bit-identical to the reference's sequential
// `sum += Dot(...)` loop.
#include <cstdlib>
#include <type_traits>

#include "ovfq_device.h"
#include "ovfq_launch.h"
#include "kquant_blocks.h"

namespace ovfq {

struct KJob {
    const uint8_t* w;
    const float* ws;
    const float* bias;
    float* y;
    int n_rows;
    int wg_begin;
};

struct KArgs {
    KJob job[kMaxJobs];
    int njobs;
    int in;     // K
    int spr;    // K / 256 (K-quants) or K / 32 (Q8_0)
    int rows;   // M
    const int8_t* q;
    const float* s;
    const int16_t* b;
    int rows_per_wave;  // Q8_0 only
    int inc_b, inc_r;   // Q8_0 only: 64 % spr, 64 / spr
};

// ------------------------------------------------------------------------------------------ K-quant kernel
template <class F, int R>
__global__ __launch_bounds__(256) void kquant_project_kernel(const KArgs a) {
    __shared__ float red[4][64][17];
    const int wg = blockIdx.x;
    int j = 0;
#pragma unroll
    for (int i = 1; i < kMaxJobs; i++) j = (i < a.njobs && wg >= a.job[i].wg_begin) ? i : j;
    const uint8_t* jw = a.job[j].w;
    const float* jbias = a.job[j].bias;
    float* jy = a.job[j].y;
    const int n_rows = a.job[j].n_rows;
    const int wave = wave_id();
    const int lane = threadIdx.x & 63;
    const int q = lane >> 2, t = lane & 3;
    const int row0 = ((wg - a.job[j].wg_begin) * 4 + wave) * R;
    if (row0 >= n_rows) return;
    const int nr = min(R, n_rows - row0);
    const int spr = a.spr;
    const uint32_t row_bytes = (uint32_t)spr * F::kBytes;
    const uint64_t base_off = (uint64_t)row0 * row_bytes;
    const uint64_t al = base_off & ~3ull;
    const uint32_t extra = (uint32_t)(base_off & 3ull);
    const __amdgpu_buffer_rsrc_t wr =
        make_rsrc(jw + al, rsrc_bytes((uint64_t)n_rows * row_bytes, al));
    const __amdgpu_buffer_rsrc_t qr = make_rsrc(a.q, rsrc_bytes((uint64_t)a.rows * a.in, 0));
    const __amdgpu_buffer_rsrc_t sr = make_rsrc(a.s, rsrc_bytes((uint64_t)a.rows * spr * 4, 0));
    const __amdgpu_buffer_rsrc_t br = make_rsrc(a.b, rsrc_bytes((uint64_t)a.rows * spr * 32, 0));
    const int nchunks = (spr + 15) >> 4;
    constexpr int kMTile = 64 / R;

    for (int m0 = 0; m0 < a.rows; m0 += kMTile) {
        const int mt = min(kMTile, a.rows - m0);
        float acc = 0.0f;  // lane L = ml * R + r holds the running sum of (activation row m0+ml, output row r)
        for (int c = 0; c < nchunks; c++) {
            const int sb = c * 16 + q;
            const bool live = sb < spr;
            const int nq = min(16, spr - c * 16);
            typename F::W w[R];
#pragma unroll
            for (int r = 0; r < R; r++) w[r] = F::load_w(wr, extra + r * row_bytes + (uint32_t)sb * F::kBytes, t);
            for (int ml = 0; ml < mt; ml++) {
                const typename F::A av = F::load_a(qr, sr, br, a.in, spr, m0 + ml, sb, t);
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const float v = F::dot(w[r], av, t);
                    if (t == 0 && live) red[wave][ml * R + r][q] = v;
                }
            }
            wave_sync();
            if (lane < mt * R) {
                for (int qq = 0; qq < nq; qq++) acc += red[wave][lane][qq];
            }
            wave_sync();
        }
        if (lane < mt * R) {
            const int r = lane % R, ml = lane / R;
            if (r < nr) {
                const int row = row0 + r;
                const float v = jbias ? jbias[row] + acc : acc;
                jy[(size_t)(m0 + ml) * n_rows + row] = v;
            }
        }
    }
}

// ------------------------------------------------------------------------------------------ Q8_0 kernel
// Q8DotKernel.Project / ProjectBatched (RT/Q8DotKernel.cs:155-445): y[o] = (bias +) sum over 32-blocks in
// ascending order of (wScale * aScale) * int8dot. Lanes take (row, block) slots of the wave's rows; block values
// go through LDS and one lane per row adds them in order.
__global__ __launch_bounds__(256) void q8_0_project_kernel(const KArgs a) {
    extern __shared__ float red8[];
    const int wg = blockIdx.x;
    int j = 0;
#pragma unroll
    for (int i = 1; i < kMaxJobs; i++) j = (i < a.njobs && wg >= a.job[i].wg_begin) ? i : j;
    const int n_rows = a.job[j].n_rows;
    const int wave = wave_id();
    const int lane = threadIdx.x & 63;
    const int rw = a.rows_per_wave;
    const int row0 = ((wg - a.job[j].wg_begin) * 4 + wave) * rw;
    if (row0 >= n_rows) return;
    const int nr = min(rw, n_rows - row0);
    const int bpr = a.spr;
    const int stride = bpr + 1;
    float* red = red8 + wave * rw * stride;
    const __amdgpu_buffer_rsrc_t wq =
        make_rsrc(a.job[j].w + (uint64_t)row0 * a.in, rsrc_bytes((uint64_t)n_rows * a.in, (uint64_t)row0 * a.in));
    const __amdgpu_buffer_rsrc_t wsr =
        make_rsrc(a.job[j].ws + (uint64_t)row0 * bpr,
                  rsrc_bytes((uint64_t)n_rows * bpr * 4, (uint64_t)row0 * bpr * 4));
    const __amdgpu_buffer_rsrc_t qr = make_rsrc(a.q, rsrc_bytes((uint64_t)a.rows * a.in, 0));
    const __amdgpu_buffer_rsrc_t sr = make_rsrc(a.s, rsrc_bytes((uint64_t)a.rows * bpr * 4, 0));
    const int slots = nr * bpr;
    for (int m = 0; m < a.rows; m++) {
        int r = lane / bpr, b = lane - r * bpr;
        for (int s = lane; s < slots; s += 64) {
            const uint32_t wo = (uint32_t)r * a.in + b * 32;
            const u32x4 w0 = ld4(wq, wo), w1 = ld4(wq, wo + 16);
            const float wsc = __builtin_bit_cast(float, ld1(wsr, ((uint32_t)r * bpr + b) * 4));
            const uint32_t ao = (uint32_t)m * a.in + b * 32;
            const u32x4 x0 = ld4(qr, ao), x1 = ld4(qr, ao + 16);
            const float asc = __builtin_bit_cast(float, ld1(sr, ((uint32_t)m * bpr + b) * 4));
            int dot = 0;
            dot = sdot4(w0.x, x0.x, dot);
            dot = sdot4(w0.y, x0.y, dot);
            dot = sdot4(w0.z, x0.z, dot);
            dot = sdot4(w0.w, x0.w, dot);
            dot = sdot4(w1.x, x1.x, dot);
            dot = sdot4(w1.y, x1.y, dot);
            dot = sdot4(w1.z, x1.z, dot);
            dot = sdot4(w1.w, x1.w, dot);
            red[r * stride + b] = wsc * asc * (float)dot;
            b += a.inc_b;
            r += a.inc_r;
            if (b >= bpr) {
                b -= bpr;
                r++;
            }
        }
        wave_sync();
        if (lane < nr) {
            float acc = 0.0f;
            for (int bb = 0; bb < bpr; bb++) acc += red[lane * stride + bb];
            const int row = row0 + lane;
            const float* bias = a.job[j].bias;
            a.job[j].y[(size_t)m * n_rows + row] = bias ? bias[row] + acc : acc;
        }
        wave_sync();
    }
}

// ------------------------------------------------------------------------------------------ launchers

template <class F, int R>
static hipError_t launch_kq(KArgs& ka, const ProjJob* jobs, int njobs, hipStream_t st) {
    constexpr int rows_per_wg = 4 * R;
    int wg = 0;
    for (int i = 0; i < njobs; i++) {
        ka.job[i].wg_begin = wg;
        wg += (jobs[i].n_rows + rows_per_wg - 1) / rows_per_wg;
    }
    hipLaunchKernelGGL((kquant_project_kernel<F, R>), dim3(wg), dim3(256), 0, st, ka);
    return hipGetLastError();
}

static void fill_jobs(KArgs& ka, const ProjJob* jobs, int njobs) {
    for (int i = 0; i < kMaxJobs; i++) {
        if (i < njobs) {
            ka.job[i].w = jobs[i].w;
            ka.job[i].ws = jobs[i].ws;
            ka.job[i].bias = jobs[i].bias;
            ka.job[i].y = jobs[i].y;
            ka.job[i].n_rows = jobs[i].n_rows;
        } else {
            ka.job[i] = KJob{nullptr, nullptr, nullptr, nullptr, 0, 0x7fffffff};
        }
    }
    ka.njobs = njobs;
}

// Rows per wave: enough waves to cover the 256 CUs several times over, more rows per wave (more bytes in flight
// per wave, fewer activation re-reads) once the matrix is large.
static int pick_rows_per_wave(int total_rows) {
    if (total_rows >= 16384) return 4;
    if (total_rows >= 4096) return 2;
    return 1;
}

hipError_t launch_project_kquant(int type, const ProjJob* jobs, int njobs, int in, int rows, ActQ act,
                                 hipStream_t st) {
    KArgs ka{};
    fill_jobs(ka, jobs, njobs);
    ka.in = in;
    ka.spr = in / kQK;
    ka.rows = rows;
    ka.q = act.q;
    ka.s = act.s;
    ka.b = act.b;
    int total = 0;
    for (int i = 0; i < njobs; i++) total += jobs[i].n_rows;
    const int R = pick_rows_per_wave(total);
    if (type == 12) {
        if (R == 4) return launch_kq<Q4K, 4>(ka, jobs, njobs, st);
        if (R == 2) return launch_kq<Q4K, 2>(ka, jobs, njobs, st);
        return launch_kq<Q4K, 1>(ka, jobs, njobs, st);
    }
    if (R == 4) return launch_kq<Q6K, 4>(ka, jobs, njobs, st);
    if (R == 2) return launch_kq<Q6K, 2>(ka, jobs, njobs, st);
    return launch_kq<Q6K, 1>(ka, jobs, njobs, st);
}

hipError_t launch_project_q8_0(const ProjJob* jobs, int njobs, int in, int rows, ActQ act, hipStream_t st) {
    KArgs ka{};
    fill_jobs(ka, jobs, njobs);
    ka.in = in;
    ka.spr = in / 32;
    ka.rows = rows;
    ka.q = act.q;
    ka.s = act.s;
    ka.b = nullptr;
    const int bpr = ka.spr;
    int rw = 512 / bpr;
    rw = rw < 1 ? 1 : (rw > 16 ? 16 : rw);
    ka.rows_per_wave = rw;
    ka.inc_b = 64 % bpr;
    ka.inc_r = 64 / bpr;
    const int rows_per_wg = 4 * rw;
    int wg = 0;
    for (int i = 0; i < njobs; i++) {
        ka.job[i].wg_begin = wg;
        wg += (jobs[i].n_rows + rows_per_wg - 1) / rows_per_wg;
    }
    const size_t lds = (size_t)4 * rw * (bpr + 1) * sizeof(float);
    hipLaunchKernelGGL(q8_0_project_kernel, dim3(wg), dim3(256), lds, st, ka);
    return hipGetLastError();
}

// ------------------------------------------------------------------------------------------ Q8_0 decode GEMV
// Q8DotKernel.Project / ProjectParallel (RT/Q8DotKernel.cs:155-350) at M = 1 (and ProjectBatched at 2 .. 8 rows) on
// a persistent grid. Each workgroup copies the Q8_0 activation rows (K int8 + K/32 f32 scales each) into LDS once; its waves then walk row groups of R rows
// in items of 64 blocks: lane l takes block 64c + l of each row (its 32 weight bytes and scale; the wave reads
// 64 consecutive blocks of a row), and the next item's loads are issued before the current item is computed. The
// lane forms the reference's (wScale * aScale) * dot for every activation row; per (activation row, output row), one
// lane adds the item's 64 block values in ascending order (RT/Q8DotKernel.cs:127-137), and bias + sum is written
// after the row's last item.
struct Q8GJob {
    const int8_t* w;
    const float* ws;
    const float* bias;
    float* y;
    int n_rows;
    int g_begin;  // first row group of this job
};

struct Q8GArgs {
    Q8GJob job[kMaxJobs];
    int njobs;
    int total_groups;
    int in;
    int nb;          // blocks per row
    int m_rows;      // activation rows (1 .. kQ8GemvMaxRows), outputs [m_rows][n_rows] per job
    const float* x;  // fp32 activation (one row), quantised in the kernel (in <= kQ8GemvQuantMaxIn); NULL -> q / s
    const int8_t* q;
    const float* s;
};

constexpr int kQ8GemvMaxIn = 32768;       // LDS copy of the activation rows: 32 KB + 4 KB of scales
constexpr int kQ8GemvMaxRows = 8;         // activation rows per launch
constexpr int kQ8GemvQuantMaxIn = 8192;   // in-launch quantisation (every workgroup quantises the whole input)
constexpr int kQ8Red = 68;                // floats per block-value row: 64 values, 16-byte aligned rows
typedef float f32x4q __attribute__((ext_vector_type(4)));

template <int R, bool kMulti>
__global__ __launch_bounds__(256) void q8_0_gemv_kernel(const Q8GArgs a) {
    extern __shared__ __align__(16) uint8_t smem8[];
    const int K = a.in, nb = a.nb, M = a.m_rows;
    uint8_t* lq = smem8;                                          // [M][K] activation quants
    float* ls = reinterpret_cast<float*>(smem8 + M * K);          // [M][nb] activation scales
    float* red = ls + ((M * nb + 3) & ~3);                        // per wave [R][M][kQ8Red] block values
    const int wave = wave_id();
    const int lane = threadIdx.x & 63;
    const int nchunks = (nb + 63) >> 6;
    const int stride = gridDim.x * 4;
    const int total = a.total_groups;
    float* rw = red + wave * R * kQ8GemvMaxRows * kQ8Red;

    struct Item {
        u32x4 w[R][2];
        uint32_t ws[R];
        uint32_t bias;
    };
    struct Cur {
        const int8_t* w;
        const float* ws;
        const float* bias;
        float* y;
        int n_rows;
        int row0;
    };
    auto locate = [&](int g) -> Cur {
        Cur c{a.job[0].w, a.job[0].ws, a.job[0].bias, a.job[0].y, a.job[0].n_rows, 0};
        if constexpr (kMulti) {
#pragma unroll
            for (int i = 1; i < kMaxJobs; i++) {
                const bool take = i < a.njobs && g >= a.job[i].g_begin;
                c.w = take ? a.job[i].w : c.w;
                c.ws = take ? a.job[i].ws : c.ws;
                c.bias = take ? a.job[i].bias : c.bias;
                c.y = take ? a.job[i].y : c.y;
                c.n_rows = take ? a.job[i].n_rows : c.n_rows;
                c.row0 = take ? a.job[i].g_begin : c.row0;
            }
        }
        c.row0 = (g - c.row0) * R;
        return c;
    };
    // Loads of item (row group of jb, chunk c); an invalid item reads through zero-length resources. Lanes past the
    // row's last block read the next row's bytes (or zeros past the group) and are not used.
    auto load_item = [&](const Cur& jb, int c, bool valid, Item& it) {
        const int rows = min(R, jb.n_rows - jb.row0);
        const __amdgpu_buffer_rsrc_t wr =
            make_rsrc(jb.w + (uint64_t)jb.row0 * K, valid ? (uint32_t)rows * (uint32_t)K : 0u);
        const __amdgpu_buffer_rsrc_t wsr =
            make_rsrc(jb.ws + (uint64_t)jb.row0 * nb, valid ? (uint32_t)rows * (uint32_t)nb * 4u : 0u);
        const uint32_t blk = (uint32_t)(c * 64 + lane);
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t off = (uint32_t)r * (uint32_t)K + blk * 32u;
            it.w[r][0] = ld4(wr, off);
            it.w[r][1] = ld4(wr, off + 16);
            it.ws[r] = ld1(wsr, ((uint32_t)r * (uint32_t)nb + blk) * 4u);
        }
        const bool want_bias = valid && jb.bias != nullptr && c == nchunks - 1;
        const __amdgpu_buffer_rsrc_t bsr = make_rsrc(jb.bias, want_bias ? (uint32_t)jb.n_rows * 4u : 0u);
        it.bias = ld1(bsr, (uint32_t)(jb.row0 + (lane < R * M ? lane / M : 0)) * 4u);
    };

    int g = blockIdx.x * 4 + wave;
    int c = 0;
    Item ia, ib;
    if (a.x) {
        // Q8DotKernel.Quantize of the fp32 activation into LDS (the standalone quantiser's device function): pass p
        // covers 1024 floats, 8 lanes per block; loads first, then the first item's weights, then the quantisation.
        constexpr int kPasses = kQ8GemvQuantMaxIn / 1024;
        const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, (uint32_t)K * 4u);
        u32x4 xv[kPasses];
#pragma unroll
        for (int p = 0; p < kPasses; p++) xv[p] = ld4(xr, (uint32_t)(p * 1024 + threadIdx.x * 4) * 4u);  // past K: 0
        load_item(locate(g < total ? g : 0), 0, g < total, ia);
#pragma unroll
        for (int p = 0; p < kPasses; p++) {
            const Q80Lane r = q8_0_quantize_lane(xv[p]);  // every lane takes part
            const int blk = p * 32 + (int)(threadIdx.x >> 3), sub = (int)(threadIdx.x & 7);
            if (blk < nb) {
                reinterpret_cast<uint32_t*>(lq + blk * 32)[sub] = r.packed;
                if (sub == 0) ls[blk] = r.scale;
            }
        }
    } else {
        // activation -> LDS: the quant loads go out first, then the first item's weights, then the LDS stores
        constexpr int kPasses = kQ8GemvMaxIn / 4096;
        const __amdgpu_buffer_rsrc_t qr = make_rsrc(a.q, (uint32_t)(M * K));  // [M][K]: the LDS layout
        const __amdgpu_buffer_rsrc_t sr = make_rsrc(a.s, (uint32_t)(M * nb) * 4u);
        // unconditional: offsets past K (or past the scales) read zeros through the resources' bounds
        u32x4 qv[kPasses];
#pragma unroll
        for (int p = 0; p < kPasses; p++) qv[p] = ld4(qr, (uint32_t)(p * 4096 + threadIdx.x * 16));
        uint32_t sv[kQ8GemvMaxIn / 32 / 256];
#pragma unroll
        for (int p = 0; p < kQ8GemvMaxIn / 32 / 256; p++) sv[p] = ld1(sr, (uint32_t)(p * 256 + threadIdx.x) * 4u);
        load_item(locate(g < total ? g : 0), 0, g < total, ia);
#pragma unroll
        for (int p = 0; p < kPasses; p++) {
            const int i = p * 4096 + (int)threadIdx.x * 16;
            if (i < M * K) *reinterpret_cast<u32x4*>(lq + i) = qv[p];
        }
#pragma unroll
        for (int p = 0; p < kQ8GemvMaxIn / 32 / 256; p++) {
            const int i = p * 256 + (int)threadIdx.x;
            if (i < M * nb) ls[i] = as_float(sv[p]);
        }
    }
    __syncthreads();
    if (g >= total) return;
    Cur cj = locate(g);

    float acc = 0.0f;
    auto step = [&](Item& cur, Item& nxt) -> bool {
        int ng = g, nc = c + 1;
        if (nc == nchunks) {
            nc = 0;
            ng += stride;
        }
        const bool more = ng < total;
        Cur nj = cj;
        if (nc == 0) nj = locate(more ? ng : 0);
        load_item(nj, nc, more, nxt);
        const int blk = c * 64 + lane;
        const bool live = blk < nb;
        const int ab = live ? blk : 0;
#pragma unroll
        for (int m = 0; m < kQ8GemvMaxRows; m++) {
            if (m >= M) break;  // uniform
            const u32x4 x0 = *reinterpret_cast<const u32x4*>(lq + m * K + ab * 32);
            const u32x4 x1 = *reinterpret_cast<const u32x4*>(lq + m * K + ab * 32 + 16);
            const float xs = ls[m * nb + ab];
#pragma unroll
            for (int r = 0; r < R; r++) {
                int dot = 0;
                dot = sdot4(cur.w[r][0].x, x0.x, dot);
                dot = sdot4(cur.w[r][0].y, x0.y, dot);
                dot = sdot4(cur.w[r][0].z, x0.z, dot);
                dot = sdot4(cur.w[r][0].w, x0.w, dot);
                dot = sdot4(cur.w[r][1].x, x1.x, dot);
                dot = sdot4(cur.w[r][1].y, x1.y, dot);
                dot = sdot4(cur.w[r][1].z, x1.z, dot);
                dot = sdot4(cur.w[r][1].w, x1.w, dot);
                // (wScale * aScale) * dot; +0 for the blocks past the row (a short last chunk)
                rw[(r * M + m) * kQ8Red + lane] = live ? as_float(cur.ws[r]) * xs * (float)dot : 0.0f;
            }
        }
        wave_sync();
        if (lane < R * M) {  // lane = r * M + m: weight row r, activation row m
            // the 64 block values in ascending order, read as sixteen 16-byte pieces up front; the running sum starts
            // at +0 and is never -0, so the trailing +0 of a short chunk leaves it unchanged
            f32x4q v[16];
#pragma unroll
            for (int i = 0; i < 16; i++) v[i] = *reinterpret_cast<const f32x4q*>(rw + lane * kQ8Red + 4 * i);
#pragma unroll
            for (int i = 0; i < 16; i++) {
                acc += v[i].x;
                acc += v[i].y;
                acc += v[i].z;
                acc += v[i].w;
            }
        }
        wave_sync();
        if (c == nchunks - 1) {
            const int row = cj.row0 + lane / M, m = lane % M;
            if (lane < R * M && row < cj.n_rows)
                cj.y[(size_t)m * cj.n_rows + row] = cj.bias ? as_float(cur.bias) + acc : acc;
            acc = 0.0f;
        }
        g = ng;
        c = nc;
        cj = nj;
        return more;
    };
    while (step(ia, ib) && step(ib, ia)) {
    }
}

bool q8_0_gemv_supported(int in) { return in % 32 == 0 && in <= kQ8GemvMaxIn; }
bool q8_0_gemv_rows_supported(int in, int rows) {
    return rows >= 1 && rows <= kQ8GemvMaxRows && in % 32 == 0 && (long)rows * in <= kQ8GemvMaxIn;
}
bool q8_0_gemv_quantize_inside(int in) { return q8_0_gemv_supported(in) && in <= kQ8GemvQuantMaxIn; }

namespace {
int q8_cu_count() {
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

template <int R>
hipError_t launch_q8g(Q8GArgs& ga, const ProjJob* jobs, int njobs, hipStream_t st) {
    int groups = 0;
    for (int i = 0; i < njobs; i++) {
        ga.job[i].g_begin = groups;
        groups += (jobs[i].n_rows + R - 1) / R;
    }
    ga.total_groups = groups;
    static const int forced_wg = [] {
        const char* v = getenv("OVFQ_Q8_GEMV_WG_PER_CU");
        return v && *v ? atoi(v) : 0;
    }();
    const int wg_per_cu = forced_wg > 0 ? forced_wg : 2;
    int wgs = (groups + 3) / 4;
    const int cap = q8_cu_count() * wg_per_cu;
    if (wgs > cap) wgs = cap;
    const size_t lds = (size_t)ga.m_rows * ga.in + 4 * (size_t)((ga.m_rows * ga.nb + 3) & ~3) +
                       4 * (size_t)4 * R * kQ8GemvMaxRows * kQ8Red;
    if (njobs > 1)
        hipLaunchKernelGGL((q8_0_gemv_kernel<R, true>), dim3(wgs), dim3(256), lds, st, ga);
    else
        hipLaunchKernelGGL((q8_0_gemv_kernel<R, false>), dim3(wgs), dim3(256), lds, st, ga);
    return hipGetLastError();
}
}  // namespace

hipError_t launch_q8_0_gemv(const ProjJob* jobs, int njobs, int in, int rows, const float* x, ActQ act,
                            hipStream_t st) {
    if ((x && (rows != 1 || !q8_0_gemv_quantize_inside(in))) || !q8_0_gemv_rows_supported(in, rows))
        return hipErrorInvalidValue;
    Q8GArgs ga{};
    for (int i = 0; i < kMaxJobs; i++) {
        if (i < njobs)
            ga.job[i] = Q8GJob{reinterpret_cast<const int8_t*>(jobs[i].w), jobs[i].ws, jobs[i].bias, jobs[i].y,
                               jobs[i].n_rows, 0};
        else
            ga.job[i] = Q8GJob{nullptr, nullptr, nullptr, nullptr, 0, 0x7fffffff};
    }
    ga.njobs = njobs;
    ga.in = in;
    ga.nb = in / 32;
    ga.m_rows = rows;
    ga.x = x;
    ga.q = act.q;
    ga.s = act.s;
    static const int forced_r = [] {
        const char* v = getenv("OVFQ_Q8_GEMV_ROWS_PER_WAVE");
        return v && *v ? atoi(v) : 0;
    }();
    const int R = forced_r == 1 || forced_r == 2 || forced_r == 4 ? forced_r : 2;
    if (R == 4) return launch_q8g<4>(ga, jobs, njobs, st);
    if (R == 1) return launch_q8g<1>(ga, jobs, njobs, st);
    return launch_q8g<2>(ga, jobs, njobs, st);
}

// ------------------------------------------------------------------------------------------ Q8_0 on int8 MFMA
// Q8DotKernel.ProjectBatched (RT/Q8DotKernel.cs:352-445) for several activation rows. The weights are int8 already,
// so each 32-element block is one v_mfma_i32_16x16x32_i8 per 16 x 16 (activation row, output) tile, giving the
// block's exact int32 dot; the reference's tail (wScale * aScale) * dot is then added per (row, output) in
// ascending block order from +0 (Dot, RT/Q8DotKernel.cs:127-137), and bias + sum is written.
// Workgroup: 64 outputs (wave w: outputs 16w .. 16w + 15, the B operand, column o = lane % 16) x 16 T activation
// rows (T 16-row A tiles: 1 or 2 for batches of up to 16 or 32 rows, else 4). Lane group g = lane / 16 carries K bytes 8g .. 8g + 7 of the block in both operands;
// the four results a lane holds, D[4g + i][lane % 16], are (activation row 4g + i of the tile, its own output).
// Blocks go in groups of four: the lane's four weight scales and, per tile row 4g + i, four activation scales are
// one 16-byte load each.
struct Q8MArgs {
    const int8_t* w;
    const float* ws;
    const float* bias;
    float* y;
    int n_out;
    int in;
    int rows;
    const int8_t* q;
    const float* s;
};

typedef int i32x4m __attribute__((ext_vector_type(4)));

// LDS staging of one four-block group (128 K bytes): row r, piece g (bytes 8g .. 8g + 7 of a block) and block j sit
// at r * kQ8Row + 32 g + 8 j, so a lane's operand pieces of all four blocks are 32 contiguous bytes (two 16-byte
// reads); rows are padded to 144 bytes so the 16 rows one read instruction covers start on different banks.
constexpr int kQ8Row = 144;

__device__ __forceinline__ void q8_stage_block(uint8_t* base, int row, int j, u32x4 lo, u32x4 hi) {
    uint8_t* p = base + row * kQ8Row + 8 * j;
    *reinterpret_cast<u32x2*>(p) = u32x2{lo.x, lo.y};
    *reinterpret_cast<u32x2*>(p + 32) = u32x2{lo.z, lo.w};
    *reinterpret_cast<u32x2*>(p + 64) = u32x2{hi.x, hi.y};
    *reinterpret_cast<u32x2*>(p + 96) = u32x2{hi.z, hi.w};
}

// T: 16-row activation tiles per workgroup (1 or 2 when the whole batch has at most 16 / 32 rows, else 4).
// kW: waves per workgroup (16 outputs each): 4, or 1 for one-tile batches, so that few outputs still spread over
// every CU (each wave then stages its own 16-row activation tile).
template <int T, int kW>
__global__ __launch_bounds__(256, 2) void q8_0_mfma_kernel(const Q8MArgs a) {
    static_assert(kW == 4 || T == 1, "a one-wave workgroup stages one 16-row tile");
    __shared__ __align__(16) uint8_t la[2][16 * T * kQ8Row];  // activation tile, double-buffered
    __shared__ __align__(16) float lxs[2][16 * T * 4];         // its scales [row][block]
    __shared__ __align__(16) uint8_t lw[kW][2][16 * kQ8Row];  // each wave's weight rows, double-buffered
    const int tid = (int)threadIdx.x;
    const int wave = wave_id();
    const int lane = tid & 63;
    const int g = lane >> 4, c16 = lane & 15;
    const int o0 = (int)blockIdx.x * 16 * kW + wave * 16;  // this wave's outputs (past n_out: zeros, no store)
    const int m0 = (int)blockIdx.y * 16 * T;
    const uint32_t K = (uint32_t)a.in, nb = K / 32;
    const uint32_t wrows = (uint32_t)max(0, min(16, a.n_out - o0)), arows = (uint32_t)min(16 * T, a.rows - m0);
    const uint64_t obase = o0 < a.n_out ? (uint64_t)o0 : 0;
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.w + obase * K, wrows * K);
    const __amdgpu_buffer_rsrc_t wsr = make_rsrc(a.ws + obase * nb, wrows * nb * 4);
    const __amdgpu_buffer_rsrc_t qr = make_rsrc(a.q + (uint64_t)m0 * K, arows * K);
    const __amdgpu_buffer_rsrc_t sr = make_rsrc(a.s + (uint64_t)m0 * nb, arows * nb * 4);
    // staging assignments: thread tid < 64 T copies block (tid & 3) of activation row tid >> 2 and its scale; lane
    // copies block (lane & 3) of the wave's weight row lane >> 2
    const int ar = tid >> 2, aj = tid & 3, wrow = lane >> 2, wj = lane & 3;
    const bool astage = tid < 64 * T;  // wave-uniform
    struct Stage {
        u32x4 a0, a1, w0, w1;
        uint32_t xs;
    };
    auto fetch = [&](uint32_t b4, Stage& st) {  // past the row's blocks: the next row's bytes or zeros, unused
        if (astage) {
            const uint32_t ao = (uint32_t)ar * K + (b4 + aj) * 32;
            st.a0 = ld4(qr, ao);
            st.a1 = ld4(qr, ao + 16);
            st.xs = ld1(sr, ((uint32_t)ar * nb + b4 + aj) * 4);
        }
        const uint32_t wo = (uint32_t)wrow * K + (b4 + wj) * 32;
        st.w0 = ld4(wr, wo);
        st.w1 = ld4(wr, wo + 16);
    };
    auto stage = [&](int buf, const Stage& st) {
        if (astage) {
            q8_stage_block(la[buf], ar, aj, st.a0, st.a1);
            lxs[buf][ar * 4 + aj] = as_float(st.xs);
        }
        q8_stage_block(lw[wave][buf], wrow, wj, st.w0, st.w1);
    };
    float acc[T][4];
#pragma unroll
    for (int t = 0; t < T; t++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[t][i] = 0.0f;
    // Two groups in flight: while group k is computed from LDS, group k + 1 (fetched during group k - 1) waits in
    // registers for its LDS stores and group k + 2's loads are issued.
    Stage sa, sb;
    fetch(0, sa);
    stage(0, sa);
    if (4 < nb) fetch(4, sb);
    __syncthreads();
    int buf = 0;
    uint32_t b4 = 0;
    // next: group k + 1 (in registers); after: free. A full group (four blocks) has no per-block test, so the
    // compiler can interleave its 16 MFMAs with the fp32 tails; only the row's last group can be partial.
    auto group = [&](auto full_tag, Stage& next, Stage& after) -> bool {
        constexpr bool kFull = decltype(full_tag)::value;
        if (b4 + 8 < nb) fetch(b4 + 8, after);
        const u32x4 wsv = ld4(wsr, ((uint32_t)c16 * nb + b4) * 4);  // the lane's weight scales of the four blocks
        const uint8_t* wp = lw[wave][buf] + c16 * kQ8Row + 32 * g;
        const u32x4 wlo = *reinterpret_cast<const u32x4*>(wp), whi = *reinterpret_cast<const u32x4*>(wp + 16);
        const uint32_t bw[8] = {wlo.x, wlo.y, wlo.z, wlo.w, whi.x, whi.y, whi.z, whi.w};
#pragma unroll
        for (int t = 0; t < T; t++) {
            const uint8_t* ap = la[buf] + (16 * t + c16) * kQ8Row + 32 * g;
            const u32x4 alo = *reinterpret_cast<const u32x4*>(ap), ahi = *reinterpret_cast<const u32x4*>(ap + 16);
            const uint32_t aw[8] = {alo.x, alo.y, alo.z, alo.w, ahi.x, ahi.y, ahi.z, ahi.w};
            u32x4 xv[4];  // scales of rows 16t + 4g + i, blocks b4 .. b4 + 3
#pragma unroll
            for (int i = 0; i < 4; i++) xv[i] = *reinterpret_cast<const u32x4*>(&lxs[buf][(16 * t + 4 * g + i) * 4]);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                if (kFull || b4 + j < nb) {  // wave-uniform
                    const long aop = (long)(((uint64_t)aw[2 * j + 1] << 32) | aw[2 * j]);
                    const long bop = (long)(((uint64_t)bw[2 * j + 1] << 32) | bw[2 * j]);
                    const i32x4m d = __builtin_amdgcn_mfma_i32_16x16x32_i8(aop, bop, i32x4m{0, 0, 0, 0}, 0, 0, 0);
                    const uint32_t wsw = j == 0 ? wsv.x : j == 1 ? wsv.y : j == 2 ? wsv.z : wsv.w;
                    const float wsc = as_float(wsw);
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const uint32_t xw = j == 0 ? xv[i].x : j == 1 ? xv[i].y : j == 2 ? xv[i].z : xv[i].w;
                        // (wScale * aScale) * blockDot, then the ascending sum
                        acc[t][i] += (wsc * as_float(xw)) * (float)d[i];
                    }
                }
            }
        }
        if (b4 + 4 < nb) stage(buf ^ 1, next);
        __syncthreads();  // the other buffer is complete; this one is free for the group after next
        buf ^= 1;
        b4 += 4;
        return b4 < nb;
    };
    for (;;) {
        if (b4 + 4 > nb) {
            group(std::false_type{}, sb, sa);
            break;
        }
        if (!group(std::true_type{}, sb, sa)) break;
        if (b4 + 4 > nb) {
            group(std::false_type{}, sa, sb);
            break;
        }
        if (!group(std::true_type{}, sa, sb)) break;
    }
    const int o = o0 + c16;
    if (o < a.n_out) {
        const float bo = a.bias ? a.bias[o] : 0.0f;
#pragma unroll
        for (int t = 0; t < T; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int m = m0 + 16 * t + 4 * g + i;
                if (m < a.rows) a.y[(size_t)m * a.n_out + o] = a.bias ? bo + acc[t][i] : acc[t][i];
            }
    }
}

// ------------------------------------------------------------------------------------------ per-head Q8_0 Wo on MFMA
// The attention output projection of prefill rows with per-head Q8_0 Wo (RT/CachedMultiHeadAttention.cs:600-614,
// :689-710: BatchedQuantProjection.Dispatch of each head's attention rows through its own Wo_h [d_model][head_dim],
// then TensorPrimitives.Add into the output, heads ascending, the output starting as the attention bias or zero). The
// kernel above with the contraction walked head by head: a group of up to four blocks never crosses a head, so its
// weight rows come from one head's planes (a wave-uniform resource per group); each head's blocks are summed from +0
// in block order (the head's Q8 Dot), and at the head's last group that value is added to the running output, which
// starts as bias-or-zero. Every (row, output) therefore gets ((bias + head 0) + head 1) + ... bit for bit.
struct Q8HMArgs {
    const int8_t* wq[kHeadsMax];
    const float* ws[kHeadsMax];
    const float* bias;
    float* y;
    int n_out;     // d_model
    int n_heads;
    int head_dim;
    int rows;
    const int8_t* q;  // Q8_0 activation [rows][n_heads * head_dim]
    const float* s;
};

// The 64 x 64 tile (T = 4) of the two kernels above on eight-wave workgroups with the operands staged by LDS DMA:
// wave w takes outputs 16 (w % 4) .. + 15 and activation tiles 2 (w / 4) and 2 (w / 4) + 1, so a launch of one
// 64 x 64 tile per workgroup keeps four waves per SIMD instead of two. Per group of four blocks the activation rows
// (128 bytes each), their scales, the workgroup's 64 weight rows and their scales are DMA'd (`buffer_load ... lds`)
// into one of two slots while the other slot is computed; each slot is its own set of LDS objects, so the compiler's
// wait before reading one slot leaves the DMA into the other in flight. A row's eight 16-byte pieces sit
// XOR-swizzled by row % 8 (physical piece p holds logical piece p ^ (row % 8)) against LDS bank conflicts. Per
// (row, output) the block values are added in ascending block order from +0; kHeads: the contraction walks the heads
// (a group never crosses a head, its weight rows come from the head's planes) and each head's value is added to the
// running output, which starts as bias or zero, in ascending head order, as q8_0_heads_mfma_kernel does.
constexpr int kQ8DmaWaves = 8;

template <bool kHeads, class Args>
__global__ __launch_bounds__(64 * kQ8DmaWaves, 2) void q8_0_mfma_dma_kernel(const Args a) {
    __shared__ __align__(16) uint8_t act0[64 * 128], act1[64 * 128];  // activation rows of the group
    __shared__ __align__(16) uint8_t wt0[64 * 128], wt1[64 * 128];    // weight rows of the group
    __shared__ __align__(16) float xs0[64 * 4], xs1[64 * 4];          // activation scales [row][block]
    __shared__ __align__(16) float ws0[64 * 4], ws1[64 * 4];          // weight scales [row][block]
    const int wave = wave_id();
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4, c16 = lane & 15;
    const int ow = wave & 3, ah = wave >> 2;
    const int obase = (int)blockIdx.x * 64;
    const int m0 = (int)blockIdx.y * 64;
    uint32_t K, wk;  // activation row length; weight row length (the head dimension for per-head planes)
    if constexpr (kHeads) {
        K = (uint32_t)a.n_heads * (uint32_t)a.head_dim;
        wk = (uint32_t)a.head_dim;
    } else {
        K = (uint32_t)a.in;
        wk = K;
    }
    const uint32_t nb = K / 32, wnb = wk / 32;
    const int gph = (int)(wnb + 3) / 4;              // groups per weight plane (per head)
    int ng = gph;  // groups in the contraction
    if constexpr (kHeads) ng = a.n_heads * gph;
    // (readfirstlane: the compiler otherwise clamps these in vector registers and loops each DMA over lanes)
    const uint32_t wrows = (uint32_t)__builtin_amdgcn_readfirstlane(max(0, min(64, a.n_out - obase)));
    const uint32_t arows = (uint32_t)__builtin_amdgcn_readfirstlane(min(64, a.rows - m0));
    // resources end with the tile's last row: rows past the matrix or the batch read zeros
    const __amdgpu_buffer_rsrc_t qr = make_rsrc(a.q + (uint64_t)m0 * K, arows * K);
    const __amdgpu_buffer_rsrc_t sr = make_rsrc(a.s + (uint64_t)m0 * nb, arows * nb * 4);
    // DMA sources. Wave w moves rows 8w .. 8w + 7 of the activation and of the weights (1 KiB each: lane L writes
    // physical piece L % 8 of row 8w + L / 8), and the scales of rows 16 (w % 4) .. + 15 (lane L: row + L / 4, block
    // L % 4) of the activation (w < 4) or of the weights (w >= 4).
    const uint32_t prow = 8u * (uint32_t)wave + ((uint32_t)lane >> 3);
    const uint32_t pcol = 16u * (((uint32_t)lane & 7u) ^ (prow & 7u));
    const uint32_t srow = 16u * (uint32_t)ow + ((uint32_t)lane >> 2), sblk = (uint32_t)lane & 3u;
    const bool scale_act = wave < 4;  // wave-uniform
    // group gi: its head, its first block in the weight plane and in the activation row, its block count
    struct Grp {
        int h;
        uint32_t lb0, b0;
        int nblk;
    };
    auto group_of = [&](int gi) -> Grp {
        const int h = kHeads ? (gph == 1 ? gi : gi / gph) : 0;
        const uint32_t lb0 = (uint32_t)(gi - h * gph) * 4u;
        return Grp{h, lb0, (uint32_t)h * wnb + lb0, min(4, (int)(wnb - lb0))};
    };
    auto stage = [&](auto sc, int gi) {
        constexpr int S = decltype(sc)::value;
        uint8_t* const act = S ? act1 : act0;
        uint8_t* const wt = S ? wt1 : wt0;
        float* const xs = S ? xs1 : xs0;
        float* const ws = S ? ws1 : ws0;
        const Grp gr = group_of(gi);
        const int8_t* wplane;
        const float* splane;
        if constexpr (kHeads) {
            wplane = a.wq[gr.h];
            splane = a.ws[gr.h];
        } else {
            wplane = a.w;
            splane = a.ws;
        }
        // blocks past the plane's last (a short group) read other bytes or zeros, unused
        const __amdgpu_buffer_rsrc_t wr = make_rsrc(wplane + (uint64_t)obase * wk, wrows * wk);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(qr, (__attribute__((address_space(3))) void*)&act[1024 * wave], 16,
                                                 (int)(prow * K + gr.b0 * 32u + pcol), 0, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, (__attribute__((address_space(3))) void*)&wt[1024 * wave], 16,
                                                 (int)(prow * wk + gr.lb0 * 32u + pcol), 0, 0, 0);
        if (scale_act) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(sr, (__attribute__((address_space(3))) void*)&xs[64 * ow], 4,
                                                     (int)((srow * nb + gr.b0 + sblk) * 4u), 0, 0, 0);
        } else {
            const __amdgpu_buffer_rsrc_t wsr = make_rsrc(splane + (uint64_t)obase * wnb, wrows * wnb * 4);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(wsr, (__attribute__((address_space(3))) void*)&ws[64 * ow], 4,
                                                     (int)((srow * wnb + gr.lb0 + sblk) * 4u), 0, 0, 0);
        }
    };
    // byte offset of this lane's 8 bytes of block j in row `row` (lane group g holds K bytes 8g .. 8g + 7 of a block)
    auto piece = [&](uint32_t row, int j) -> uint32_t {
        return row * 128u + (((2u * (uint32_t)j + ((uint32_t)g >> 1)) ^ (row & 7u)) * 16u) + 8u * ((uint32_t)g & 1u);
    };
    const int o = obase + 16 * ow + c16;
    float acc[2][4], tot[2][4];
    {
        const float start = (kHeads && a.bias && o < a.n_out) ? a.bias[o] : 0.0f;  // per-head: bias or zero
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                acc[t][i] = 0.0f;
                tot[t][i] = start;
            }
    }
    auto compute = [&](auto sc, int gi) {
        constexpr int S = decltype(sc)::value;
        const uint8_t* const act = S ? act1 : act0;
        const uint8_t* const wt = S ? wt1 : wt0;
        const float* const xs = S ? xs1 : xs0;
        const float* const ws = S ? ws1 : ws0;
        const Grp gr = group_of(gi);  // nblk < 4 only for a plane's short last group (wave-uniform)
        const uint32_t wrow = 16u * (uint32_t)ow + (uint32_t)c16;
        const u32x4 wsv = *reinterpret_cast<const u32x4*>(&ws[wrow * 4]);  // the lane's weight row, blocks 0 .. 3
        u32x2 bw[4];
#pragma unroll
        for (int j = 0; j < 4; j++) bw[j] = *reinterpret_cast<const u32x2*>(wt + piece(wrow, j));
#pragma unroll
        for (int tt = 0; tt < 2; tt++) {
            const uint32_t t = 2u * (uint32_t)ah + (uint32_t)tt;
            u32x2 aw[4];
#pragma unroll
            for (int j = 0; j < 4; j++) aw[j] = *reinterpret_cast<const u32x2*>(act + piece(16u * t + (uint32_t)c16, j));
            u32x4 xv[4];  // scales of activation rows 16t + 4g + i, blocks 0 .. 3
#pragma unroll
            for (int i = 0; i < 4; i++) xv[i] = *reinterpret_cast<const u32x4*>(&xs[(16u * t + 4u * g + i) * 4u]);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                if (j < gr.nblk) {
                    const long aop = (long)(((uint64_t)aw[j].y << 32) | aw[j].x);
                    const long bop = (long)(((uint64_t)bw[j].y << 32) | bw[j].x);
                    const i32x4m d = __builtin_amdgcn_mfma_i32_16x16x32_i8(aop, bop, i32x4m{0, 0, 0, 0}, 0, 0, 0);
                    const float wsc = as_float(j == 0 ? wsv.x : j == 1 ? wsv.y : j == 2 ? wsv.z : wsv.w);
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const uint32_t xw = j == 0 ? xv[i].x : j == 1 ? xv[i].y : j == 2 ? xv[i].z : xv[i].w;
                        // (wScale * aScale) * blockDot, then the ascending sum
                        acc[tt][i] += (wsc * as_float(xw)) * (float)d[i];
                    }
                }
            }
        }
        if constexpr (kHeads) {
            if (gr.lb0 + 4u >= wnb) {  // the head's last group: output += head value
#pragma unroll
                for (int tt = 0; tt < 2; tt++)
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        tot[tt][i] = tot[tt][i] + acc[tt][i];
                        acc[tt][i] = 0.0f;
                    }
            }
        }
    };
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    stage(S0{}, 0);
    for (int k = 0; k < ng; k += 2) {
        __builtin_amdgcn_s_waitcnt(0);  // this wave's DMAs of group k have landed
        __syncthreads();                // every wave's; and slot 1 is no longer read
        if (k + 1 < ng) stage(S1{}, k + 1);
        compute(S0{}, k);
        if (k + 1 >= ng) break;
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (k + 2 < ng) stage(S0{}, k + 2);
        compute(S1{}, k + 1);
    }
    if (o < a.n_out) {
        const float bo = (!kHeads && a.bias) ? a.bias[o] : 0.0f;
#pragma unroll
        for (int tt = 0; tt < 2; tt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int m = m0 + 16 * (2 * ah + tt) + 4 * g + i;
                if (m >= a.rows) continue;
                float v;
                if constexpr (kHeads) {
                    v = tot[tt][i];
                } else {
                    v = a.bias ? bo + acc[tt][i] : acc[tt][i];  // bias[o] + sum; no add at all without a bias
                }
                a.y[(size_t)m * a.n_out + o] = v;
            }
    }
}

template <int T, int kW>
__global__ __launch_bounds__(256, 2) void q8_0_heads_mfma_kernel(const Q8HMArgs a) {
    static_assert(kW == 4 || T == 1, "a one-wave workgroup stages one 16-row tile");
    __shared__ __align__(16) uint8_t la[2][16 * T * kQ8Row];
    __shared__ __align__(16) float lxs[2][16 * T * 4];
    __shared__ __align__(16) uint8_t lw[kW][2][16 * kQ8Row];
    const int tid = (int)threadIdx.x;
    const int wave = wave_id();
    const int lane = tid & 63;
    const int g = lane >> 4, c16 = lane & 15;
    const int o0 = (int)blockIdx.x * 16 * kW + wave * 16;
    const int m0 = (int)blockIdx.y * 16 * T;
    const uint32_t hd = (uint32_t)a.head_dim, nbh = hd / 32;
    const uint32_t K = (uint32_t)a.n_heads * hd, nb = K / 32;
    const int gph = (int)(nbh + 3) / 4;  // groups per head
    const int G = a.n_heads * gph;
    const uint32_t wrows = (uint32_t)max(0, min(16, a.n_out - o0)), arows = (uint32_t)min(16 * T, a.rows - m0);
    const uint64_t obase = o0 < a.n_out ? (uint64_t)o0 : 0;
    const __amdgpu_buffer_rsrc_t qr = make_rsrc(a.q + (uint64_t)m0 * K, arows * K);
    const __amdgpu_buffer_rsrc_t sr = make_rsrc(a.s + (uint64_t)m0 * nb, arows * nb * 4);
    const int ar = tid >> 2, aj = tid & 3, wrow = lane >> 2, wj = lane & 3;
    const bool astage = tid < 64 * T;
    struct Stage {
        u32x4 a0, a1, w0, w1;
        uint32_t xs;
    };
    auto head_of = [&](int gi) { return gph == 1 ? gi : gi / gph; };
    auto fetch = [&](int gi, Stage& st) {  // blocks past the head's last: other bytes or zeros, unused
        const int h = head_of(gi);
        const uint32_t lb0 = (uint32_t)(gi - h * gph) * 4;
        const uint32_t b0 = (uint32_t)h * nbh + lb0;  // the group's first block of the activation row
        if (astage) {
            const uint32_t ao = (uint32_t)ar * K + (b0 + aj) * 32;
            st.a0 = ld4(qr, ao);
            st.a1 = ld4(qr, ao + 16);
            st.xs = ld1(sr, ((uint32_t)ar * nb + b0 + aj) * 4);
        }
        const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.wq[h] + obase * hd, wrows * hd);
        const uint32_t wo = (uint32_t)wrow * hd + (lb0 + wj) * 32;
        st.w0 = ld4(wr, wo);
        st.w1 = ld4(wr, wo + 16);
    };
    auto stage = [&](int buf, const Stage& st) {
        if (astage) {
            q8_stage_block(la[buf], ar, aj, st.a0, st.a1);
            lxs[buf][ar * 4 + aj] = as_float(st.xs);
        }
        q8_stage_block(lw[wave][buf], wrow, wj, st.w0, st.w1);
    };
    const int o = o0 + c16;
    const float start = (a.bias && o < a.n_out) ? a.bias[o] : 0.0f;  // the output starts as bias or zero
    float tot[T][4], hacc[T][4];
#pragma unroll
    for (int t = 0; t < T; t++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            tot[t][i] = start;
            hacc[t][i] = 0.0f;
        }
    Stage sa, sb;
    fetch(0, sa);
    stage(0, sa);
    if (1 < G) fetch(1, sb);
    __syncthreads();
    int buf = 0;
    int gi = 0;
    auto group = [&](auto full_tag, Stage& next, Stage& after) -> bool {
        constexpr bool kFull = decltype(full_tag)::value;
        if (gi + 2 < G) fetch(gi + 2, after);
        const int h = head_of(gi);
        const uint32_t lb0 = (uint32_t)(gi - h * gph) * 4;
        const uint32_t nblk = min(4u, nbh - lb0);
        const __amdgpu_buffer_rsrc_t wsr = make_rsrc(a.ws[h] + obase * nbh, wrows * nbh * 4);
        const u32x4 wsv = ld4(wsr, ((uint32_t)c16 * nbh + lb0) * 4);
        const uint8_t* wp = lw[wave][buf] + c16 * kQ8Row + 32 * g;
        const u32x4 wlo = *reinterpret_cast<const u32x4*>(wp), whi = *reinterpret_cast<const u32x4*>(wp + 16);
        const uint32_t bw[8] = {wlo.x, wlo.y, wlo.z, wlo.w, whi.x, whi.y, whi.z, whi.w};
#pragma unroll
        for (int t = 0; t < T; t++) {
            const uint8_t* ap = la[buf] + (16 * t + c16) * kQ8Row + 32 * g;
            const u32x4 alo = *reinterpret_cast<const u32x4*>(ap), ahi = *reinterpret_cast<const u32x4*>(ap + 16);
            const uint32_t aw[8] = {alo.x, alo.y, alo.z, alo.w, ahi.x, ahi.y, ahi.z, ahi.w};
            u32x4 xv[4];
#pragma unroll
            for (int i = 0; i < 4; i++) xv[i] = *reinterpret_cast<const u32x4*>(&lxs[buf][(16 * t + 4 * g + i) * 4]);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                if (kFull || (uint32_t)j < nblk) {  // wave-uniform
                    const long aop = (long)(((uint64_t)aw[2 * j + 1] << 32) | aw[2 * j]);
                    const long bop = (long)(((uint64_t)bw[2 * j + 1] << 32) | bw[2 * j]);
                    const i32x4m d = __builtin_amdgcn_mfma_i32_16x16x32_i8(aop, bop, i32x4m{0, 0, 0, 0}, 0, 0, 0);
                    const uint32_t wsw = j == 0 ? wsv.x : j == 1 ? wsv.y : j == 2 ? wsv.z : wsv.w;
                    const float wsc = as_float(wsw);
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const uint32_t xw = j == 0 ? xv[i].x : j == 1 ? xv[i].y : j == 2 ? xv[i].z : xv[i].w;
                        hacc[t][i] += (wsc * as_float(xw)) * (float)d[i];
                    }
                }
            }
        }
        if (lb0 + 4 >= nbh) {  // the head's last group: output += head value
#pragma unroll
            for (int t = 0; t < T; t++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    tot[t][i] = tot[t][i] + hacc[t][i];
                    hacc[t][i] = 0.0f;
                }
        }
        if (gi + 1 < G) stage(buf ^ 1, next);
        __syncthreads();
        buf ^= 1;
        gi += 1;
        return gi < G;
    };
    auto step = [&](Stage& next, Stage& after) -> bool {
        const int h = head_of(gi);
        const uint32_t lb0 = (uint32_t)(gi - h * gph) * 4;
        return nbh - lb0 >= 4 ? group(std::true_type{}, next, after) : group(std::false_type{}, next, after);
    };
    for (;;) {
        if (!step(sb, sa)) break;
        if (!step(sa, sb)) break;
    }
    if (o < a.n_out) {
#pragma unroll
        for (int t = 0; t < T; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int m = m0 + 16 * t + 4 * g + i;
                if (m < a.rows) a.y[(size_t)m * a.n_out + o] = tot[t][i];
            }
    }
}

bool q8_0_heads_mfma_supported(int n_heads, int head_dim, int rows) {
    const uint64_t K = (uint64_t)n_heads * head_dim;
    return n_heads >= 1 && n_heads <= kHeadsMax && head_dim >= 32 && head_dim % 32 == 0 && rows >= 1 &&
           K * 64 < (1ull << 31) && K * (uint64_t)rows < (1ull << 31);
}

// Batches past 16 rows take the eight-wave LDS-DMA kernel (MI355X, Q8_0 4096x4096 with its quantise launch, us,
// register-staged four-wave kernel / DMA kernel: 17-32 rows 38.7-39.2 / 30.4-30.9, 512 rows 58.7-59.7 / 52.5-52.9;
// per-head Llama-3-8B Wo at 32 / 64 / 512 rows 46.1 / 64.3 / 73.7 / 35.9 / 36.3 / 54.3). OVFQ_Q8_MFMA_DMA=0 keeps
// the register-staged kernels, for measurements.
static bool q8_mfma_dma() {
    static const bool on = [] {
        const char* v = getenv("OVFQ_Q8_MFMA_DMA");
        return !(v && *v == '0');
    }();
    return on;
}

hipError_t launch_q8_0_heads_mfma(const int8_t* const* wq, const float* const* ws, int n_heads, int head_dim,
                                  int d_model, int rows, const float* bias, ActQ act, float* y, hipStream_t st) {
    if (!q8_0_heads_mfma_supported(n_heads, head_dim, rows) || !act.q || !act.s) return hipErrorInvalidValue;
    Q8HMArgs ha{};
    for (int h = 0; h < n_heads; h++) {
        ha.wq[h] = wq[h];
        ha.ws[h] = ws[h];
    }
    ha.bias = bias;
    ha.y = y;
    ha.n_out = d_model;
    ha.n_heads = n_heads;
    ha.head_dim = head_dim;
    ha.rows = rows;
    ha.q = act.q;
    ha.s = act.s;
    const int T = rows <= 16 ? 1 : rows <= 32 ? 2 : 4;
    const dim3 grid4((d_model + 63) / 64, (rows + 16 * T - 1) / (16 * T));
    if (T == 1)
        hipLaunchKernelGGL((q8_0_heads_mfma_kernel<1, 1>), dim3((d_model + 15) / 16, 1), dim3(64), 0, st, ha);
    else if (q8_mfma_dma())
        hipLaunchKernelGGL((q8_0_mfma_dma_kernel<true, Q8HMArgs>), dim3((d_model + 63) / 64, (rows + 63) / 64),
                           dim3(64 * kQ8DmaWaves), 0, st, ha);
    else if (T == 2)
        hipLaunchKernelGGL((q8_0_heads_mfma_kernel<2, 4>), grid4, dim3(256), 0, st, ha);
    else
        hipLaunchKernelGGL((q8_0_heads_mfma_kernel<4, 4>), grid4, dim3(256), 0, st, ha);
    return hipGetLastError();
}

bool q8_0_mfma_supported(int in, int rows) {
    // 32-bit resource offsets: 64 activation rows and 16 weight rows of K bytes, and the whole activation
    return in % 32 == 0 && (uint64_t)in * 64 < (1ull << 31) && (uint64_t)in * (uint64_t)rows < (1ull << 31);
}

hipError_t launch_project_q8_0_mfma(const ProjJob* jobs, int njobs, int in, int rows, ActQ act, hipStream_t st) {
    for (int i = 0; i < njobs; i++) {
        Q8MArgs ma{};
        ma.w = reinterpret_cast<const int8_t*>(jobs[i].w);
        ma.ws = jobs[i].ws;
        ma.bias = jobs[i].bias;
        ma.y = jobs[i].y;
        ma.n_out = jobs[i].n_rows;
        ma.in = in;
        ma.rows = rows;
        ma.q = act.q;
        ma.s = act.s;
        const int T = rows <= 16 ? 1 : rows <= 32 ? 2 : 4;
        const dim3 grid4((jobs[i].n_rows + 63) / 64, (rows + 16 * T - 1) / (16 * T));
        if (T == 1)
            hipLaunchKernelGGL((q8_0_mfma_kernel<1, 1>), dim3((jobs[i].n_rows + 15) / 16, 1), dim3(64), 0, st, ma);
        else if (q8_mfma_dma())
            hipLaunchKernelGGL((q8_0_mfma_dma_kernel<false, Q8MArgs>), dim3((jobs[i].n_rows + 63) / 64, (rows + 63) / 64),
                               dim3(64 * kQ8DmaWaves), 0, st, ma);
        else if (T == 2)
            hipLaunchKernelGGL((q8_0_mfma_kernel<2, 4>), grid4, dim3(256), 0, st, ma);
        else
            hipLaunchKernelGGL((q8_0_mfma_kernel<4, 4>), grid4, dim3(256), 0, st, ma);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace ovfq
