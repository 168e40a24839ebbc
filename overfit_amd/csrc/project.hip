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

// ------------------------------------------------------------------------------------------ Q8_0 on int8 MFMA
// Q8DotKernel.ProjectBatched (RT/Q8DotKernel.cs:352-445) for several activation rows. The weights are int8 already,
// so each 32-element block is one v_mfma_i32_16x16x32_i8 per 16 x 16 (activation row, output) tile, giving the
// block's exact int32 dot; the reference's tail (wScale * aScale) * dot is then added per (row, output) in
// ascending block order from +0 (Dot, RT/Q8DotKernel.cs:127-137), and bias + sum is written.
// Workgroup: 64 outputs (wave w: outputs 16w .. 16w + 15, the B operand, column o = lane % 16) x 64 activation
// rows (four 16-row A tiles). Lane group g = lane / 16 carries K bytes 8g .. 8g + 7 of the block in both operands;
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

__global__ __launch_bounds__(256) void q8_0_mfma_kernel(const Q8MArgs a) {
    const int wave = wave_id();
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4, c16 = lane & 15;
    const int o0 = (int)blockIdx.x * 64 + wave * 16;
    const int m0 = (int)blockIdx.y * 64;
    if (o0 >= a.n_out) return;  // wave-uniform; the kernel has no barrier
    const uint32_t K = (uint32_t)a.in, nb = K / 32;
    // Resources over this wave's weight rows and the workgroup's activation rows: rows past the end read zeros.
    const uint32_t wrows = (uint32_t)min(16, a.n_out - o0), arows = (uint32_t)min(64, a.rows - m0);
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.w + (uint64_t)o0 * K, wrows * K);
    const __amdgpu_buffer_rsrc_t wsr = make_rsrc(a.ws + (uint64_t)o0 * nb, wrows * nb * 4);
    const __amdgpu_buffer_rsrc_t qr = make_rsrc(a.q + (uint64_t)m0 * K, arows * K);
    const __amdgpu_buffer_rsrc_t sr = make_rsrc(a.s + (uint64_t)m0 * nb, arows * nb * 4);
    const uint32_t woff = (uint32_t)c16 * K + 8u * g;
    float acc[4][4];
#pragma unroll
    for (int t = 0; t < 4; t++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[t][i] = 0.0f;
    for (uint32_t b4 = 0; b4 < nb; b4 += 4) {
        // scales of blocks b4 .. b4 + 3 (past the row's last block: unused)
        const u32x4 wsv = ld4(wsr, ((uint32_t)c16 * nb + b4) * 4);
        u32x4 xs[4][4];
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) xs[t][i] = ld4(sr, ((uint32_t)(16 * t + 4 * g + i) * nb + b4) * 4);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t b = b4 + j;
            if (b < nb) {  // wave-uniform
                const u32x2 wv = ld2(wr, woff + 32 * b);
                const long bop = (long)(((uint64_t)wv.y << 32) | wv.x);
                const uint32_t wsw = j == 0 ? wsv.x : j == 1 ? wsv.y : j == 2 ? wsv.z : wsv.w;
                const float wsc = as_float(wsw);
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    const u32x2 av = ld2(qr, (uint32_t)(16 * t + c16) * K + 32 * b + 8u * g);
                    const long aop = (long)(((uint64_t)av.y << 32) | av.x);
                    const i32x4m d = __builtin_amdgcn_mfma_i32_16x16x32_i8(aop, bop, i32x4m{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const u32x4 xv = xs[t][i];
                        const uint32_t xw = j == 0 ? xv.x : j == 1 ? xv.y : j == 2 ? xv.z : xv.w;
                        // (wScale * aScale) * blockDot, then the ascending sum
                        acc[t][i] += (wsc * as_float(xw)) * (float)d[i];
                    }
                }
            }
        }
    }
    const int o = o0 + c16;
    if (o < a.n_out) {
        const float bo = a.bias ? a.bias[o] : 0.0f;
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int m = m0 + 16 * t + 4 * g + i;
                if (m < a.rows) a.y[(size_t)m * a.n_out + o] = a.bias ? bo + acc[t][i] : acc[t][i];
            }
    }
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
        const dim3 grid((jobs[i].n_rows + 63) / 64, (rows + 63) / 64);
        hipLaunchKernelGGL(q8_0_mfma_kernel, grid, dim3(256), 0, st, ma);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace ovfq
