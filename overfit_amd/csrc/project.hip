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
    // Q4KDotKernel.Dot (RT/Q4KDotKernel.cs:216-256) for one block; valid in every lane of the quad.
    __device__ __forceinline__ static float dot(const W& w, const A& a, int t) {
        // UnpackQ4_KScalesMins (LD/GgmlDequant.cs:49-77) for sub-blocks j = 2t, 2t+1: bytes j&3 of the three
        // packed words, two bytes at a time.
        const uint32_t sh = (t & 1) * 16;
        const uint32_t A16 = (w.h.y >> sh) & 0xffffu, B16 = (w.h.z >> sh) & 0xffffu, C16 = (w.h.w >> sh) & 0xffffu;
        const bool upper = t >= 2;
        const uint32_t sc01 = upper ? ((C16 & 0x0f0fu) | ((A16 >> 2) & 0x3030u)) : (A16 & 0x3f3fu);
        const uint32_t m01 = upper ? (((C16 >> 4) & 0x0f0fu) | ((B16 >> 2) & 0x3030u)) : (B16 & 0x3f3fu);
        const uint32_t qw[8] = {w.a.x, w.a.y, w.a.z, w.a.w, w.b.x, w.b.y, w.b.z, w.b.w};
        const uint32_t aw[16] = {a.q[0].x, a.q[0].y, a.q[0].z, a.q[0].w, a.q[1].x, a.q[1].y, a.q[1].z, a.q[1].w,
                                 a.q[2].x, a.q[2].y, a.q[2].z, a.q[2].w, a.q[3].x, a.q[3].y, a.q[3].z, a.q[3].w};
        int dlo = 0, dhi = 0;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            dlo = sdot4(qw[k] & 0x0f0f0f0fu, aw[k], dlo);
            dhi = sdot4((qw[k] >> 4) & 0x0f0f0f0fu, aw[8 + k], dhi);
        }
        int main_acc = (int)(sc01 & 0xffu) * dlo + (int)(sc01 >> 8) * dhi;
        int min_acc = sdot2_k(a.bs.x, (int)(m01 & 0xffu), 0);
        min_acc = sdot2_k(a.bs.y, (int)(m01 >> 8), min_acc);
        main_acc = quad_sum(main_acc);
        min_acc = quad_sum(min_acc);
        const float d = half_lo(w.h.x), dmin = half_hi(w.h.x);
        // q8Scale * (d * mainAcc - dmin * minAcc)
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
        // unsignedDot - 32 * bsumTerm, exact in int32 (|.| < 2^28).
        int part = s1 * (d1 - 32 * b1) + s2 * (d2 - 32 * b2) + s3 * (d3 - 32 * b3) + s4 * (d4 - 32 * b4);
        part = quad_sum(part);
        const float d = half_lo(w.d);
        // d * q8Scale * mainAcc
        return d * a.s * (float)part;
    }
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

}  // namespace ovfq
