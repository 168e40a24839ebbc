// rows.hip — small-batch (2 <= M < 32) and grouped-expert Q4_K / Q6_K projections.
//
// The batched projections of a few activation rows (ProjectBatched / ProjectBatchedWeightStationary,
// RT/Q4KDotKernel.cs:681-955, RT/Q6KDotKernel.cs:403-510) and the per-expert batched SwiGLU of the routed MoE
// (MoeFeedForwardBlock.DecodeBatched, RT/MoeFeedForwardBlock.cs:140-241) are weight-streaming problems: each
// weight byte is used by only a handful of rows, so the kernel is the decode GEMV's (persistent waves walking
// (R weight rows x 16 super-blocks) items with the next item's loads in flight) with MB activation rows staged
// in LDS instead of one. A weight block is unpacked once and dotted with every staged row; per (row, block) the
// fp32 value is the reference's Dot, and each output's block sum runs in ascending block order in one lane, so
// results are bit-identical to the reference's batched kernels.
//
// Grouping: grid.y is the expert. Expert e owns pairs [expert_off[e], expert_off[e+1]) of a pair list; pair p
// reads activation row pair_row[p] and writes output row p. Without a pair list the launch is one expert whose
// pairs are the activation rows 0..rows-1. An expert with more than MB pairs is processed in passes of MB rows
// (the weights are streamed once per pass).
#include <cstdlib>

#include "kquant_blocks.h"
#include "ovfq_device.h"
#include "ovfq_launch.h"

namespace ovfq {

struct RArgs {
    const uint8_t* w0[kMaxExperts];  // first matrix of each expert (gate, or the only one)
    const uint8_t* w1[kMaxExperts];  // second matrix (up), when nmat == 2
    const float* bias0;              // only without a pair list
    const float* bias1;
    float* y0;  // [pairs][n_rows]
    float* y1;
    int n_rows;
    int spr;
    int groups;  // row groups of one matrix
    int nmat;
    int rows;                // pairs of the single expert when expert_off == NULL
    const int* expert_off;   // [experts + 1] or NULL
    const int* pair_row;     // [pairs] or NULL (identity)
    const int8_t* q;         // Q8_K activation rows
    const float* s;
    const int16_t* b;
};

constexpr int kRowsMaxSpr = 64;

template <class F, int R, int MB>
__global__ __launch_bounds__(256) void kquant_rows_kernel(const RArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int spr = a.spr;
    const int slot_bytes = spr * (kLdsSlot + 36);  // quants, bsums, scale of one activation row
    float* red = reinterpret_cast<float*>(smem + ((MB * slot_bytes + 15) & ~15));
    const int wave = wave_id();
    const int lane = threadIdx.x & 63;
    const int q = lane >> 2, t = lane & 3;
    const int nchunks = (spr + 15) >> 4;
    const int stride = gridDim.x * 4;
    const int total = a.groups * a.nmat;
    const uint32_t row_bytes = (uint32_t)spr * F::kBytes;
    const uint32_t K = (uint32_t)spr * kQK;
    float* rw = red + wave * (R * MB) * 17;

    const int e = blockIdx.y;
    const int pbeg = a.expert_off ? a.expert_off[e] : 0;
    const int cnt = a.expert_off ? a.expert_off[e + 1] - pbeg : a.rows;
    if (cnt <= 0) return;  // uniform over the workgroup

    struct Item {
        typename F::W w[R];
        uint32_t bias;
    };
    // matrix and first row of row group g (wave-uniform)
    auto locate = [&](int g, int& mat, int& row0) {
        mat = g >= a.groups ? 1 : 0;
        row0 = (g - mat * a.groups) * R;
    };
    auto load_item = [&](int g, int c, bool valid, Item& it) {
        int mat, row0;
        locate(valid ? g : 0, mat, row0);
        const uint8_t* w = mat ? a.w1[e] : a.w0[e];
        const uint64_t base_off = (uint64_t)row0 * row_bytes;
        const uint64_t al = base_off & ~3ull;  // Q6_K rows are only 2-byte aligned
        const uint32_t extra = (uint32_t)(base_off - al);
        const __amdgpu_buffer_rsrc_t wr =
            make_rsrc(w + al, valid ? rsrc_bytes((uint64_t)a.n_rows * row_bytes, al) : 0u);
        const uint32_t sb = (uint32_t)(c * 16 + q);
#pragma unroll
        for (int r = 0; r < R; r++) it.w[r] = F::load_w(wr, extra + r * row_bytes + sb * F::kBytes, t);
        const float* bias = mat ? a.bias1 : a.bias0;
        const bool want_bias = valid && bias != nullptr && c == nchunks - 1;
        const __amdgpu_buffer_rsrc_t bsr = make_rsrc(bias, want_bias ? (uint32_t)a.n_rows * 4 : 0u);
        it.bias = ld1(bsr, (uint32_t)(row0 + lane % R) * 4);
    };

    for (int m0 = 0; m0 < cnt; m0 += MB) {
        const int mb = min(MB, cnt - m0);
        // Stage rows m0..m0+mb-1 (absent rows read as zeros): wave w takes super-blocks 4w..4w+3 of each
        // 16-block pass, one per 16-lane row; lane l16 moves bsum group l16 (16 quants) of its block.
        {
            const int l16 = lane & 15, rr = lane >> 4;
            const int pos = F::lds_pos(16 * l16);
#pragma unroll
            for (int m = 0; m < MB; m++) {
                const int p = pbeg + m0 + m;
                const bool have = m < mb;
                const int arow = have ? (a.pair_row ? a.pair_row[p] : p) : 0;
                const __amdgpu_buffer_rsrc_t qr = make_rsrc(a.q + (uint64_t)arow * K, have ? K : 0u);
                const __amdgpu_buffer_rsrc_t br = make_rsrc(a.b + (uint64_t)arow * spr * 16, have ? spr * 32u : 0u);
                const __amdgpu_buffer_rsrc_t sr = make_rsrc(a.s + (uint64_t)arow * spr, have ? spr * 4u : 0u);
                uint8_t* lq = smem + m * slot_bytes;
                int16_t* lb = reinterpret_cast<int16_t*>(lq + spr * kLdsSlot);
                float* ls = reinterpret_cast<float*>(lq + spr * (kLdsSlot + 32));
                for (int p16 = 0; p16 < spr; p16 += 16) {
                    const int sb = p16 + wave * 4 + rr;
                    const u32x4 qv = ld4(qr, (uint32_t)sb * kQK + l16 * 16);
                    const uint32_t bv =
                        __builtin_amdgcn_raw_buffer_load_b16(br, (int)((uint32_t)sb * 32 + l16 * 2), 0, 0);
                    const uint32_t sv = ld1(sr, (uint32_t)sb * 4);
                    if (sb < spr) {
                        *reinterpret_cast<u32x4*>(lq + sb * kLdsSlot + pos) = qv;
                        lb[sb * 16 + l16] = (int16_t)bv;
                        if (l16 == 0) ls[sb] = as_float(sv);
                    }
                }
            }
        }
        __syncthreads();

        int g = blockIdx.x * 4 + wave;
        int c = 0;
        if (g < total) {
            Item ia, ib;
            load_item(g, 0, true, ia);
            float acc = 0.0f;
            int a_chunk = -1;
            typename F::A av[MB];
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
                if (c != a_chunk) {
#pragma unroll
                    for (int m = 0; m < MB; m++) {
                        const uint8_t* lq = smem + m * slot_bytes;
                        av[m] = F::load_a_lds(lq, reinterpret_cast<const int16_t*>(lq + spr * kLdsSlot),
                                              reinterpret_cast<const float*>(lq + spr * (kLdsSlot + 32)),
                                              live ? sb : 0, t);
                    }
                    a_chunk = c;
                }
#pragma unroll
                for (int r = 0; r < R; r++)
#pragma unroll
                    for (int m = 0; m < MB; m++) {
                        const float v = F::dot(cur.w[r], av[m], t);
                        if (t == 0 && live) rw[(m * R + r) * 17 + q] = v;
                    }
                wave_sync();
                if (lane < R * MB) {
                    const int nq = min(16, spr - c * 16);
                    for (int qq = 0; qq < nq; qq++) acc += rw[lane * 17 + qq];
                }
                wave_sync();
                if (c == nchunks - 1) {
                    int mat, row0;
                    locate(g, mat, row0);
                    const int r = lane % R, m = lane / R;
                    if (lane < R * MB && m < mb && row0 + r < a.n_rows) {
                        const float* bias = mat ? a.bias1 : a.bias0;
                        float* y = mat ? a.y1 : a.y0;
                        // biasO + sum (RT/Q4KDotKernel.cs:785); no add without a bias
                        y[(size_t)(pbeg + m0 + m) * a.n_rows + row0 + r] = bias ? as_float(cur.bias) + acc : acc;
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
        __syncthreads();  // every wave is done with this pass's rows before the next pass restages them
    }
}

namespace {

int rows_env(const char* name, int dflt) {
    const char* v = getenv(name);
    return v && *v ? atoi(v) : dflt;
}

int rows_cu_count() {
    static int n = 0;
    if (!n) {
        int dev = 0, c = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0)
            c = 256;
        n = c;
    }
    return n;
}

template <class F, int R, int MB>
hipError_t launch_rows(RArgs& ra, int experts, hipStream_t st) {
    ra.groups = (ra.n_rows + R - 1) / R;
    const int total = ra.groups * ra.nmat;
    const size_t lds = (size_t)((MB * ra.spr * (kLdsSlot + 36) + 15) & ~15) + 4 * (R * MB) * 17 * sizeof(float);
    // persistent: spread about `wg_per_cu` workgroups per CU over the experts of the launch
    static const int forced_wg = rows_env("OVFQ_ROWS_WG_PER_CU", 0);
    const int wg_per_cu = forced_wg > 0 ? forced_wg : 2;
    int per_expert = (rows_cu_count() * wg_per_cu + experts - 1) / experts;
    const int need = (total + 3) / 4;
    if (per_expert > need) per_expert = need;
    if (per_expert < 1) per_expert = 1;
    hipLaunchKernelGGL((kquant_rows_kernel<F, R, MB>), dim3(per_expert, experts), dim3(256), lds, st, ra);
    return hipGetLastError();
}

template <class F>
hipError_t launch_rows_f(RArgs& ra, int experts, int mb, hipStream_t st) {
    const bool long_rows = ra.spr > 16;
    if (mb <= 4) return long_rows ? launch_rows<F, 1, 4>(ra, experts, st) : launch_rows<F, 2, 4>(ra, experts, st);
    return long_rows ? launch_rows<F, 1, 8>(ra, experts, st) : launch_rows<F, 2, 8>(ra, experts, st);
}

}  // namespace

bool rows_supported(int type, int in) { return (type == 12 || type == 14) && in % kQK == 0 && in / kQK <= kRowsMaxSpr; }

int rows_pass_rows() {
    static const int v = rows_env("OVFQ_ROWS_PASS", 4);
    return v == 8 ? 8 : 4;
}

hipError_t launch_rows_kquant(int type, const RowsLaunch& L, hipStream_t st) {
    RArgs ra{};
    for (int i = 0; i < L.experts; i++) {
        ra.w0[i] = L.w0[i];
        ra.w1[i] = L.w1 ? L.w1[i] : nullptr;
    }
    ra.bias0 = L.bias0;
    ra.bias1 = L.bias1;
    ra.y0 = L.y0;
    ra.y1 = L.y1;
    ra.n_rows = L.n_rows;
    ra.spr = L.in / kQK;
    ra.nmat = L.w1 ? 2 : 1;
    ra.rows = L.rows;
    ra.expert_off = L.expert_off;
    ra.pair_row = L.pair_row;
    ra.q = L.act.q;
    ra.s = L.act.s;
    ra.b = L.act.b;
    const int mb = L.pass_rows > 0 ? L.pass_rows : rows_pass_rows();
    if (type == 12) return launch_rows_f<Q4K>(ra, L.experts, mb, st);
    return launch_rows_f<Q6K>(ra, L.experts, mb, st);
}

}  // namespace ovfq
