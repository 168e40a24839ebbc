// heads.hip — the attention output projection with per-head Q8_0 Wo, in one launch.
//
// The reference's default Llama o-path (LD/GgufLlamaLoader.cs:977-995 requantises Wo per head to Q8_0): the output
// starts as the attention bias (or zero), every head h projects its head_dim slice of the attention output through
// its own Wo_h [d_model][head_dim] with Q8DotKernel.Project (no bias; RT/CachedSingleHeadAttention.cs:323-337), and
// the head outputs are added into the output in ascending head order (RT/CachedMultiHeadAttention.cs:185-194,
// :292-297; prefill rows :600-614, :703-711). Each head's value for an output is its blocks' (wScale * aScale) * dot
// summed from +0 in ascending block order (RT/Q8DotKernel.cs:127-137).
//
// Work split: a workgroup owns 16 consecutive outputs; its eight waves take heads w, w + 8, w + 16, ... For one head,
// the 16 outputs' rows are 16 * head_dim contiguous bytes of Wo_h, so lane u of the wave loads block u of that
// region (32 bytes: output u / nb, block u % nb, nb = head_dim / 32) and the block's weight scale: a coalesced read of
// the tile. All of a wave's heads (up to four, a ring refilled as each is computed past that) are in flight at
// once. The lane dots its block with every activation row (the activation is quantised to Q8_0 into LDS in the
// launch, or copied from a prequantised one); the nb lanes of one output gather their block values with DPP moves
// (lane shuffles for head_dim 256) and add them in block order into the head value (head_dim 32 / 64 / 128 / 256;
// other head sizes go through LDS). After all heads, one lane per (row, output) adds bias-or-zero and the head values
// in head order.
#include "ovfq_device.h"
#include "ovfq_launch.h"

namespace ovfq {

namespace {

constexpr int kTile = 16;   // outputs per workgroup
constexpr int kWaves = 8;   // waves per workgroup
constexpr int kRing = 4;    // heads in flight per wave (blocks per lane U = 1; 2 for U = 2)
// Per-wave activation staging: in-launch quantisation of up to kXPasses * 256 of the wave's columns (all rows), or a
// copy of up to kQPasses * 64 16-byte pieces and kSPasses * 64 scales of a prequantised activation.
constexpr int kXPasses = 8;
constexpr int kQPasses = 8;
constexpr int kSPasses = 4;

struct HArgs {
    const int8_t* wq[kHeadsMax];
    const float* ws[kHeadsMax];
    const float* bias;
    float* y;
    const float* x;    // fp32 [rows][K], quantised in the launch; NULL -> q / s
    const int8_t* q;   // Q8_0 [rows][K]
    const float* s;    // [rows][K / 32]
    int n_heads;
    int head_dim;
    int d_model;
    int rows;
};

// LDS layout (bytes): activation quants [M][K], activation scales [M][K/32], head values [M][16][H + pad] (head
// fastest, the row padded to a multiple of 4 floats), per wave block values [M][64 U] (the LDS gather for head sizes
// whose output rows do not tile a wave).
__host__ __device__ inline int heads_hv_stride(int n_heads) { return (n_heads + 3) & ~3; }

// Lane `lane`'s value of the lane (lane & ~3) + b of its quad, through DPP (a VALU move, no LDS round trip).
template <int B>
__device__ __forceinline__ float quad_lane(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), B * 0x55, 0xf, 0xf,
                                                                 false));
}

// The head value of the output whose NB blocks are this lane's group of NB consecutive lanes: the block values added
// in block order from +0 (Dot, RT/Q8DotKernel.cs:131-137). Every lane of the group receives it.
template <int NB>
__device__ __forceinline__ float ordered_group_sum(float v, int lane) {
    if constexpr (NB == 1) {
        return 0.0f + v;
    } else if constexpr (NB == 2) {
        const float e = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xa0, 0xf,
                                                                              0xf, false));  // quad_perm [0,0,2,2]
        const float o = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xf5, 0xf,
                                                                              0xf, false));  // quad_perm [1,1,3,3]
        return (0.0f + e) + o;
    } else if constexpr (NB == 4) {
        return (((0.0f + quad_lane<0>(v)) + quad_lane<1>(v)) + quad_lane<2>(v)) + quad_lane<3>(v);
    } else {
        const int base = lane & ~(NB - 1);
        float g[NB];
#pragma unroll
        for (int b = 0; b < NB; b++) g[b] = __shfl(v, base + b, 64);
        float hsum = 0.0f;
#pragma unroll
        for (int b = 0; b < NB; b++) hsum += g[b];
        return hsum;
    }
}

// U: blocks per lane and head (1 for head_dim <= 128, 2 for head_dim <= 256). NB: blocks per head when a head's
// output rows tile a 64-lane unit group (head_dim 32, 64, 128, 256: NB = 1, 2, 4, 8); 0 for the other head sizes,
// whose block values are gathered through LDS.
template <int U, int NB>
__global__ __launch_bounds__(kWaves * 64) void q8_0_heads_kernel(const HArgs a) {
    constexpr int D = kRing / U;
    extern __shared__ __align__(16) uint8_t smem_h[];
    const int H = a.n_heads, hd = a.head_dim, nb = NB ? NB : hd >> 5, M = a.rows, dm = a.d_model;
    const int K = H * hd, kb = K >> 5, hs = heads_hv_stride(H);
    uint8_t* lq = smem_h;                                                 // [M][K]
    float* ls = reinterpret_cast<float*>(smem_h + M * K);                // [M][kb]
    float* hv = ls + ((M * kb + 3) & ~3);                                // [M][16][hs]
    float* vs = hv + M * kTile * hs;                                     // per wave [M][64 U]
    const int wave = wave_id();
    const int lane = threadIdx.x & 63;
    const int o0 = blockIdx.x * kTile;
    const int rows_here = min(kTile, dm - o0);
    const int units = kTile * nb;         // blocks of the tile per head
    float* wv = vs + wave * (M * 64 * U);

    struct Item {
        u32x4 w[U][2];
        uint32_t s[U];
    };
    const int J = wave < H ? (H - wave + kWaves - 1) / kWaves : 0;  // heads of this wave: wave + 8 j, j < J
    auto load = [&](int j, Item& it) {
        const bool valid = j < J;
        const int h = valid ? wave + kWaves * j : 0;
        const __amdgpu_buffer_rsrc_t wr =
            make_rsrc(a.wq[h] + (uint64_t)o0 * hd, valid ? (uint32_t)(rows_here * hd) : 0u);
        const __amdgpu_buffer_rsrc_t sr =
            make_rsrc(a.ws[h] + (uint64_t)o0 * nb, valid ? (uint32_t)(rows_here * nb) * 4u : 0u);
#pragma unroll
        for (int k = 0; k < U; k++) {
            const uint32_t u = (uint32_t)(lane + 64 * k);  // past the tile: the reads return 0
            it.w[k][0] = ld4(wr, u * 32u);
            it.w[k][1] = ld4(wr, u * 32u + 16u);
            it.s[k] = ld1(sr, u * 4u);
        }
    };

    Item ring[D];
    // The wave's activation: for every row m, the head_dim columns of each of its heads h = wave + 8 j (j < J), in
    // the [M][K] layout of the whole activation; only this wave reads them, so a wave barrier orders the staging.
    const int per_row = J * hd;  // the wave's columns per row
    if (J == 0) {
        // a wave without heads (fewer than eight heads) stages nothing; its ring reads through zero-length resources
#pragma unroll
        for (int s = 0; s < D; s++) load(s, ring[s]);
    } else if (a.x) {
        // Q8DotKernel.Quantize of the wave's columns into LDS (the standalone quantiser's device function): lane l
        // of pass p takes four consecutive columns; eight lanes form one 32-element block (a head's columns are
        // whole blocks). Loads first, then the weight ring, then the quantisation.
        const int n = M * K;
        const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, (uint32_t)n * 4u);
        u32x4 xv[kXPasses];
        int off[kXPasses];
#pragma unroll
        for (int p = 0; p < kXPasses; p++) {
            const int e = p * 256 + lane * 4;
            const int m = e / per_row, rem = e - m * per_row, j = rem / hd, t = rem - j * hd;
            off[p] = m < M ? m * K + (wave + kWaves * j) * hd + t : n;  // past the wave's columns: reads 0
            xv[p] = ld4(xr, (uint32_t)off[p] * 4u);
        }
#pragma unroll
        for (int s = 0; s < D; s++) load(s, ring[s]);
#pragma unroll
        for (int p = 0; p < kXPasses; p++) {
            if (p * 256 >= M * per_row) break;  // uniform
            const Q80Lane r = q8_0_quantize_lane(xv[p]);  // every lane takes part
            if (off[p] < n) {
                *reinterpret_cast<uint32_t*>(lq + off[p]) = r.packed;
                if ((lane & 7) == 0) ls[off[p] >> 5] = r.scale;
            }
        }
    } else {
        // copy of the wave's columns of the prequantised activation: 16-byte pieces of quants, then scales
        const int n = M * K;
        const __amdgpu_buffer_rsrc_t qr = make_rsrc(a.q, (uint32_t)n);
        const __amdgpu_buffer_rsrc_t sr = make_rsrc(a.s, (uint32_t)(M * kb) * 4u);
        const int pieces = per_row >> 4, nbw = per_row >> 5;
        u32x4 qv[kQPasses];
        int qo[kQPasses];
#pragma unroll
        for (int p = 0; p < kQPasses; p++) {
            const int i = p * 64 + lane;
            const int m = i / pieces, rem = (i - m * pieces) * 16, j = rem / hd, t = rem - j * hd;
            qo[p] = m < M ? m * K + (wave + kWaves * j) * hd + t : n;
            qv[p] = ld4(qr, (uint32_t)qo[p]);
        }
        uint32_t sv[kSPasses];
        int so[kSPasses];
#pragma unroll
        for (int p = 0; p < kSPasses; p++) {
            const int i = p * 64 + lane;
            const int m = i / nbw, rem = i - m * nbw, j = rem / nb, b = rem - j * nb;
            so[p] = m < M ? m * kb + (wave + kWaves * j) * nb + b : M * kb;
            sv[p] = ld1(sr, (uint32_t)so[p] * 4u);
        }
#pragma unroll
        for (int s = 0; s < D; s++) load(s, ring[s]);
#pragma unroll
        for (int p = 0; p < kQPasses; p++)
            if (qo[p] < n) *reinterpret_cast<u32x4*>(lq + qo[p]) = qv[p];
#pragma unroll
        for (int p = 0; p < kSPasses; p++)
            if (so[p] < M * kb) ls[so[p]] = as_float(sv[p]);
    }
    wave_sync();

    // Block value (wScale * aScale) * dot (RT/Q8DotKernel.cs:136) of the lane's unit k against row m of head h.
    auto block_value = [&](const Item& it, int k, int m, int h) -> float {
        const int b = (lane + 64 * k) % nb;
        const uint8_t* xa = lq + m * K + h * hd + b * 32;
        const u32x4 x0 = *reinterpret_cast<const u32x4*>(xa);
        const u32x4 x1 = *reinterpret_cast<const u32x4*>(xa + 16);
        int d0 = sdot4(it.w[k][0].x, x0.x, 0);
        int d1 = sdot4(it.w[k][1].x, x1.x, 0);
        d0 = sdot4(it.w[k][0].y, x0.y, d0);
        d1 = sdot4(it.w[k][1].y, x1.y, d1);
        d0 = sdot4(it.w[k][0].z, x0.z, d0);
        d1 = sdot4(it.w[k][1].z, x1.z, d1);
        d0 = sdot4(it.w[k][0].w, x0.w, d0);
        d1 = sdot4(it.w[k][1].w, x1.w, d1);
        const float xs = ls[m * kb + h * nb + b];
        return as_float(it.s[k]) * xs * (float)(d0 + d1);
    };

    if constexpr (NB != 0) {
        // The output's NB blocks are NB consecutive lanes of a unit group: gathered with DPP moves (or lane shuffles
        // for NB = 8) and added in block order. The ring's heads are computed together, so their dependency chains
        // interleave.
        for (int j0 = 0; j0 < J; j0 += D) {
#pragma unroll 1
            for (int m = 0; m < M; m++) {
                float v[D][U];
#pragma unroll
                for (int s = 0; s < D; s++) {
                    const int j = j0 + s;
                    const int h = j < J ? wave + kWaves * j : wave;  // a slot past the wave's heads reads head `wave`
#pragma unroll
                    for (int k = 0; k < U; k++) v[s][k] = block_value(ring[s], k, m, h);
                }
#pragma unroll
                for (int s = 0; s < D; s++) {
                    const int j = j0 + s;
#pragma unroll
                    for (int k = 0; k < U; k++) {
                        const int u = lane + 64 * k, b = u % NB, r = u / NB;
                        const float hsum = ordered_group_sum<NB>(v[s][k], lane);
                        if (j < J && b == 0 && r < kTile) hv[(m * kTile + r) * hs + wave + kWaves * j] = hsum;
                    }
                }
            }
#pragma unroll
            for (int s = 0; s < D; s++) load(j0 + s + D, ring[s]);  // past the wave's heads: zero-length reads
        }
    } else {
        // Other head sizes: block values through this wave's LDS slice, one lane per (row, output) adds them.
        for (int j0 = 0; j0 < J; j0 += D) {
#pragma unroll
            for (int s = 0; s < D; s++) {
                const int j = j0 + s;
                if (j < J) {
                    const int h = wave + kWaves * j;
#pragma unroll 1
                    for (int m = 0; m < M; m++) {
#pragma unroll
                        for (int k = 0; k < U; k++) {
                            const float v = block_value(ring[s], k, m, h);
                            if (lane + 64 * k < units) wv[m * 64 * U + lane + 64 * k] = v;
                        }
                    }
                    wave_sync();
                    for (int p = lane; p < M * kTile; p += 64) {
                        const int m = p / kTile, r = p % kTile;
                        float hsum = 0.0f;
                        for (int b = 0; b < nb; b++) hsum += wv[m * 64 * U + r * nb + b];
                        hv[(m * kTile + r) * hs + h] = hsum;
                    }
                    wave_sync();
                }
                load(j + D, ring[s]);
            }
        }
    }
    __syncthreads();
    // output = bias (or zero), then += each head's value, heads ascending
    for (int p = (int)threadIdx.x; p < M * kTile; p += kWaves * 64) {
        const int m = p / kTile, r = p % kTile;
        if (r < rows_here) {
            float acc = a.bias ? a.bias[o0 + r] : 0.0f;
            const float* row = hv + (m * kTile + r) * hs;
            int h = 0;
            for (; h + 4 <= H; h += 4) {
                const float4 v4 = *reinterpret_cast<const float4*>(row + h);
                acc += v4.x;
                acc += v4.y;
                acc += v4.z;
                acc += v4.w;
            }
            for (; h < H; h++) acc += row[h];
            a.y[(size_t)m * dm + o0 + r] = acc;
        }
    }
}

}  // namespace

// Heads of the wave that takes the most (wave 0): ceil(n_heads / 8).
static int heads_per_wave(int n_heads) { return (n_heads + kWaves - 1) / kWaves; }

size_t q8_0_heads_lds_bytes(int n_heads, int head_dim, int rows) {
    const int K = n_heads * head_dim, U = head_dim <= 128 ? 1 : 2;
    return (size_t)rows * K + 4 * (size_t)((rows * (K / 32) + 3) & ~3) +
           4 * (size_t)rows * kTile * heads_hv_stride(n_heads) + 4 * (size_t)kWaves * rows * 64 * U;
}

bool q8_0_heads_supported(int n_heads, int head_dim, int rows) {
    if (n_heads < 1 || n_heads > kHeadsMax || head_dim < 32 || head_dim > kHeadsMaxDim || head_dim % 32) return false;
    const int per_wave = rows * heads_per_wave(n_heads) * head_dim;  // the wave's staged columns, all rows
    return rows >= 1 && rows <= kHeadsMaxRows && rows * n_heads * head_dim <= kHeadsMaxIn &&
           rows * n_heads <= kHeadsMaxRowHeads && per_wave <= kQPasses * 64 * 16 &&
           per_wave / 32 <= kSPasses * 64 && q8_0_heads_lds_bytes(n_heads, head_dim, rows) <= kHeadsMaxLds;
}

bool q8_0_heads_quantize_inside(int n_heads, int head_dim, int rows) {
    return rows * heads_per_wave(n_heads) * head_dim <= kXPasses * 256;
}

hipError_t launch_q8_0_heads(const int8_t* const* wq, const float* const* ws, int n_heads, int head_dim,
                             int d_model, int rows, const float* bias, const float* x, ActQ act, float* y,
                             hipStream_t st) {
    if (!q8_0_heads_supported(n_heads, head_dim, rows) || (x && !q8_0_heads_quantize_inside(n_heads, head_dim, rows)))
        return hipErrorInvalidValue;
    if (!x && (!act.q || !act.s)) return hipErrorInvalidValue;
    HArgs a{};
    for (int h = 0; h < n_heads; h++) {
        a.wq[h] = wq[h];
        a.ws[h] = ws[h];
    }
    a.bias = bias;
    a.y = y;
    a.x = x;
    a.q = act.q;
    a.s = act.s;
    a.n_heads = n_heads;
    a.head_dim = head_dim;
    a.d_model = d_model;
    a.rows = rows;
    const dim3 grid((d_model + kTile - 1) / kTile), block(kWaves * 64);
    const size_t lds = q8_0_heads_lds_bytes(n_heads, head_dim, rows);
    switch (head_dim) {
        case 32: hipLaunchKernelGGL((q8_0_heads_kernel<1, 1>), grid, block, lds, st, a); break;
        case 64: hipLaunchKernelGGL((q8_0_heads_kernel<1, 2>), grid, block, lds, st, a); break;
        case 128: hipLaunchKernelGGL((q8_0_heads_kernel<1, 4>), grid, block, lds, st, a); break;
        case 256: hipLaunchKernelGGL((q8_0_heads_kernel<2, 8>), grid, block, lds, st, a); break;
        default:
            if (head_dim <= 128)
                hipLaunchKernelGGL((q8_0_heads_kernel<1, 0>), grid, block, lds, st, a);
            else
                hipLaunchKernelGGL((q8_0_heads_kernel<2, 0>), grid, block, lds, st, a);
    }
    return hipGetLastError();
}

}  // namespace ovfq
