// moe.hip — the routed-MoE pieces around the grouped expert projections (mfma.hip, small-M kernel).
//
// MoeFeedForwardBlock.DecodeBatched (RT/MoeFeedForwardBlock.cs:140-241) without its router projection:
//   1. MoeRouter.SelectTopK per token (RT/MoeRouter.cs:40-128)                       -> moe_topk_kernel
//   2. group the (token, top-k slot) pairs by expert, tokens ascending, and quantise
//      the tokens' activation to Q8_K in the same launch                            -> moe_plan_kernel
//   3. per expert: gate/up = batched projections of its tokens, all experts in one launch (mfma.hip: the
//      expert-stream kernel for Q4_K with few pairs, else the small-M or tiled MFMA kernel)
//   4. SiLU(gate) * up, quantised to Q8_K for the down projection                    -> gate_up_q8k_kernel
//   5. per expert: down projection of its pairs, one launch                      (mfma.hip, as step 3)
//   6. y[token] = sum over top-k slots, in slot order, of weight * expert output     -> moe_combine_kernel
// Pairs are numbered expert-major (expert 0's tokens first, ascending), which is the order the reference
// gathers rows in; pair_of[token * k + slot] maps a slot back to its pair.
#include <algorithm>
#include <cmath>

#include "ovfq_device.h"
#include "ovfq_launch.h"

namespace ovfq {

typedef float f32x4 __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------------------------------ router
// One thread per token: insertion of each logit into a descending top-k list (ties keep the lower index), then
// softmax over the k kept logits (normalize) or the full softmax evaluated at them. The workgroup's 64 logit rows
// are first copied to LDS with coalesced loads, so the sequential scan reads LDS, not memory.
//
// The list has KM >= k entries, every one indexed at compile time so that it lives in registers (a list indexed
// at run time would sit in scratch memory). One insertion is the reference's loop written as a selection per
// entry: with pos0 = min(filled, k - 1), the entries j in (p, pos0] take entry j - 1 and entry p takes the new
// logit, where p is where the reference's `while (pos > 0 && w[pos - 1] < l) pos--` stops (RT/MoeRouter.cs:70-91).
// Token n's selection from its logits l[0 .. n_experts): indices and weights of its top k (k <= KM) in idx / wv.
template <int KM>
__device__ __forceinline__ void topk_select(const float* l, int n_experts, int k, int normalize, int (&idx)[KM],
                                            float (&wv)[KM]) {
#pragma unroll
    for (int i = 0; i < KM; i++) {
        idx[i] = -1;
        wv[i] = -INFINITY;
    }
    int filled = 0;
    for (int e = 0; e < n_experts; e++) {
        const float v = l[e];
        float last = wv[0];
#pragma unroll
        for (int i = 1; i < KM; i++) last = i == k - 1 ? wv[i] : last;
        if (filled == k && v <= last) continue;
        const int pos0 = filled < k ? filled : k - 1;
        float nw[KM];
        int ni[KM];
        bool shift_above = false;  // entry j + 1 takes entry j
#pragma unroll
        for (int j = KM - 1; j >= 0; j--) {
            const bool in_run = j <= pos0 && (j == pos0 || shift_above);
            const bool shift = j > 0 && in_run && wv[j > 0 ? j - 1 : 0] < v;
            const bool place = in_run && !shift;
            nw[j] = shift ? wv[j > 0 ? j - 1 : 0] : (place ? v : wv[j]);
            ni[j] = shift ? idx[j > 0 ? j - 1 : 0] : (place ? e : idx[j]);
            shift_above = shift;
        }
#pragma unroll
        for (int j = 0; j < KM; j++) {
            wv[j] = nw[j];
            idx[j] = ni[j];
        }
        if (filled < k) filled++;
    }
    const float mx = wv[0];
    if (normalize) {
        float sum = 0.0f;
#pragma unroll
        for (int i = 0; i < KM; i++) {
            if (i < k) {
                const float w = expf(wv[i] - mx);
                wv[i] = w;
                sum += w;
            }
        }
        const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
#pragma unroll
        for (int i = 0; i < KM; i++) wv[i] *= inv;
    } else {
        float total = 0.0f;
        for (int e = 0; e < n_experts; e++) total += expf(l[e] - mx);
        const float inv = total > 0.0f ? 1.0f / total : 0.0f;
#pragma unroll
        for (int i = 0; i < KM; i++) wv[i] = expf(wv[i] - mx) * inv;
    }
}

template <int KM>
__global__ __launch_bounds__(64) void moe_topk_kernel(const float* __restrict__ logits, int rows, int n_experts,
                                                      int k, int stride, int normalize, int* __restrict__ idx_out,
                                                      float* __restrict__ w_out) {
    __shared__ float sl[64 * kMaxExperts];
    const int row0 = blockIdx.x * 64;
    const int nrow = min(64, rows - row0);
    for (int i = threadIdx.x; i < nrow * n_experts; i += 64) sl[i] = logits[(size_t)row0 * n_experts + i];
    __syncthreads();
    const int n = row0 + threadIdx.x;
    if (n >= rows) return;
    int idx[KM];
    float wv[KM];
    topk_select<KM>(sl + threadIdx.x * n_experts, n_experts, k, normalize, idx, wv);
#pragma unroll
    for (int i = 0; i < KM; i++) {
        if (i < k) {
            idx_out[(size_t)n * stride + i] = idx[i];
            w_out[(size_t)n * stride + i] = wv[i];
        }
    }
}

// ------------------------------------------------------------------------------------------ grouping
// The grouping plan of up to 64 (token, slot) entries in one wave: lane i holds entry i's expert `ex` (token i / k,
// slot i % k; -1 past the entries). Per expert a ballot of its claiming lanes gives the count and each lane's rank
// (entries of lower tokens come first, and a token claims an expert at most once), so the positions are the ones
// the general path of moe_plan_kernel computes.
__device__ __forceinline__ void plan_one_wave(int ex, int rows, int k, int n_experts, int* __restrict__ expert_off,
                                              int* __restrict__ pair_row, int* __restrict__ pair_of, int nt,
                                              int* __restrict__ tiles, int* __restrict__ tile_count) {
    const int lane = threadIdx.x & 63;
    const uint64_t below = (1ull << lane) - 1ull;
    const bool valid = lane < rows * k;
    const int slot = valid ? lane % k : 0;
    bool claim = valid && ex >= 0 && ex < n_experts;
    for (int d = 1; d < k; d++) {  // an earlier slot of the same token with the same expert claims it instead
        const int prev = __shfl(ex, lane - d < 0 ? 0 : lane - d, 64);
        if (slot >= d && prev == ex) claim = false;
    }
    int pos = -1, off = 0, tb = 0;
    for (int e = 0; e < n_experts; e++) {
        const uint64_t m = __ballot(claim && ex == e);
        if (claim && ex == e) pos = off + __popcll(m & below);
        if (lane == 0) expert_off[e] = off;
        const int c = __popcll(m);
        if (tiles) {
            const int nt_e = (c + nt - 1) / nt;
            for (int i = lane; i < nt_e; i += 64) tiles[tb + i] = e | (i << 8);
            tb += nt_e;
        }
        off += c;
    }
    if (lane == 0) {
        expert_off[n_experts] = off;
        if (tiles) *tile_count = tb;
    }
    if (valid) pair_of[lane] = pos;
    if (pos >= 0) pair_row[pos] = lane / k;
}

// One workgroup. Expert e's pairs are the tokens n (ascending) with a slot j such that idx[n][j] == e (the first
// such slot: RT/MoeFeedForwardBlock.cs:191-204). A slot whose expert is out of range, or repeats an earlier slot's
// expert, belongs to no pair (pair_of = -1) and contributes nothing to the combine.
// Tokens are taken 256 at a time, one per thread. For each expert a wave ballot of the tokens that claim it gives
// the per-wave count and each token's rank among the wave's claimers (popcount of the lower lanes), so a pair's
// position is expert_off[e] + (claimers of e in earlier chunks) + (in earlier waves of this chunk) + rank. The
// routing table is staged in LDS when it fits (rows * k ints <= 48 KB).
// With `tiles`, it also lists the experts' pair ranges in tiles of `nt` rows, expert-major: entry t = expert | (tile
// index within the expert << 8), with the list's length at *tile_count.
// Workgroup 0 does all of the above (up to 64 entries in one wave, without barriers); workgroups 1.. quantise the
// tokens' activation x to Q8_K (one wave per 256-element block, the standalone quantiser's arithmetic), which the
// plan does not depend on: one launch for both.
__global__ __launch_bounds__(256) void moe_plan_kernel(const int* __restrict__ idx_g, int rows, int k, int n_experts,
                                                       int* __restrict__ expert_off, int* __restrict__ pair_row,
                                                       int* __restrict__ pair_of, int staged, int nt,
                                                       int* __restrict__ tiles, int* __restrict__ tile_count,
                                                       const float* __restrict__ x, int64_t n_blocks,
                                                       int8_t* __restrict__ xq, float* __restrict__ xs,
                                                       int16_t* __restrict__ xb) {
    if (blockIdx.x > 0) {
        const int64_t blk = (int64_t)(blockIdx.x - 1) * 4 + wave_id();
        if (blk < n_blocks) q8k_quantize_block(x, blk, xq, xs, xb);
        return;
    }
    if (rows * k <= 64) {
        // Up to 64 (token, slot) entries: one wave does the whole plan, without barriers.
        if (wave_id() != 0) return;
        const int lane = threadIdx.x & 63;
        plan_one_wave(lane < rows * k ? idx_g[lane] : -1, rows, k, n_experts, expert_off, pair_row, pair_of, nt, tiles,
                      tile_count);
        return;
    }
    extern __shared__ int sidx[];
    __shared__ int run[kMaxExperts];        // first position of the current chunk's claimers, per expert
    __shared__ int wcnt[4][kMaxExperts];    // claimers per wave of the current chunk, per expert
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const uint64_t below = (1ull << lane) - 1ull;
    for (int i = tid; i < rows * k; i += blockDim.x) {
        pair_of[i] = -1;
        if (staged) sidx[i] = idx_g[i];
    }
    if (tid < n_experts) run[tid] = 0;
    __syncthreads();
    const int* idx = staged ? sidx : idx_g;
    // first slot of token n holding expert e, or -1
    auto claim_slot = [&](int n, int e) -> int {
        if (n >= rows) return -1;
        for (int j = 0; j < k; j++)
            if (idx[n * k + j] == e) return j;
        return -1;
    };
    // pass 1: claimers per expert
    for (int c0 = 0; c0 < rows; c0 += 256) {
        for (int e = 0; e < n_experts; e++) {
            const uint64_t m = __ballot(claim_slot(c0 + tid, e) >= 0);
            if (lane == 0) wcnt[wave][e] = __popcll(m);
        }
        __syncthreads();
        if (tid < n_experts) run[tid] += wcnt[0][tid] + wcnt[1][tid] + wcnt[2][tid] + wcnt[3][tid];
        __syncthreads();
    }
    __shared__ int tbase[kMaxExperts + 1];  // first tile-list entry per expert
    if (tid == 0) {
        int acc = 0, tacc = 0;
        for (int e = 0; e < n_experts; e++) {
            const int c = run[e];
            run[e] = acc;
            expert_off[e] = acc;
            acc += c;
            tbase[e] = tacc;
            tacc += (c + nt - 1) / nt;
        }
        expert_off[n_experts] = acc;
        tbase[n_experts] = tacc;
        if (tiles) *tile_count = tacc;
    }
    __syncthreads();
    if (tiles) {
        for (int e = 0; e < n_experts; e++)
            for (int i = tid; i < tbase[e + 1] - tbase[e]; i += blockDim.x) tiles[tbase[e] + i] = e | (i << 8);
    }
    // pass 2: positions, tokens ascending within each expert
    for (int c0 = 0; c0 < rows; c0 += 256) {
        const int n = c0 + tid;
        for (int e = 0; e < n_experts; e++) {
            const int j = claim_slot(n, e);
            const uint64_t m = __ballot(j >= 0);
            if (lane == 0) wcnt[wave][e] = __popcll(m);
            if (j >= 0) pair_of[n * k + j] = __popcll(m & below);  // rank within the wave, completed below
        }
        __syncthreads();
        if (n < rows) {
            for (int j = 0; j < k; j++) {
                const int e = idx[n * k + j];
                if (e < 0 || e >= n_experts || claim_slot(n, e) != j) continue;
                int p = run[e] + pair_of[n * k + j];
                for (int w = 0; w < wave; w++) p += wcnt[w][e];
                pair_of[n * k + j] = p;
                pair_row[p] = n;
            }
        }
        __syncthreads();
        if (tid < n_experts) run[tid] += wcnt[0][tid] + wcnt[1][tid] + wcnt[2][tid] + wcnt[3][tid];
        __syncthreads();
    }
}

// Router + grouping plan in one launch (MoeFeedForwardBlock.DecodeBatched's SelectTopK and grouping, RT/
// MoeFeedForwardBlock.cs:140-204): for up to 64 tokens and 64 (token, slot) entries, wave 0 of workgroup 0 selects
// each token's top k (lane n = token n, topk_select as in moe_topk_kernel), writes the indices and weights
// [rows][k], hands entry i's expert to lane i by lane shuffles and runs plan_one_wave; workgroups 1.. quantise x to
// Q8_K as in moe_plan_kernel.
template <int KM>
__global__ __launch_bounds__(256) void moe_route_plan_kernel(const float* __restrict__ logits, int rows, int k,
                                                             int n_experts, int normalize, int* __restrict__ idx_out,
                                                             float* __restrict__ w_out, int* __restrict__ expert_off,
                                                             int* __restrict__ pair_row, int* __restrict__ pair_of,
                                                             int nt, int* __restrict__ tiles,
                                                             int* __restrict__ tile_count, const float* __restrict__ x,
                                                             int64_t n_blocks, int8_t* __restrict__ xq,
                                                             float* __restrict__ xs, int16_t* __restrict__ xb) {
    if (blockIdx.x > 0) {
        const int64_t blk = (int64_t)(blockIdx.x - 1) * 4 + wave_id();
        if (blk < n_blocks) q8k_quantize_block(x, blk, xq, xs, xb);
        return;
    }
    if (wave_id() != 0) return;
    __shared__ float sl[64 * kMaxExperts];
    const int lane = threadIdx.x & 63;
    // The logits (rows * n_experts <= 4096) go to LDS in batches of eight coalesced loads per lane, so the scan
    // below does not wait for memory once per expert.
    const int total = rows * n_experts;
    for (int u0 = 0; u0 < total; u0 += 8 * 64) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int i = u0 + u * 64 + lane;
            v[u] = i < total ? logits[i] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int i = u0 + u * 64 + lane;
            if (i < total) sl[i] = v[u];
        }
    }
    wave_sync();
    int idx[KM];
    float wv[KM];
#pragma unroll
    for (int i = 0; i < KM; i++) idx[i] = -1;
    if (lane < rows) {
        topk_select<KM>(sl + lane * n_experts, n_experts, k, normalize, idx, wv);
#pragma unroll
        for (int i = 0; i < KM; i++) {
            if (i < k) {
                idx_out[lane * k + i] = idx[i];
                w_out[lane * k + i] = wv[i];
            }
        }
    }
    // entry i = (token i / k, slot i % k): its expert from lane i / k's list
    const int src = lane < rows * k ? lane / k : 0, slot = lane < rows * k ? lane % k : 0;
    int ex = -1;
#pragma unroll
    for (int i = 0; i < KM; i++) {
        const int v = __shfl(idx[i], src, 64);
        if (i == slot) ex = v;
    }
    plan_one_wave(lane < rows * k ? ex : -1, rows, k, n_experts, expert_off, pair_row, pair_of, nt, tiles,
                  tile_count);
}

// ------------------------------------------------------------------------------------------ gate * up
// One wave per (pair, 256-element block) of the intermediate: gate <- act(gate), up <- gate * up (ApplyGate +
// TensorPrimitives.Multiply, RT/CachedFeedForwardBlock.cs:339-344, :474-485), then the Q8_K quantisation the down
// projection's BatchedQuantProjection.Dispatch applies to its input (RT/Q4KDotKernel.cs:71-136). act is SiLU,
// g * sigmoid(g) (ApplySiLU :464-472), or with GELU the tanh approximation 0.5 g (1 + tanh(sqrt(2/pi) (g + 0.044715
// g^3))) in ApplyGeLU's operation order (:498-517). Pairs at or past expert_off[n_experts] are skipped.
// The launch also does the MoeFold work (zeroing the step's output, the per-pair combine weights), one element per
// thread of the grid, which covers both.
template <bool GELU>
__global__ __launch_bounds__(256) void gate_up_q8k_kernel(const float* __restrict__ gate, const float* __restrict__ up,
                                                         const int* __restrict__ expert_off, int n_experts,
                                                         int max_pairs, int spr, int8_t* __restrict__ q,
                                                         float* __restrict__ s, int16_t* __restrict__ bs,
                                                         const MoeFold fold) {
    {
        const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
        for (int64_t j = i * 4; j < fold.y_len && j < i * 4 + 4; j++) fold.y[j] = 0.0f;
        if (i < fold.slots) {
            const int p = fold.pair_of[i];
            if (p >= 0) fold.pw[p] = fold.w[i];
        }
    }
    const int64_t blk = (int64_t)blockIdx.x * 4 + wave_id();
    if (blk >= (int64_t)max_pairs * spr) return;
    const int lane = threadIdx.x & 63;
    // The block's loads go out before the pair count arrives (both buffers hold max_pairs rows); a block past the
    // count stores nothing.
    const __amdgpu_buffer_rsrc_t gr = make_rsrc(gate + blk * kQK, kQK * 4);
    const __amdgpu_buffer_rsrc_t ur = make_rsrc(up + blk * kQK, kQK * 4);
    const u32x4 gv = ld4(gr, lane * 16), uv = ld4(ur, lane * 16);
    const int pairs = expert_off ? expert_off[n_experts] : max_pairs;
    const bool live = blk / spr < pairs;
    const float g[4] = {as_float(gv.x), as_float(gv.y), as_float(gv.z), as_float(gv.w)};
    const float u[4] = {as_float(uv.x), as_float(uv.y), as_float(uv.z), as_float(uv.w)};
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        float act;
        if (GELU) {
            const float x3 = g[i] * g[i] * g[i];
            const float inner = 0.7978845608028654f * (g[i] + 0.044715f * x3);
            act = 0.5f * g[i] * (1.0f + tanhf(inner));
        } else {
            const float sig = 1.0f / (1.0f + expf(-g[i]));
            act = g[i] * sig;
        }
        v[i] = act * u[i];
    }
    const Q8KLane r = q8k_quantize_wave(v[0], v[1], v[2], v[3]);
    if (!live) return;
    reinterpret_cast<uint32_t*>(q + blk * kQK)[lane] = r.packed;
    if ((lane & 3) == 0) bs[blk * 16 + (lane >> 2)] = (int16_t)r.group_sum;
    if (lane == 0) s[blk] = r.scale;
}

// ------------------------------------------------------------------------------------------ combine
// y[n][d] = 0; for each slot j in order: y[n][d] += w[n][j] * out[pair_of[n][j]][d] (RT/MoeFeedForwardBlock.cs:
// 225-239). Each thread owns four consecutive d of one token (dmodel % 4 == 0). Slots go four at a time: their
// pair numbers and weights, then their four output rows, are each loaded together before any is used, so a token's
// k slots cost ceil(k / 4) dependent memory round trips rather than 2k. A slot without a pair (pair_of < 0) reads
// pair 0 (out holds at least one row) and adds nothing.
__global__ __launch_bounds__(256) void moe_combine_kernel(const float* __restrict__ out, const int* __restrict__ pair_of,
                                                          const float* __restrict__ w, int rows, int k, int dmodel,
                                                          float* __restrict__ y) {
    const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
    if (i >= (int64_t)rows * dmodel) return;
    const int n = (int)(i / dmodel), d = (int)(i % dmodel);
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int j0 = 0; j0 < k; j0 += 4) {
        int p[4];
        float wj[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int j = j0 + u;
            p[u] = j < k ? pair_of[n * k + j] : -1;
            wj[u] = j < k ? w[n * k + j] : 0.0f;
        }
        f32x4 v[4];
#pragma unroll
        for (int u = 0; u < 4; u++)
            v[u] = *reinterpret_cast<const f32x4*>(out + (size_t)(p[u] < 0 ? 0 : p[u]) * dmodel + d);
#pragma unroll
        for (int u = 0; u < 4; u++) {
            if (p[u] < 0) continue;
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const float prod = wj[u] * v[u][c];
                acc[c] = acc[c] + prod;
            }
        }
    }
#pragma unroll
    for (int c = 0; c < 4; c++) y[i + c] = acc[c];
}

hipError_t launch_moe_topk(const float* logits, int rows, int n_experts, int k, int stride, int normalize, int* idx,
                           float* w, hipStream_t st) {
    const dim3 grid((rows + 63) / 64), block(64);
    if (k <= 2)
        hipLaunchKernelGGL(moe_topk_kernel<2>, grid, block, 0, st, logits, rows, n_experts, k, stride, normalize, idx, w);
    else if (k <= 4)
        hipLaunchKernelGGL(moe_topk_kernel<4>, grid, block, 0, st, logits, rows, n_experts, k, stride, normalize, idx, w);
    else if (k <= 8)
        hipLaunchKernelGGL(moe_topk_kernel<8>, grid, block, 0, st, logits, rows, n_experts, k, stride, normalize, idx, w);
    else if (k <= 16)
        hipLaunchKernelGGL(moe_topk_kernel<16>, grid, block, 0, st, logits, rows, n_experts, k, stride, normalize, idx, w);
    else
        hipLaunchKernelGGL(moe_topk_kernel<kMaxExperts>, grid, block, 0, st, logits, rows, n_experts, k, stride, normalize,
                           idx, w);
    return hipGetLastError();
}

bool moe_route_plan_fused(int rows, int k) { return rows * k <= 64 && k <= kMaxExperts; }

hipError_t launch_moe_route_plan(const float* logits, int rows, int k, int n_experts, int normalize, int* idx,
                                 float* w, int* expert_off, int* pair_row, int* pair_of, int nt, int* tiles,
                                 int* tile_count, const float* x, int64_t n_blocks, int8_t* xq, float* xs, int16_t* xb,
                                 hipStream_t st) {
    if (!moe_route_plan_fused(rows, k)) {
        hipError_t e = launch_moe_topk(logits, rows, n_experts, k, k, normalize, idx, w, st);
        if (e != hipSuccess) return e;
        return launch_moe_plan(idx, rows, k, n_experts, expert_off, pair_row, pair_of, nt, tiles, tile_count, x,
                               n_blocks, xq, xs, xb, st);
    }
    const int64_t grid = 1 + (n_blocks + 3) / 4;
#define OVFQ_ROUTE_PLAN(KM)                                                                                           \
    hipLaunchKernelGGL(moe_route_plan_kernel<KM>, dim3((unsigned)grid), dim3(256), 0, st, logits, rows, k, n_experts, \
                       normalize, idx, w, expert_off, pair_row, pair_of, nt, tiles, tile_count, x, n_blocks, xq, xs,  \
                       xb)
    if (k <= 2)
        OVFQ_ROUTE_PLAN(2);
    else if (k <= 4)
        OVFQ_ROUTE_PLAN(4);
    else if (k <= 8)
        OVFQ_ROUTE_PLAN(8);
    else if (k <= 16)
        OVFQ_ROUTE_PLAN(16);
    else
        OVFQ_ROUTE_PLAN(kMaxExperts);
#undef OVFQ_ROUTE_PLAN
    return hipGetLastError();
}

hipError_t launch_moe_plan(const int* idx, int rows, int k, int n_experts, int* expert_off, int* pair_row,
                           int* pair_of, int nt, int* tiles, int* tile_count, const float* x, int64_t n_blocks,
                           int8_t* xq, float* xs, int16_t* xb, hipStream_t st) {
    const size_t bytes = (size_t)rows * k * sizeof(int);
    const int staged = bytes <= 48 * 1024;
    const int64_t grid = 1 + (n_blocks + 3) / 4;
    hipLaunchKernelGGL(moe_plan_kernel, dim3((unsigned)grid), dim3(256), staged ? bytes : 0, st, idx, rows, k,
                       n_experts, expert_off, pair_row, pair_of, staged, nt, tiles, tile_count, x, n_blocks, xq, xs,
                       xb);
    return hipGetLastError();
}

hipError_t launch_gate_up_q8k(const float* gate, const float* up, const int* expert_off, int n_experts, int max_pairs,
                              int dff, bool gelu, int8_t* q, float* s, int16_t* b, hipStream_t st,
                              const MoeFold& fold) {
    const int spr = dff / kQK;
    const int64_t waves = (int64_t)max_pairs * spr;
    const int64_t fold_threads = std::max<int64_t>((fold.y_len + 3) / 4, fold.slots);
    const dim3 grid((unsigned)std::max((waves + 3) / 4, (fold_threads + 255) / 256)), block(256);
    if (gelu)
        hipLaunchKernelGGL(gate_up_q8k_kernel<true>, grid, block, 0, st, gate, up, expert_off, n_experts, max_pairs, spr,
                           q, s, b, fold);
    else
        hipLaunchKernelGGL(gate_up_q8k_kernel<false>, grid, block, 0, st, gate, up, expert_off, n_experts, max_pairs,
                           spr, q, s, b, fold);
    return hipGetLastError();
}

hipError_t launch_moe_combine(const float* out, const int* pair_of, const float* w, int rows, int k, int dmodel,
                              float* y, hipStream_t st) {
    const int64_t threads = (int64_t)rows * dmodel / 4;
    hipLaunchKernelGGL(moe_combine_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st, out, pair_of, w,
                       rows, k, dmodel, y);
    return hipGetLastError();
}

}  // namespace ovfq
