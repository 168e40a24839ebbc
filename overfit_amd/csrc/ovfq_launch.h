// ovfq_launch.h — host-side launchers for the ovfq kernels (internal to libovfq).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ovfq {

constexpr int kMaxJobs = 4;
constexpr int kMaxExperts = 64;

// One output matrix of a (possibly fused) projection launch. Every job of a launch shares the activation.
struct ProjJob {
    const uint8_t* w;   // Q4_K / Q6_K blocks, or the Q8_0 int8 quant plane
    const float* ws;    // Q8_0 f32 scale plane (NULL for K-quants)
    const float* bias;  // may be NULL
    float* y;           // [rows][n_rows]
    int n_rows;         // output size of this matrix
    const uint8_t* pre = nullptr;  // MFMA-ready copy of a K-quant weight (batched kernel), or NULL
};

// Q8_K activation (RT/Q4KDotKernel.cs:64-136 layout) or Q8_0 activation (bsums == NULL).
struct ActQ {
    const int8_t* q;
    const float* s;
    const int16_t* b;
    const uint16_t* bh = nullptr;  // the bsums again as fp16 (the quantiser's optional second plane), or NULL
};

// bh != NULL: the bsums are also written as fp16 (exact: |bsum| <= 16 * 127), the tiled Q4_K kernels' min-term operand.
hipError_t launch_quantize_q8k(const float* x, int64_t n_blocks, int8_t* q, float* s, int16_t* b, hipStream_t st,
                               uint16_t* bh = nullptr);
hipError_t launch_quantize_q8_0(const float* x, int64_t n_blocks, int8_t* q, float* s, hipStream_t st);

// type: 12 (Q4_K) or 14 (Q6_K). `in` % 256 == 0. rows = activation rows (M).
hipError_t launch_project_kquant(int type, const ProjJob* jobs, int njobs, int in, int rows, ActQ act,
                                 hipStream_t st);
// Decode (M = 1) K-quant projection with the activation staged in LDS: x != NULL quantises the fp32 activation
// inside the launch; x == NULL copies the prequantised `act`. Requires gemv_supported(in).
bool gemv_supported(int in);
bool gemv_quantize_inside(int in);
// Decode kernel over 1 .. 8 activation rows (rows * in / 256 <= 128; one row only where gemv_supported fails): from
// the fp32 rows x, quantised inside the launch (requires gemv_rows_quantize_inside), or, x == NULL, from the
// prequantised `act`.
bool gemv_rows_supported(int in, int rows);
bool gemv_rows_quantize_inside(int in, int rows);
hipError_t launch_gemv_rows_kquant(int type, const ProjJob* jobs, int njobs, int in, int rows, const float* x,
                                   ActQ act, hipStream_t st);
hipError_t launch_gemv_kquant(int type, const ProjJob* jobs, int njobs, int in, const float* x, ActQ act,
                              hipStream_t st);
// Batched K-quant projection on int8 MFMA over 64-row weight tiles x 64/128-row activation tiles; bit-identical
// to launch_project_kquant at any rows.
bool mfma_supported(int type);
// Automatic choice of that kernel over the small-M kernel for `rows` activation rows against weights of `o_tiles`
// 64-row tiles and `out_rows` output rows in all (both kernels able to run).
bool mfma_tiled_preferred(int type, int rows, int o_tiles, long out_rows);
// Rows from which the tiled kernel runs where the small-M kernel cannot (input sizes past 16384).
constexpr int kMfmaMinRows = 32;
hipError_t launch_project_mfma(int type, const ProjJob* jobs, int njobs, int in, int rows, ActQ act,
                               hipStream_t st);
// Small-batch / grouped-expert K-quant projection. One or two matrices per expert (gate, up) of equal shape;
// expert_off/pair_row (device arrays) select each expert's activation rows, or NULL for a single expert over
// activation rows 0..rows-1 (outputs row-major [pairs][n_rows]).
struct GroupLaunch {
    const uint8_t* const* w0;  // [experts]
    const uint8_t* const* w1;  // [experts] or NULL
    const float* bias0;        // single expert only
    const float* bias1;
    float* y0;
    float* y1;
    int n_rows;
    int in;
    int experts;
    int rows;
    const int* expert_off;
    const int* pair_row;
    ActQ act;
    int pairs = 0;  // grouped launches: the pair count bound (rows x top_k), sizing the pair -> row map
    // Grouped single-matrix launch_mfma_small launches only: instead of storing y0[pair][o], add
    // comb_w[pair] * value to comb[comb_tok[pair]][o] with a float atomic (comb zeroed beforehand). Exact when at
    // most two pairs add to one output: (0 + a) + b == (0 + b) + a in fp32.
    float* comb = nullptr;
    const int* comb_tok = nullptr;
    const float* comb_w = nullptr;
};
// On MFMA with super-block-parallel waves (mfma.hip), 16 activation rows per tile.
bool mfma_small_supported(int type, int in);
// Whether a gate/up-shaped pair of Q4_K weights (n_rows outputs each, `in` inputs) runs on the expert-stream kernel
// when it takes the small-M path.
bool stream_pair_preferred(int type, int in, int n_rows);
hipError_t launch_mfma_small(int type, const GroupLaunch& launch, hipStream_t st);
// MFMA-ready copy of a Q4_K / Q6_K weight: its size, and the kernel that writes it from the GGUF blocks.
size_t mfma_prepared_bytes(int in, int out);
hipError_t launch_mfma_prepare(int type, const uint8_t* w, int in, int out, uint8_t* pre, hipStream_t st);

// Routed MoE (moe.hip).
hipError_t launch_moe_topk(const float* logits, int rows, int n_experts, int k, int stride, int normalize, int* idx,
                           float* w, hipStream_t st);
// `tiles` (optional, else NULL): the experts' pair ranges in tiles of `nt` rows (expert | tile << 8), the count at
// *tile_count; at most ceil(rows * k / nt) + n_experts entries. The same launch quantises the n_blocks Q8_K blocks
// of x into xq / xs / xb (n_blocks may be 0).
hipError_t launch_moe_plan(const int* idx, int rows, int k, int n_experts, int* expert_off, int* pair_row,
                           int* pair_of, int nt, int* tiles, int* tile_count, const float* x, int64_t n_blocks,
                           int8_t* xq, float* xs, int16_t* xb, hipStream_t st);
// Router top-k (writing idx / w [rows][k]) and the plan above from router logits [rows][n_experts] (k <=
// n_experts): one launch when moe_route_plan_fused(rows, k), else launch_moe_topk then launch_moe_plan.
bool moe_route_plan_fused(int rows, int k);
hipError_t launch_moe_route_plan(const float* logits, int rows, int k, int n_experts, int normalize, int* idx,
                                 float* w, int* expert_off, int* pair_row, int* pair_of, int nt, int* tiles,
                                 int* tile_count, const float* x, int64_t n_blocks, int8_t* xq, float* xs, int16_t* xb,
                                 hipStream_t st);
// The batched int8-MFMA kernel over expert groups: tile list entry t covers rows [64 i, 64 i + 64) of expert e's
// pairs; gate/up pairs (w1 set) share the launch. Activation rows are gathered through pair_row (NULL: pair p reads
// row p); outputs are pair-major.
hipError_t launch_mfma_grouped(int type, const GroupLaunch& launch, const int* tiles, const int* tile_count,
                               int max_tiles, hipStream_t st);
constexpr int kGroupedTileRows = 64;
// Work for a MoE step whose down projection adds into its output (GroupLaunch::comb), done in the launch before it:
// y[0 .. y_len) = 0, and pw[pair_of[i]] = w[i] for the slots i < slots that hold a pair (pair_of[i] >= 0).
struct MoeFold {
    float* y = nullptr;
    int64_t y_len = 0;
    const int* pair_of = nullptr;
    const float* w = nullptr;
    int slots = 0;
    float* pw = nullptr;
};
// act(gate) * up (act: SiLU, or GELU with the tanh approximation), quantised to Q8_K for the down projection.
hipError_t launch_gate_up_q8k(const float* gate, const float* up, const int* expert_off, int n_experts, int max_pairs,
                              int dff, bool gelu, int8_t* q, float* s, int16_t* b, hipStream_t st,
                              const MoeFold& fold = MoeFold{});
hipError_t launch_moe_combine(const float* out, const int* pair_of, const float* w, int rows, int k, int dmodel,
                              float* y, hipStream_t st);

hipError_t launch_project_q8_0(const ProjJob* jobs, int njobs, int in, int rows, ActQ act, hipStream_t st);
// Q8_0 decode (M = 1) on a persistent grid with the activation in LDS (K <= 32768), bit-identical to
// launch_project_q8_0: from the fp32 x, quantised inside the launch (requires q8_0_gemv_quantize_inside), or,
// x == NULL, from the prequantised `act`.
// With 2 .. 8 activation rows (rows * in <= 32768) from the prequantised `act` only: each block is loaded once and
// dotted with every row.
bool q8_0_gemv_supported(int in);
bool q8_0_gemv_rows_supported(int in, int rows);
bool q8_0_gemv_quantize_inside(int in);
hipError_t launch_q8_0_gemv(const ProjJob* jobs, int njobs, int in, int rows, const float* x, ActQ act,
                            hipStream_t st);
// Q8_0 over several activation rows on int8 MFMA (one 16x16x32 MFMA per 32-element block), bit-identical to
// launch_project_q8_0.
bool q8_0_mfma_supported(int in, int rows);
hipError_t launch_project_q8_0_mfma(const ProjJob* jobs, int njobs, int in, int rows, ActQ act, hipStream_t st);

// Fixed device scratch of ovfq_project_noalloc_dev (noalloc.hip): one copy per GPU, kNoAllocScratchBytes long.
// noalloc_scratch_init(device) resolves the current device's copy (call with `device` current, once per
// device; later calls return at once); noalloc_scratch(device) returns its device address, NULL before init.
// Activation rows x input size up to kNoAllocMaxElems fit (Q8_K: n + n/8 + n/64 bytes, Q8_0: n + n/8, each
// piece 256-byte aligned).
constexpr int64_t kNoAllocMaxElems = (int64_t)1 << 21;
constexpr size_t kNoAllocScratchBytes = (size_t)5 << 19;  // 2.5 MiB
hipError_t noalloc_scratch_init(int device);
void* noalloc_scratch(int device);

// Attention output projection with per-head Q8_0 Wo (heads.hip): y[rows][d_model] = (bias or 0) + the heads'
// projections of their head_dim slices of x, added in ascending head order, in one launch. wq[h] / ws[h] are head h's
// int8 [d_model][head_dim] and f32 [d_model][head_dim / 32] planes. From the fp32 x (quantised to Q8_0 inside the
// launch; requires q8_0_heads_quantize_inside) or, x == NULL, a Q8_0 activation [rows][n_heads * head_dim].
constexpr int kHeadsMax = 128;          // heads per launch
constexpr int kHeadsMaxDim = 256;       // head_dim
constexpr int kHeadsMaxRows = 8;        // activation rows per launch
constexpr int kHeadsMaxIn = 32768;      // rows * n_heads * head_dim staged in LDS
constexpr int kHeadsMaxRowHeads = 256;  // rows * n_heads head values kept in LDS
constexpr size_t kHeadsMaxLds = 65536;
bool q8_0_heads_supported(int n_heads, int head_dim, int rows);
bool q8_0_heads_quantize_inside(int n_heads, int head_dim, int rows);
size_t q8_0_heads_lds_bytes(int n_heads, int head_dim, int rows);
hipError_t launch_q8_0_heads(const int8_t* const* wq, const float* const* ws, int n_heads, int head_dim, int d_model,
                             int rows, const float* bias, const float* x, ActQ act, float* y, hipStream_t st);
// The same projection for batches on int8 MFMA (project.hip): 64 outputs x 16-64 activation rows per workgroup, the
// contraction walked head by head; act is the Q8_0 activation [rows][n_heads * head_dim].
bool q8_0_heads_mfma_supported(int n_heads, int head_dim, int rows);
hipError_t launch_q8_0_heads_mfma(const int8_t* const* wq, const float* const* ws, int n_heads, int head_dim,
                                  int d_model, int rows, const float* bias, ActQ act, float* y, hipStream_t st);

// GGUF Q8_0 (34-byte blocks) -> int8 quant plane + f32 scale plane.
hipError_t launch_q8_0_deinterleave(const void* gguf, int64_t n_blocks, int8_t* q, float* s, hipStream_t st);
// GGUF Q5_0 (22-byte blocks of 32) or Q5_K (176-byte super-blocks) -> resident Q8_0 planes: decoded and requantised
// in registers; n_blocks counts 32-element blocks.
hipError_t launch_q5_to_q8_0(const void* gguf, bool q5k, int64_t n_blocks, int8_t* q, float* s, hipStream_t st);
hipError_t launch_encode_q4k(const float* w, int64_t n_blocks, uint8_t* dst, hipStream_t st);
hipError_t launch_encode_q6k(const float* w, int64_t n_blocks, uint8_t* dst, hipStream_t st);

// Row dequantisation (type 8/12/14). For Q8_0, `blocks` is the quant plane and `scales` the scale plane.
hipError_t launch_decode_row(int type, const void* blocks, const float* scales, int in, int row, float* dst,
                             hipStream_t st);

}  // namespace ovfq
