/*
 * ovfq.h — C ABI of libovfq, the MI355X (gfx950) GGUF quantized-linear library.
 *
 * Drop-in device backing for Overfit's CPU quantized projections. Reference paths are relative to the
 * reference root; RT/ = Sources/Main/LanguageModels/Runtime/, LD/ = Sources/Main/LanguageModels/Loading/.
 *
 * Conventions (kept from the reference, RT/Q4KDotKernel.cs:77-97, :957-976):
 *  - Every entry point validates its arguments BEFORE any device work and returns a status code instead of
 *    throwing: OVFQ_ERR_NULL ~ ArgumentNullException, OVFQ_ERR_SIZE ~ ArgumentException,
 *    OVFQ_ERR_RANGE ~ ArgumentOutOfRangeException. ovfq_last_error() gives the message (per thread).
 *  - Outputs are overwritten, never accumulated. A NULL bias means "no bias" (the reference's empty span).
 *  - Weights are immutable after creation; they are copied to HBM once, in their native GGUF layout
 *    (Q4_K 144-byte and Q6_K 210-byte super-blocks, output-major), or as the reference's resident Q8_0 planes
 *    (int8 quants + f32 scales, RT/Q8Weight.cs:21-75).
 *  - Host-pointer entry points (no suffix) are synchronous, like the reference's calls: they return after the
 *    output is written, and never retain a host pointer.
 *  - Entry points with the _dev suffix take device pointers and enqueue on the context's stream (see
 *    ovfq_ctx_set_stream); they return once the work is enqueued. Call ovfq_ctx_synchronize() to wait.
 *  - Thread safety: any number of host threads may call into one context; calls are serialised by a
 *    per-context lock and run in order on the context's stream (the reference calls Project concurrently from
 *    its head-parallel workers, RT/CachedMultiHeadAttention.cs:280, :876-907).
 *  - Lifetime: a weight belongs to the context it was created on, and that context must outlive it
 *    (ovfq_ctx_destroy returns OVFQ_ERR_STATE, destroying nothing, while any of its weights is alive; the
 *    reference's counterpart of that state error is InvalidOperationException).
 *  - Sizes: every activation and output plane (rows x its width) stays below 2^31 elements, the length limit
 *    of the reference's Span<T> scratch and outputs; larger calls return OVFQ_ERR_SIZE.
 *  - Scratch and HIP graphs: the context grows its device scratch on demand (activation quantisation, FFN and
 *    MoE intermediates, host staging) and never frees a superseded buffer before ovfq_ctx_destroy (or
 *    ovfq_ctx_release_retired), so a graph captured from _dev calls stays valid after later, larger calls on the
 *    same context. Work captured into a graph and work issued eagerly on the same context share that scratch:
 *    they must not run concurrently.
 */
#ifndef OVFQ_H
#define OVFQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OVFQ_API __attribute__((visibility("default")))

/* Status codes. */
#define OVFQ_OK 0
#define OVFQ_ERR_NULL (-1)  /* a required pointer was NULL                */
#define OVFQ_ERR_SIZE (-2)  /* a size or shape is inconsistent            */
#define OVFQ_ERR_RANGE (-3) /* a count is zero/negative or an index is out of range */
#define OVFQ_ERR_TYPE (-4)  /* unsupported weight type for this entry point */
#define OVFQ_ERR_STATE (-5) /* the object's state forbids the call (a context that still owns weights) */
#define OVFQ_ERR_HIP (-10)  /* the HIP runtime reported an error          */

/* Weight formats (numbered as ggml's type ids). */
#define OVFQ_TYPE_Q8_0 8
#define OVFQ_TYPE_Q4_K 12
#define OVFQ_TYPE_Q6_K 14
/* GGUF-only source types: ovfq_weight_create_gguf / _experts_gguf turn them into resident Q8_0 weights. */
#define OVFQ_TYPE_Q5_0 6
#define OVFQ_TYPE_Q5_K 13

/* Block geometry. */
#define OVFQ_QK 256          /* elements per K-quant super-block (RT/Q4KWeight.cs:26) */
#define OVFQ_Q4K_BYTES 144   /* RT/Q4KWeight.cs:29 */
#define OVFQ_Q6K_BYTES 210   /* RT/Q6KWeight.cs SuperBlockBytes */
#define OVFQ_Q8_BLOCK 32     /* RT/Q8DotKernel.cs:34 */
#define OVFQ_GROUP 16        /* Q8_K bsum group (RT/Q4KDotKernel.cs:47) */

typedef struct ovfq_ctx ovfq_ctx;
typedef struct ovfq_weight ovfq_weight;

/* ------------------------------------------------------------------------------------------------ context */

/* Creates a context on HIP device `device` with its own (default-priority) stream. New; the reference has
 * no device context. */
OVFQ_API int ovfq_ctx_create(int device, ovfq_ctx** out);
OVFQ_API int ovfq_ctx_destroy(ovfq_ctx* ctx);
/* Makes the context enqueue its work on `stream` (a hipStream_t; NULL is the device's null stream). Work
 * already queued on the previous stream is waited for first. */
OVFQ_API int ovfq_ctx_set_stream(ovfq_ctx* ctx, void* stream);
/* Returns the context to its own stream. */
OVFQ_API int ovfq_ctx_reset_stream(ovfq_ctx* ctx);
OVFQ_API int ovfq_ctx_synchronize(ovfq_ctx* ctx);
/* Frees the scratch buffers that later, larger calls have superseded (kept until now so that HIP graphs captured
 * from earlier _dev calls stay valid). Waits for the context's stream first. Only for callers that hold no graph
 * captured from this context's calls, or have destroyed every such graph: replaying one afterwards reads freed
 * memory. New; the reference has no device scratch. */
OVFQ_API int ovfq_ctx_release_retired(ovfq_ctx* ctx);
/* Device scratch the context holds: `live` bytes in use by its growable buffers, `retired` bytes of superseded
 * buffers kept for captured graphs (either pointer may be NULL). New; for serving code that watches memory. */
OVFQ_API int ovfq_ctx_scratch_bytes(ovfq_ctx* ctx, size_t* live, size_t* retired);
/* Kernel choice for batched K-quant work of 2 or more activation rows (projections, fused q/k/v and gate/up
 * launches, the SwiGLU FFN, routed expert groups). OVFQ_BATCHED_AUTO (the default) picks by shape;
 * OVFQ_BATCHED_SMALL forces the super-block-parallel small-M MFMA kernel wherever it takes the shape (3 or more
 * rows, input sizes up to 16384); OVFQ_BATCHED_TILED the 64-row-tiled MFMA kernel (3 or more rows);
 * OVFQ_BATCHED_ROWS the multi-row decode kernel (2 to 8 rows, rows * input_size <= 32768). Shapes a forced
 * kernel does not take keep the automatic choice (routed experts: only SMALL / TILED apply). For Q8_0 weights,
 * TILED forces the tiled int8-MFMA kernel from 2 rows, ROWS the multi-row decode kernel (up to 8 rows, rows *
 * input_size <= 32768) and SMALL the row kernel (automatic: the decode kernel where it takes the shape, else the MFMA
 * kernel from 8 rows, for inputs up to 8192 from 6 rows, or from 4 with 8192 outputs or more). Every choice gives
 * bit-identical outputs. Counterpart of the reference's test-only A/B toggle
 * BatchedQuantProjection.UseWeightStationaryQ4K (RT/BatchedQuantProjection.cs:21-24): for parity tests and
 * benches that cover every kernel on one shape. */
#define OVFQ_BATCHED_AUTO 0
#define OVFQ_BATCHED_SMALL 1
#define OVFQ_BATCHED_TILED 2
#define OVFQ_BATCHED_ROWS 3
OVFQ_API int ovfq_ctx_set_batched_kernel(ovfq_ctx* ctx, int kernel);
/* Message for the last non-zero status returned on the calling thread ("" if none). */
OVFQ_API const char* ovfq_last_error(void);
/* Library version string. */
OVFQ_API const char* ovfq_version(void);

/* ------------------------------------------------------------------------------------------------ weights */

/* Replaces the constructors Q4KWeight(ReadOnlyMemory<byte> blocks, int inputSize, int outputSize)
 * (RT/Q4KWeight.cs:44-66) and Q6KWeight(...) (RT/Q6KWeight.cs:47): `blocks` holds output_size rows of
 * input_size/256 super-blocks (host memory, e.g. a slice of a memory-mapped GGUF file); `nbytes` is the
 * region length and must be >= the expected size. For Q8_0 (Q8Weight(sbyte[] quants, float[] scales, int
 * inputSize, int outputSize), RT/Q8Weight.cs:23-50) `blocks` is the int8 quant plane [out*in] and `q8_scales`
 * the f32 scale plane [out*in/32]; `nbytes` is the quant plane length. The bytes are copied once to HBM. */
OVFQ_API int ovfq_weight_create(ovfq_ctx* ctx, int type, const void* blocks, size_t nbytes,
                                const float* q8_scales, int input_size, int output_size, ovfq_weight** out);
/* As ovfq_weight_create, but `blocks` / `q8_scales` are device pointers (device-to-device copy). */
OVFQ_API int ovfq_weight_create_from_device(ovfq_ctx* ctx, int type, const void* blocks, size_t nbytes,
                                            const float* q8_scales, int input_size, int output_size,
                                            ovfq_weight** out);
/* A tensor exactly as stored in a GGUF file (a slice of the memory-mapped file): Q4_K / Q6_K super-blocks are
 * uploaded verbatim (GgufReader.LoadTensorQ4_KRaw / Q6_KRaw, LD/GgufReader.cs:276-344); Q8_0's 34-byte blocks (fp16 d +
 * 32 int8, GgufReader.LoadTensorQ8_0Raw, LD/GgufReader.cs:198-266) are de-interleaved on the device into the
 * resident int8 quant plane and f32 scale plane (d widened exactly). Q5_0 (22-byte blocks of 32) and Q5_K (176-byte
 * super-blocks) tensors become resident Q8_0 weights as the reference's loader makes them (LD/GgufLlamaLoader.cs:
 * 665-680 and its F32 fallback for per-layer tensors): every block decoded exactly as GgmlDequant.DecodeQ5_0Block /
 * DecodeQ5_KBlock (LD/GgmlDequant.cs:222-320), then requantised with Q8Weight.QuantizeRows (RT/Q8Weight.cs:115-175),
 * both on the device; ovfq_weight_info then reports OVFQ_TYPE_Q8_0. `nbytes` must cover output_size rows. */
OVFQ_API int ovfq_weight_create_gguf(ovfq_ctx* ctx, int type, const void* gguf_bytes, size_t nbytes, int input_size,
                                     int output_size, ovfq_weight** out);
/* As ovfq_weight_create_gguf, from device memory. */
OVFQ_API int ovfq_weight_create_gguf_dev(ovfq_ctx* ctx, int type, const void* gguf_bytes, size_t nbytes,
                                         int input_size, int output_size, ovfq_weight** out);
/* Replaces GgufLlamaLoader.LoadExperts (LD/GgufLlamaLoader.cs:600-690) for Q4_K / Q5_0 / Q5_K / Q6_K / Q8_0: a 3-D
 * expert tensor
 * (ffn_gate_exps / ffn_up_exps / ffn_down_exps) as stored in a GGUF file, dims [ne0 = input_size, ne1 = output_size,
 * ne2 = n_experts] with the expert axis slowest, -> n_experts weights written to out[0 .. n_experts). Each expert is
 * the contiguous slice e of the tensor: Q4_K / Q6_K bytes verbatim, Q8_0 blocks de-interleaved per expert, Q5_0 / Q5_K
 * decoded and requantised to Q8_0 per expert (as ovfq_weight_create_gguf does; LD/GgufLlamaLoader.cs:665-680). All experts
 * share one device allocation (each slice 256-byte aligned), freed when the last of them is destroyed; each is
 * destroyed with ovfq_weight_destroy like any weight. `nbytes` must cover n_experts slices. 1 <= n_experts <=
 * OVFQ_MAX_EXPERT_SLICES. */
#define OVFQ_MAX_EXPERT_SLICES 4096
OVFQ_API int ovfq_weight_create_experts_gguf(ovfq_ctx* ctx, int type, const void* gguf_bytes, size_t nbytes,
                                             int input_size, int output_size, int n_experts, ovfq_weight** out);
/* As ovfq_weight_create_experts_gguf, from device memory. */
OVFQ_API int ovfq_weight_create_experts_gguf_dev(ovfq_ctx* ctx, int type, const void* gguf_bytes, size_t nbytes,
                                                 int input_size, int output_size, int n_experts, ovfq_weight** out);
OVFQ_API int ovfq_weight_destroy(ovfq_weight* w);
/* Opt-in MFMA-ready copy of a Q6_K weight, written on the device: for every 16 output rows and super-block, the
 * int8 weight operands the batched (M >= 32) int8-MFMA kernel otherwise rebuilds from the GGUF bytes for every
 * activation tile, plus the block scale. Batched projections whose weights all have it skip that build; outputs
 * are bit-identical with or without it. Costs 8704 bytes per 16 rows and super-block (~2.5x the Q6_K bytes), freed
 * with the weight; the GGUF blocks stay resident for decode. Idempotent. For a Q4_K weight the call succeeds and
 * changes nothing (its operands are cheaper to build than to stream); other types: OVFQ_ERR_TYPE. The reference's
 * counterpart is its opt-in repacked CPU layout (RT/Q4KRepack.cs, RT/Q6KRepack.cs): a load-time layout change
 * trading memory for throughput. */
OVFQ_API int ovfq_weight_prepare_mfma(ovfq_ctx* ctx, ovfq_weight* w);
/* Shape/format query (InputSize / OutputSize / ByteCount of the weight classes). Any out pointer may be NULL.
 * `device_blocks` receives the HBM address of the resident blocks (the quant plane for Q8_0). */
OVFQ_API int ovfq_weight_info(const ovfq_weight* w, int* type, int* input_size, int* output_size,
                              size_t* byte_count, const void** device_blocks);

/* DecodeRow (RT/Q4KWeight.cs:121-138, RT/Q6KWeight.cs DecodeRow, RT/Q8Weight.cs:81-106): dequantises output
 * row `row` into dst[input_size] (F32, e.g. an embedding lookup). */
OVFQ_API int ovfq_weight_decode_row(ovfq_ctx* ctx, const ovfq_weight* w, int row, float* dst);
OVFQ_API int ovfq_weight_decode_row_dev(ovfq_ctx* ctx, const ovfq_weight* w, int row, float* dst_dev);

/* ------------------------------------------------------------------------------ activation quantisation */

/* Q4KDotKernel.QuantizeActivationQ8K (RT/Q4KDotKernel.cs:71-136), applied to `rows` rows of length k
 * (k % 256 == 0): quants[rows*k] int8, scales[rows*k/256] f32, bsums[rows*k/16] int16 — the reference's
 * caller-owned scratch layout. Bit-exact to the reference. */
OVFQ_API int ovfq_quantize_q8k(ovfq_ctx* ctx, const float* x, int rows, int k, int8_t* quants, float* scales,
                               int16_t* bsums);
OVFQ_API int ovfq_quantize_q8k_dev(ovfq_ctx* ctx, const float* x, int rows, int k, int8_t* quants,
                                   float* scales, int16_t* bsums);
/* Q8DotKernel.Quantize (RT/Q8DotKernel.cs:42-91) row by row (k % 32 == 0): quants[rows*k], scales[rows*k/32]. */
OVFQ_API int ovfq_quantize_q8_0(ovfq_ctx* ctx, const float* x, int rows, int k, int8_t* quants, float* scales);
OVFQ_API int ovfq_quantize_q8_0_dev(ovfq_ctx* ctx, const float* x, int rows, int k, int8_t* quants,
                                    float* scales);

/* ------------------------------------------------------------------------------------------- projections */

/* y[rows][out] = (bias +) x[rows][in] @ W^T.
 *  rows == 1 replaces Q4KDotKernel.Project / ProjectParallel (RT/Q4KDotKernel.cs:414-552),
 *  Q6KDotKernel.Project / ProjectParallel (RT/Q6KDotKernel.cs:245-381) and Q8DotKernel.Project /
 *  ProjectParallel (RT/Q8DotKernel.cs:155-330);
 *  rows >= 2 replaces ProjectBatched / ProjectBatchedWeightStationary (RT/Q4KDotKernel.cs:681-955,
 *  RT/Q6KDotKernel.cs:403-510, RT/Q8DotKernel.cs:352-445) and BatchedQuantProjection.Dispatch
 *  (RT/BatchedQuantProjection.cs:26-87). The activation is quantised on the device (Q8_K for Q4_K/Q6_K,
 *  Q8_0 for Q8_0), exactly as the reference does. */
OVFQ_API int ovfq_project(ovfq_ctx* ctx, const ovfq_weight* w, const float* x, int rows, const float* bias,
                          float* y);
OVFQ_API int ovfq_project_dev(ovfq_ctx* ctx, const ovfq_weight* w, const float* x, int rows,
                              const float* bias, float* y);

/* ovfq_project_dev that allocates nothing. No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments, kernels and bit-identical outputs as ovfq_project_dev; where that entry point quantises the
 * activation into the context's growable scratch, this one uses a fixed device array of 2.5 MiB that the
 * library holds on every GPU it runs on until the process ends. rows * input_size is limited to 2^21
 * (OVFQ_NOALLOC_MAX_ELEMS; e.g. 512 rows of 4096); larger calls return OVFQ_ERR_SIZE. Every call on one GPU
 * uses that GPU's one array, through any context: calls that may overlap on a GPU (two contexts, or two
 * streams) race and must be serialised by the caller. */
#define OVFQ_NOALLOC_MAX_ELEMS (1 << 21)
OVFQ_API int ovfq_project_noalloc_dev(ovfq_ctx* ctx, const ovfq_weight* w, const float* x, int rows,
                                      const float* bias, float* y);

/* Q4KDotKernel.ProjectPreQuantized (RT/Q4KDotKernel.cs:445-476) / Q6KDotKernel.ProjectPreQuantized
 * (RT/Q6KDotKernel.cs:274-305), for `rows` rows of an already-quantised Q8_K activation in the layout
 * ovfq_quantize_q8k writes. For Q8_0 weights pass the Q8_0 activation scales in `scales` and NULL bsums.
 * Precondition, as in the reference: bsums[g] is the sum of the 16 quants of group g (QuantizeActivationQ8K's
 * definition, RT/Q4KDotKernel.cs:122-135), which every quantiser here writes. The decode kernels (1 to 8 rows)
 * read the bsums plane as the reference's Dot does, and so does the tiled Q4_K MFMA kernel of large batches (as
 * fp16, exact for every group sum: |bsums| <= 2032); the other MFMA kernels form the same sums from the quants
 * themselves. Bsums that are not those sums therefore give results that depend on the row count. */
OVFQ_API int ovfq_project_prequantized(ovfq_ctx* ctx, const ovfq_weight* w, const int8_t* quants,
                                       const float* scales, const int16_t* bsums, int rows, const float* bias,
                                       float* y);
OVFQ_API int ovfq_project_prequantized_dev(ovfq_ctx* ctx, const ovfq_weight* w, const int8_t* quants,
                                           const float* scales, const int16_t* bsums, int rows,
                                           const float* bias, float* y);

/* Q4KDotKernel.ProjectGateUpParallel (RT/Q4KDotKernel.cs:563-645): one activation quantisation, gate and up
 * in one launch; no bias. gate and up must have equal shapes. Any K-quant/Q8_0 type is accepted as long as
 * both weights share it. */
OVFQ_API int ovfq_project_gate_up(ovfq_ctx* ctx, const ovfq_weight* gate, const ovfq_weight* up,
                                  const float* x, float* gate_out, float* up_out);
OVFQ_API int ovfq_project_gate_up_dev(ovfq_ctx* ctx, const ovfq_weight* gate, const ovfq_weight* up,
                                      const float* x, float* gate_out, float* up_out);

/* Several projections of the SAME activation in one launch: the attention block quantises its hidden row once
 * (QuantizeActivationQ8K) and runs the q, k and v projections against it with ProjectPreQuantized
 * (RT/CachedMultiHeadAttention.cs:196-207, RT/Q4KDotKernel.cs:445-476); gate/up is the two-weight case
 * (ProjectGateUpParallel, RT/Q4KDotKernel.cs:563-645). weights[i] share input_size and type; x is rows x input_size;
 * ys[i] receives rows x output_size_i; biases may be NULL or hold NULL entries. At most 4 weights. Host pointers,
 * synchronous (one upload of x, one launch, the outputs downloaded together). Prefill (rows >= 2) uses it for the
 * fused q/k/v and gate/up GEMMs. */
OVFQ_API int ovfq_project_multi(ovfq_ctx* ctx, int count, const ovfq_weight* const* weights, const float* x,
                                int rows, const float* const* biases, float* const* ys);
/* As ovfq_project_multi, with device pointers (enqueued on the context's stream). */
OVFQ_API int ovfq_project_multi_dev(ovfq_ctx* ctx, int count, const ovfq_weight* const* weights,
                                    const float* x, int rows, const float* const* biases, float* const* ys);

/* ovfq_project_multi_dev from an already-quantised Q8_K activation (rows rows): the attention block quantises
 * its hidden row once and runs every head's projection against it with ProjectPreQuantized
 * (RT/CachedMultiHeadAttention.cs:196-207, RT/Q4KDotKernel.cs:445-476); here all of them run in one launch.
 * K-quant weights only; at most 4. */
OVFQ_API int ovfq_project_multi_prequantized_dev(ovfq_ctx* ctx, int count, const ovfq_weight* const* weights,
                                                 const int8_t* quants, const float* scales, const int16_t* bsums,
                                                 int rows, const float* const* biases, float* const* ys);

/* ---------------------------------------------------------------------------- per-head attention output */

#define OVFQ_MAX_HEADS 128

/* The attention output projection of the reference's default Llama decode path, where Wo is requantised per head to
 * Q8_0 (LD/GgufLlamaLoader.cs:977-995, SplitOutput :1298-1336): wo[h] is head h's Q8_0 weight of input_size head_dim
 * and output_size d_model (all heads one shape; head_dim <= 256, n_heads <= OVFQ_MAX_HEADS). For every row n of
 * x [rows][n_heads * head_dim] (head h's attention output at columns h * head_dim ..):
 *   y[n] = bias (or zero), then for h = 0, 1, ..., n_heads - 1:  y[n] += Q8DotKernel.Project(x[n][h], wo[h]) (no bias)
 * — the per-head projections of RT/CachedSingleHeadAttention.cs:323-337 and the ascending head reduction of
 * RT/CachedMultiHeadAttention.cs:185-194, :292-297 (prefill rows: :600-614, :689-711), bit-identical. Up to 8 rows run
 * in one decode launch, up to 31 in launches of 8; batches of 32 rows or more (prefill) quantise the rows once and run
 * on int8 MFMA, each head's Wo streamed once per 64 rows (ovfq_ctx_set_batched_kernel: OVFQ_BATCHED_TILED forces that
 * kernel, SMALL / ROWS the decode launches). Replaces the n_heads separate projections plus the host sum. */
OVFQ_API int ovfq_project_heads_q8_0(ovfq_ctx* ctx, int n_heads, const ovfq_weight* const* wo, const float* x,
                                     int rows, const float* bias, float* y);
OVFQ_API int ovfq_project_heads_q8_0_dev(ovfq_ctx* ctx, int n_heads, const ovfq_weight* const* wo, const float* x,
                                         int rows, const float* bias, float* y);

/* ---------------------------------------------------------------------------------- gated FFN */

/* CachedFeedForwardBlock.DecodeSwiGluDispatched / DecodeSwiGluBatchedDispatched (RT/CachedFeedForwardBlock.cs:
 * 261-344) on the device: y[rows][d_model] = down(SiLU(gate(x)) * up(x)) for x[rows][d_model], gate/up
 * [d_ff][d_model] of one K-quant type, down [d_model][d_ff] K-quant. Three launches (gate/up, SiLU*up with the
 * Q8_K quantisation of the down input, down) and no host round trip. The projections are bit-identical to the
 * reference's; SiLU uses expf (the reference's TensorPrimitives.Sigmoid is itself few-ULP), so y matches to the
 * projection tolerance. No counterpart entry point in the reference (it runs the steps on the host). */
OVFQ_API int ovfq_ffn_swiglu(ovfq_ctx* ctx, const ovfq_weight* gate, const ovfq_weight* up, const ovfq_weight* down,
                             const float* x, int rows, float* y);
OVFQ_API int ovfq_ffn_swiglu_dev(ovfq_ctx* ctx, const ovfq_weight* gate, const ovfq_weight* up,
                                 const ovfq_weight* down, const float* x, int rows, float* y);

/* FeedForwardActivation's gated values (Runtime/FeedForwardActivation.cs:27, :33). */
#define OVFQ_FFN_SWIGLU 3 /* gate activation SiLU (Llama, Mistral, Qwen, Phi)      */
#define OVFQ_FFN_GEGLU 4  /* gate activation GELU, tanh approximation (Gemma)      */

/* The same FFN with the gate activation chosen as CachedFeedForwardBlock.ApplyGate does (RT/CachedFeedForwardBlock.cs:
 * 474-485): OVFQ_FFN_SWIGLU is ovfq_ffn_swiglu; OVFQ_FFN_GEGLU applies 0.5 g (1 + tanh(sqrt(2/pi) (g + 0.044715
 * g^3))) in ApplyGeLU's operation order (:498-517) with the device tanhf. Any other activation -> OVFQ_ERR_RANGE. */
OVFQ_API int ovfq_ffn_gated(ovfq_ctx* ctx, const ovfq_weight* gate, const ovfq_weight* up, const ovfq_weight* down,
                            const float* x, int rows, int activation, float* y);
OVFQ_API int ovfq_ffn_gated_dev(ovfq_ctx* ctx, const ovfq_weight* gate, const ovfq_weight* up,
                                const ovfq_weight* down, const float* x, int rows, int activation, float* y);

/* ---------------------------------------------------------------------------------- routed MoE */

#define OVFQ_MAX_EXPERTS 64

/* MoeRouter.SelectTopK (RT/MoeRouter.cs:40-128) for each of `rows` tokens: logits [rows][n_experts] ->
 * expert_indices / expert_weights [rows][top_k], indices descending by logit (ties keep the lower index),
 * weights the softmax over the kept logits (normalize != 0) or the full softmax at them (normalize == 0).
 * When top_k > n_experts only the first n_experts slots of each row are written (the reference returns
 * min(topK, n)). n_experts <= OVFQ_MAX_EXPERTS. The weights go through expf, so they match the reference to
 * within a few ULP; the indices are exact. */
OVFQ_API int ovfq_moe_select_topk(ovfq_ctx* ctx, const float* logits, int rows, int n_experts, int top_k,
                                  int normalize, int* expert_indices, float* expert_weights);
OVFQ_API int ovfq_moe_select_topk_dev(ovfq_ctx* ctx, const float* logits, int rows, int n_experts, int top_k,
                                      int normalize, int* expert_indices, float* expert_weights);

/* MoeFeedForwardBlock.DecodeBatched (RT/MoeFeedForwardBlock.cs:140-241) after routing: for `rows` tokens x
 * [rows][d_model] with their top_k experts (indices/weights [rows][top_k], e.g. from ovfq_moe_select_topk),
 * groups the tokens by expert, runs each used expert's SwiGLU FFN (gate/up [d_ff][d_model], down
 * [d_model][d_ff], K-quant weights; gate and up of one type) on its tokens with the batched projections, and
 * writes y[rows][d_model] = sum over slots j in order of weight[j] * expert output. Every projection is
 * bit-identical to the reference's; SiLU uses expf (the reference's TensorPrimitives.Sigmoid is itself only
 * specified to a few ULP), so y matches to the projection tolerance. An index outside [0, n_experts), or a
 * repeated index in a token's slots, contributes nothing. n_experts <= OVFQ_MAX_EXPERTS. With top_k <= 2 and
 * few pairs per expert, the down projection adds each weighted expert output into y with a float atomic
 * (at most two adds onto zero per element, so the sum is the in-order one) when y is ordinary device memory
 * (hipMalloc, torch); a _dev caller's y in host-mapped memory gets the separate combine launch instead. */
OVFQ_API int ovfq_moe_ffn(ovfq_ctx* ctx, int n_experts, const ovfq_weight* const* gate,
                          const ovfq_weight* const* up, const ovfq_weight* const* down, const float* x, int rows,
                          int top_k, const int* expert_indices, const float* expert_weights, float* y);
OVFQ_API int ovfq_moe_ffn_dev(ovfq_ctx* ctx, int n_experts, const ovfq_weight* const* gate,
                              const ovfq_weight* const* up, const ovfq_weight* const* down, const float* x,
                              int rows, int top_k, const int* expert_indices, const float* expert_weights,
                              float* y);

/* MoeFeedForwardBlock.DecodeBatched (RT/MoeFeedForwardBlock.cs:140-241) from the router logits on: the routing
 * of ovfq_moe_select_topk (router_logits [rows][n_experts], top_k <= n_experts, normalize as there), written to
 * expert_indices / expert_weights [rows][top_k], then ovfq_moe_ffn with it. Outputs equal those two calls'; for up
 * to 64 (token, slot) entries the routing runs inside the grouping launch (one launch fewer). */
OVFQ_API int ovfq_moe_ffn_routed(ovfq_ctx* ctx, int n_experts, const ovfq_weight* const* gate,
                                 const ovfq_weight* const* up, const ovfq_weight* const* down, const float* x,
                                 int rows, const float* router_logits, int top_k, int normalize,
                                 int* expert_indices, float* expert_weights, float* y);
OVFQ_API int ovfq_moe_ffn_routed_dev(ovfq_ctx* ctx, int n_experts, const ovfq_weight* const* gate,
                                     const ovfq_weight* const* up, const ovfq_weight* const* down, const float* x,
                                     int rows, const float* router_logits, int top_k, int normalize,
                                     int* expert_indices, float* expert_weights, float* y);

/* ---------------------------------------------------------------------------------- weight quantisation */

/* GgmlQuant.QuantizeQ4_K (LD/GgmlQuant.cs:132-161): output-major f32 [out][in] (in % 256 == 0) -> Q4_K
 * bytes [out][in/256][144], bit-exact to the reference encoder. Device pointers. */
OVFQ_API int ovfq_quantize_weight_q4k_dev(ovfq_ctx* ctx, const float* w, int input_size, int output_size,
                                          uint8_t* dst);
/* Q6_K encoder (no reference counterpart: the reference reads Q6_K but cannot write it). Plain absmax per
 * 16-element sub-block under one fp16 super-scale; decodes with GgmlDequant.DecodeQ6_KBlock
 * (LD/GgmlDequant.cs:143-209). Device pointers. */
OVFQ_API int ovfq_quantize_weight_q6k_dev(ovfq_ctx* ctx, const float* w, int input_size, int output_size,
                                          uint8_t* dst);
/* Q8Weight.QuantizeRows (RT/Q8Weight.cs:115-175): device pointers. */
OVFQ_API int ovfq_quantize_weight_q8_0_dev(ovfq_ctx* ctx, const float* w, int input_size, int output_size,
                                           int8_t* quants, float* scales);

#ifdef __cplusplus
}
#endif
#endif /* OVFQ_H */
