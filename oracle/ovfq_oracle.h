/*
 * ovfq_oracle — CPU restatement of Overfit's GGUF quantized-linear arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker the GPU path is compared against; it is never
 * linked into, loaded by, or called from the product library (overfit_amd/libovfq.so). Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may use it.
 *
 * Every function follows the reference C# source named beside it (paths relative to the reference root;
 * RT/ = Sources/Main/LanguageModels/Runtime/, LD/ = Sources/Main/LanguageModels/Loading/).
 * Float semantics restated: IEEE binary32 per operation, no FMA contraction (build with
 * -ffp-contract=off), MathF.Round == rintf (round half to even), (Half)x == RNE binary16,
 * C# left-to-right evaluation order.
 *
 * Pinning (what checks each function beyond its own formula) is listed per function in the tests:
 * tests/test_oracle_*.py. The one function no reference test, fixture or closed form pins is
 * orc_encode_q6k_block: the reference has no Q6_K encoder, so this one is the build's own design and its
 * only pins are the decode round trip and byte-format invariants.
 */
#ifndef OVFQ_ORACLE_H
#define OVFQ_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_QK 256              /* elements per K-quant super-block */
#define ORC_Q4K_BYTES 144       /* RT/Q4KWeight.cs:29 */
#define ORC_Q6K_BYTES 210       /* LD/GgmlDequant.cs:27 */
#define ORC_Q8_BLOCK 32         /* RT/Q8DotKernel.cs:34 */
#define ORC_GROUP 16            /* RT/Q4KDotKernel.cs:47 */

/* fp16 <-> fp32 (System.Half semantics). */
float orc_half_to_float(uint16_t h);
uint16_t orc_float_to_half(float f);

/* a1: LD/GgmlDequant.cs:49-77 */
void orc_unpack_q4k_scales_mins(const uint8_t* packed12, uint8_t* scales8, uint8_t* mins8);
/* a18 helper: LD/GgmlQuant.cs:164-172 (inverse of a1) */
void orc_pack_q4k_scales_mins(const uint8_t* sc8, const uint8_t* m8, uint8_t* packed12);

/* a19: LD/GgmlDequant.cs:95-141 and :143-209 */
void orc_decode_q4k_block(const uint8_t* block144, float* dst256);
/* GgmlDequant.DecodeQ5_0Block / DecodeQ5_KBlock (LD/GgmlDequant.cs:222-320). */
void orc_decode_q5_0_block(const uint8_t* block22, float* dst32);
void orc_decode_q5k_block(const uint8_t* block176, float* dst256);
/* Q5_0 (type 6) / Q5_K (type 13) rows -> resident Q8_0 planes (decode to F32, then Q8Weight.QuantizeRows). */
int orc_q5_requantize_q8_0(int type, const uint8_t* src, int rows, int len, int8_t* quants, float* scales);
void orc_decode_q6k_block(const uint8_t* block210, float* dst256);
/* a15: RT/Q4KWeight.cs:121-138, RT/Q6KWeight.cs DecodeRow, RT/Q8Weight.cs:81-106 */
int orc_q4k_decode_row(const uint8_t* blocks, int input_size, int output_size, int row, float* dst);
int orc_q6k_decode_row(const uint8_t* blocks, int input_size, int output_size, int row, float* dst);
int orc_q8_decode_row(const int8_t* quants, const float* scales, int input_size, int output_size, int row,
                      float* dst);

/* a3: RT/Q4KDotKernel.cs:71-136 (scalar) == :148-209 (AVX2). n % 256 == 0. */
int orc_quantize_q8k(const float* src, int n, int8_t* quants, float* scales, int16_t* bsums);
/* a11: RT/Q8DotKernel.cs:42-91 (also RT/Q8Weight.cs:115-175 per row). n % 32 == 0. */
int orc_quantize_q8_0(const float* src, int n, int8_t* quants, float* scales);

/* a4: RT/Q4KDotKernel.cs:366-387 (MainDotScalar) */
int32_t orc_q4k_main_dot(const uint8_t* qs128, const int8_t* q8, const uint8_t* scales8);
/* a5: min term of RT/Q4KDotKernel.cs:244-253 */
int32_t orc_q4k_min_acc(const uint8_t* mins8, const int16_t* bsums16);
/* a5: RT/Q4KDotKernel.cs:216-256 */
float orc_q4k_dot(const uint8_t* block144, const int8_t* q8, float q8_scale, const int16_t* bsums16);
/* a9: RT/Q6KDotKernel.cs:186-216 (scalar UnsignedDotSuperBlock) */
int32_t orc_q6k_unsigned_dot(const uint8_t* block210, const int8_t* q8);
/* a9: bias term of RT/Q6KDotKernel.cs:108-113 */
int32_t orc_q6k_bsum_term(const uint8_t* block210, const int16_t* bsums16);
/* a9: RT/Q6KDotKernel.cs:77-116 */
float orc_q6k_dot(const uint8_t* block210, const int8_t* q8, float q8_scale, const int16_t* bsums16);
/* a12: RT/Q8DotKernel.cs:99-140 */
float orc_q8_dot(const int8_t* a_quants, const float* a_scales, const int8_t* b_quants, const float* b_scales,
                 int length);
int32_t orc_q8_block_int_dot(const int8_t* a32, const int8_t* b32);

/* a6: RT/Q4KDotKernel.cs:445-476 (ProjectPreQuantized); bias may be NULL (empty span). */
int orc_q4k_project_prequantized(const uint8_t* blocks, int input_size, int output_size, const float* bias,
                                 float* output, const int8_t* act_q, const float* act_s, const int16_t* act_b);
/* a6: RT/Q4KDotKernel.cs:414-435 (Project = quantize + prequantized); scratch sized per the reference. */
int orc_q4k_project(const float* input, const uint8_t* blocks, int input_size, int output_size,
                    const float* bias, float* output, int8_t* act_q, float* act_s, int16_t* act_b);
/* a7: RT/Q4KDotKernel.cs:563-645 */
int orc_q4k_project_gate_up(const float* input, const uint8_t* gate, const uint8_t* up, int input_size,
                            int out_dim, float* gate_out, float* up_out, int8_t* act_q, float* act_s,
                            int16_t* act_b);
/* a8: RT/Q4KDotKernel.cs:681-786 (ProjectBatched, rows innermost) */
int orc_q4k_project_batched(const float* input, int rows, const uint8_t* blocks, int input_size,
                            int output_size, const float* bias, float* output, int8_t* act_q, float* act_s,
                            int16_t* act_b);
/* a8: RT/Q4KDotKernel.cs:819-955 (weight-stationary, 64-row tiles) */
int orc_q4k_project_batched_ws(const float* input, int rows, const uint8_t* blocks, int input_size,
                               int output_size, const float* bias, float* output, int8_t* act_q, float* act_s,
                               int16_t* act_b);
/* Batched from already-quantized activations (the tail of a8 / a10 after the per-row quantize loop). */
int orc_q4k_project_batched_prequantized(int rows, const uint8_t* blocks, int input_size, int output_size,
                                         const float* bias, float* output, const int8_t* act_q,
                                         const float* act_s, const int16_t* act_b);

/* a10: RT/Q6KDotKernel.cs:245-305 (Project / ProjectPreQuantized) and :403-510 (ProjectBatched) */
int orc_q6k_project_prequantized(const uint8_t* blocks, int input_size, int output_size, const float* bias,
                                 float* output, const int8_t* act_q, const float* act_s, const int16_t* act_b);
int orc_q6k_project(const float* input, const uint8_t* blocks, int input_size, int output_size,
                    const float* bias, float* output, int8_t* act_q, float* act_s, int16_t* act_b);
int orc_q6k_project_batched(const float* input, int rows, const uint8_t* blocks, int input_size,
                            int output_size, const float* bias, float* output, int8_t* act_q, float* act_s,
                            int16_t* act_b);
int orc_q6k_project_batched_prequantized(int rows, const uint8_t* blocks, int input_size, int output_size,
                                         const float* bias, float* output, const int8_t* act_q,
                                         const float* act_s, const int16_t* act_b);

/* a12: RT/Q8DotKernel.cs:155-215 (Project) and :352-445 (ProjectBatched) */
int orc_q8_project(const float* input, const int8_t* w_quants, const float* w_scales, int input_size,
                   int output_size, const float* bias, float* output, int8_t* in_q, float* in_s);
int orc_q8_project_batched(const float* input, int rows, const int8_t* w_quants, const float* w_scales,
                           int input_size, int output_size, const float* bias, float* output, int8_t* in_q,
                           float* in_s);
int orc_q8_project_batched_prequantized(int rows, const int8_t* w_quants, const float* w_scales,
                                        int input_size, int output_size, const float* bias, float* output,
                                        const int8_t* in_q, const float* in_s);

/* The Llama attention output projection with per-head Q8_0 Wo (LD/GgufLlamaLoader.cs:977-995 requantises Wo per
 * head): y[n] = (bias or 0) then, heads ascending, y[n] += Q8DotKernel.Project(x[n][h*head_dim ..], Wo_h), where
 * Wo_h is [d_model][head_dim] (wq[h], ws[h]). RT/CachedMultiHeadAttention.cs:185-194 and :292-297 (decode),
 * :600-614 and :703-711 (prefill rows); each head's projection RT/CachedSingleHeadAttention.cs:323-337 /
 * RT/Q8DotKernel.cs:155-215. x is [rows][n_heads * head_dim], y [rows][d_model]. */
int orc_q8_project_heads(const float* x, int rows, int n_heads, int head_dim, int d_model,
                         const int8_t* const* wq, const float* const* ws, const float* bias, float* y);

/* a18: LD/GgmlQuant.cs:31-126 (EncodeQ4_KBlock) and :132-161 (QuantizeQ4_K) */
void orc_encode_q4k_block(const float* src256, uint8_t* block144);
int orc_quantize_q4k(const float* f32, int input_size, int output_size, uint8_t* dst);
/* The build's own Q6_K encoder (the reference has none): plain absmax per 16-element sub-block under
 * one fp16 super-scale, written from the block format of LD/GgmlDequant.cs:143-209. */
void orc_encode_q6k_block(const float* src256, uint8_t* block210);
int orc_quantize_q6k(const float* f32, int input_size, int output_size, uint8_t* dst);
/* a11 applied row by row: RT/Q8Weight.cs:115-175 (QuantizeRows). */
int orc_q8_quantize_rows(const float* row_major, int row_count, int row_length, int8_t* quants, float* scales);

/* LD/GgufReader.cs:198-266 (LoadTensorQ8_0Raw): 34-byte blocks -> int8 quants + f32 scales. */
int orc_q8_0_deinterleave(const uint8_t* gguf, long n_blocks, int8_t* quants, float* scales);

/* RT/MoeRouter.cs:40-128 (SelectTopK). Returns k, or a negative status. */
int orc_moe_select_topk(const float* logits, int n, int top_k, int* expert_indices, float* expert_weights,
                        int normalize);

/* RT/CachedFeedForwardBlock.cs:328-344 (DecodeSwiGluBatchedDispatched): batched SwiGLU FFN of `rows` rows,
 * gate/up [d_ff][d_model], down [d_model][d_ff]; types 12 (Q4_K) or 14 (Q6_K). SiLU via expf. */
int orc_swiglu_batched(const float* x, int rows, const uint8_t* gate, const uint8_t* up, const uint8_t* down,
                       int gate_type, int down_type, int d_model, int d_ff, float* y);
/* The same with the gate activation of ApplyGate (RT/CachedFeedForwardBlock.cs:474-485), activation taking
 * FeedForwardActivation's values (Runtime/FeedForwardActivation.cs:11-34): 3 = SwiGLU (SiLU), 4 = GeGLU (GELU with
 * the tanh approximation, ApplyGeLU :498-517, MathF.Tanh via tanhf). */
int orc_gated_ffn_batched(const float* x, int rows, const uint8_t* gate, const uint8_t* up, const uint8_t* down,
                          int gate_type, int down_type, int d_model, int d_ff, int activation, float* y);
/* RT/MoeFeedForwardBlock.cs:140-241 (DecodeBatched) after routing: idx/w [rows][top_k]. */
int orc_moe_ffn_batched(int n_experts, const uint8_t* const* gate, const uint8_t* const* up,
                        const uint8_t* const* down, int gate_type, int down_type, const float* x, int rows,
                        int d_model, int d_ff, int top_k, const int* idx, const float* w, float* y);

/* Status codes shared with the product's C ABI. */
#define ORC_OK 0
#define ORC_ERR_NULL (-1)
#define ORC_ERR_SIZE (-2)
#define ORC_ERR_RANGE (-3)

#ifdef __cplusplus
}
#endif
#endif
