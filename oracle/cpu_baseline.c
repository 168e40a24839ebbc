/*
 * cpu_baseline.c — the reported CPU baseline: a C restatement of Overfit's AVX2 decode and batched paths,
 * threaded like the reference's OverfitParallel (contiguous row bands, caller participates). Test and bench
 * infrastructure only (bench.py's cpu_baseline leg); never part of the product library.
 *
 *   MainDot AVX2             RT/Q4KDotKernel.cs:270-302
 *   Q6_K UnsignedDotSuperBlock AVX2  RT/Q6KDotKernel.cs:129-184
 *   Q8 Int8BlockDot AVX2     RT/Q8DotKernel.cs:469-478
 *   QuantizeActivationQ8KAvx2 RT/Q4KDotKernel.cs:148-209
 *   ForDecode row bands      Sources/Main/Runtime/OverfitParallel.cs:494-580 (perChunk = ceil(n/chunks), decode
 *                            cap min(cores, 10))
 *   For (batched)            Sources/Main/Runtime/OverfitParallel.cs:399-480 (chunkCount = min(workers, n),
 *                            perChunk = ceil(n/chunkCount), the caller runs the last chunk)
 *   ProjectBatchedWeightStationary  RT/Q4KDotKernel.cs:809-955 (each super-block decoded once per 64-row tile)
 *   Q6KDotKernel.ProjectBatched     RT/Q6KDotKernel.cs:403-510 (rows innermost)
 *   BatchedQuantProjection.Dispatch RT/BatchedQuantProjection.cs:26-87 (Q4_K -> weight-stationary)
 *   DecodeSwiGluBatchedDispatched   RT/CachedFeedForwardBlock.cs:328-348
 *   MoeFeedForwardBlock.DecodeBatched (after routing) RT/MoeFeedForwardBlock.cs:187-241
 *
 * Every kernel here is integer-identical to the scalar oracle (ovfq_oracle.c) and keeps the same float
 * tail and per-row summation order, so outputs are bit-identical to the oracle; tests check that.
 */
#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <sched.h>
#include <stdatomic.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "ovfq_oracle.h"

/* ---------------------------------------------------------------- persistent worker pool */

typedef void (*cpub_chunk_fn)(int start, int end, void* ctx);

#define CPUB_MAX_WORKERS 64

static struct {
    int workers; /* total participants including the caller */
    pthread_t threads[CPUB_MAX_WORKERS];
    atomic_int generation;
    atomic_int remaining;
    atomic_int shutdown;
    cpub_chunk_fn fn;
    void* ctx;
    int n;
    int per_chunk;
    int chunks;
    int caller_last;
    int started;
} g_pool;

/* OverfitParallel.DecodeMaxWorkers: single-token projections use at most min(cores, 10) chunks (PAR:184-195). */
static int g_decode_cap = 10;

static pthread_mutex_t g_pool_lock = PTHREAD_MUTEX_INITIALIZER;

static void run_chunk(int idx) {
    if (idx < 0 || idx >= g_pool.chunks) return;
    int start = idx * g_pool.per_chunk;
    int end = start + g_pool.per_chunk;
    if (end > g_pool.n) end = g_pool.n;
    if (start < end) g_pool.fn(start, end, g_pool.ctx);
}

static void* worker_main(void* arg) {
    int idx = (int)(intptr_t)arg;
    int seen = 0;
    for (;;) {
        int gen;
        int spins = 0;
        while ((gen = atomic_load_explicit(&g_pool.generation, memory_order_acquire)) == seen) {
            if (atomic_load(&g_pool.shutdown)) return NULL;
            if (++spins > 4096) {
                sched_yield();
                spins = 0;
            } else {
                _mm_pause();
            }
        }
        seen = gen;
        /* with the caller on the last chunk, pool thread i takes chunk i - 1 of the first chunks - 1 */
        if (g_pool.caller_last) run_chunk(idx - 1 < g_pool.chunks - 1 ? idx - 1 : -1);
        else run_chunk(idx);
        atomic_fetch_sub_explicit(&g_pool.remaining, 1, memory_order_acq_rel);
    }
}

/* Start (or resize) the pool to `workers` participants. Returns the participant count. */
int cpub_set_workers(int workers) {
    if (workers < 1) workers = 1;
    if (workers > CPUB_MAX_WORKERS) workers = CPUB_MAX_WORKERS;
    pthread_mutex_lock(&g_pool_lock);
    if (g_pool.started && g_pool.workers != workers) {
        atomic_store(&g_pool.shutdown, 1);
        for (int i = 1; i < g_pool.workers; i++) pthread_join(g_pool.threads[i], NULL);
        g_pool.started = 0;
    }
    if (!g_pool.started) {
        atomic_store(&g_pool.shutdown, 0);
        atomic_store(&g_pool.generation, 0);
        g_pool.workers = workers;
        for (int i = 1; i < workers; i++) {
            pthread_create(&g_pool.threads[i], NULL, worker_main, (void*)(intptr_t)i);
        }
        g_pool.started = 1;
    }
    pthread_mutex_unlock(&g_pool_lock);
    return workers;
}

/* Split [0, n) into min(cap, workers, n) contiguous chunks of ceil(n / chunks); the calling thread runs the first
 * chunk (ForDecode) or, with caller_last, the last one (For, PAR:472) and waits for the others. One chunk, or
 * n < 2, runs inline. */
static void parallel_for_capped(int n, cpub_chunk_fn fn, void* ctx, int cap, int caller_last) {
    if (!g_pool.started) cpub_set_workers(1);
    int w = g_pool.workers;
    int chunks = cap < w ? cap : w;
    if (chunks > n) chunks = n;
    if (chunks <= 1 || n < 2) {
        fn(0, n, ctx);
        return;
    }
    g_pool.fn = fn;
    g_pool.ctx = ctx;
    g_pool.n = n;
    g_pool.chunks = chunks;
    g_pool.per_chunk = (n + chunks - 1) / chunks;
    g_pool.caller_last = caller_last;
    /* pool threads 1 .. w-1 take chunks 1 .. w-1 (caller_last: chunks 0 .. w-2); the caller the remaining one */
    atomic_store_explicit(&g_pool.remaining, w - 1, memory_order_release);
    atomic_fetch_add_explicit(&g_pool.generation, 1, memory_order_acq_rel);
    run_chunk(caller_last ? chunks - 1 : 0);
    while (atomic_load_explicit(&g_pool.remaining, memory_order_acquire) != 0) _mm_pause();
}

/* OverfitParallel.ForDecode (single-token projections). */
static void parallel_for(int n, cpub_chunk_fn fn, void* ctx) { parallel_for_capped(n, fn, ctx, g_decode_cap, 0); }

/* OverfitParallel.For over every worker (batched projections). */
static void parallel_for_all(int n, cpub_chunk_fn fn, void* ctx) { parallel_for_capped(n, fn, ctx, 1 << 30, 1); }

/* Chunk cap of the single-token (ForDecode) projections; the reference's is min(cores, 10). */
int cpub_set_decode_cap(int cap) {
    g_decode_cap = cap < 1 ? 1 : cap;
    return g_decode_cap;
}

/* ---------------------------------------------------------------- AVX2 kernels */

static inline int hsum_epi32(__m256i v) {
    __m128i s = _mm_add_epi32(_mm256_castsi256_si128(v), _mm256_extracti128_si256(v, 1));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0x4e));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0xb1));
    return _mm_cvtsi128_si32(s);
}

static inline __m256i pairs32(__m256i u8, __m256i s8) {
    return _mm256_madd_epi16(_mm256_maddubs_epi16(u8, s8), _mm256_set1_epi16(1));
}

static int32_t q4k_main_dot_avx2(const uint8_t* qs, const int8_t* q8, const uint8_t* scales) {
    const __m256i mask = _mm256_set1_epi8(0x0f);
    __m256i acc = _mm256_setzero_si256();
    for (int p = 0; p < 4; p++) {
        __m256i packed = _mm256_loadu_si256((const __m256i*)(qs + 32 * p));
        __m256i lo = _mm256_and_si256(packed, mask);
        __m256i hi = _mm256_and_si256(_mm256_srli_epi16(packed, 4), mask);
        __m256i qe = _mm256_loadu_si256((const __m256i*)(q8 + 64 * p));
        __m256i qo = _mm256_loadu_si256((const __m256i*)(q8 + 64 * p + 32));
        acc = _mm256_add_epi32(acc, _mm256_mullo_epi32(pairs32(lo, qe), _mm256_set1_epi32(scales[2 * p])));
        acc = _mm256_add_epi32(acc, _mm256_mullo_epi32(pairs32(hi, qo), _mm256_set1_epi32(scales[2 * p + 1])));
    }
    return hsum_epi32(acc);
}

static inline uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

static inline float q4k_dot_avx2(const uint8_t* b, const int8_t* q8, float q8s, const int16_t* bsums) {
    float d = orc_half_to_float(rd16(b));
    float dmin = orc_half_to_float(rd16(b + 2));
    uint8_t sc[8], m[8];
    orc_unpack_q4k_scales_mins(b + 4, sc, m);
    int32_t main_acc = q4k_main_dot_avx2(b + 16, q8, sc);
    int32_t min_acc = 0;
    for (int s = 0; s < 8; s++) min_acc += m[s] * (bsums[2 * s] + bsums[2 * s + 1]);
    return q8s * (d * (float)main_acc - dmin * (float)min_acc);
}

static inline int group_dot(__m256i q, __m256i q8, int sa, int sb) {
    __m256i p = pairs32(q, q8);
    __m128i lo = _mm256_castsi256_si128(p), hi = _mm256_extracti128_si256(p, 1);
    lo = _mm_add_epi32(lo, _mm_shuffle_epi32(lo, 0x4e));
    lo = _mm_add_epi32(lo, _mm_shuffle_epi32(lo, 0xb1));
    hi = _mm_add_epi32(hi, _mm_shuffle_epi32(hi, 0x4e));
    hi = _mm_add_epi32(hi, _mm_shuffle_epi32(hi, 0xb1));
    return sa * _mm_cvtsi128_si32(lo) + sb * _mm_cvtsi128_si32(hi);
}

static int32_t q6k_unsigned_dot_avx2(const uint8_t* b, const int8_t* q8) {
    const uint8_t* ql = b;
    const uint8_t* qh = b + 128;
    const int8_t* sc = (const int8_t*)(b + 192);
    const __m256i m4 = _mm256_set1_epi8(0x0f), m2 = _mm256_set1_epi8(0x03);
    int32_t term = 0;
    for (int h = 0; h < 2; h++) {
        __m256i a = _mm256_loadu_si256((const __m256i*)(ql + 64 * h));
        __m256i bb = _mm256_loadu_si256((const __m256i*)(ql + 64 * h + 32));
        __m256i hv = _mm256_loadu_si256((const __m256i*)(qh + 32 * h));
        __m256i alo = _mm256_and_si256(a, m4), ahi = _mm256_and_si256(_mm256_srli_epi16(a, 4), m4);
        __m256i blo = _mm256_and_si256(bb, m4), bhi = _mm256_and_si256(_mm256_srli_epi16(bb, 4), m4);
        __m256i h0 = _mm256_slli_epi16(_mm256_and_si256(hv, m2), 4);
        __m256i h1 = _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(hv, 2), m2), 4);
        __m256i h2 = _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(hv, 4), m2), 4);
        __m256i h3 = _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(hv, 6), m2), 4);
        const int8_t* q = q8 + 128 * h;
        const int8_t* s = sc + 8 * h;
        term += group_dot(_mm256_or_si256(alo, h0), _mm256_loadu_si256((const __m256i*)(q)), s[0], s[1]) +
                group_dot(_mm256_or_si256(blo, h1), _mm256_loadu_si256((const __m256i*)(q + 32)), s[2], s[3]) +
                group_dot(_mm256_or_si256(ahi, h2), _mm256_loadu_si256((const __m256i*)(q + 64)), s[4], s[5]) +
                group_dot(_mm256_or_si256(bhi, h3), _mm256_loadu_si256((const __m256i*)(q + 96)), s[6], s[7]);
    }
    return term;
}

static inline float q6k_dot_avx2(const uint8_t* b, const int8_t* q8, float q8s, const int16_t* bsums) {
    float d = orc_half_to_float(rd16(b + 208));
    int32_t u = q6k_unsigned_dot_avx2(b, q8);
    int32_t bt = 0;
    for (int s = 0; s < 16; s++) bt += (int8_t)b[192 + s] * bsums[s];
    return d * q8s * (float)(u - 32 * bt);
}

static inline int32_t q8_block_dot_avx2(const int8_t* a, const int8_t* b) {
    __m256i va = _mm256_loadu_si256((const __m256i*)a), vb = _mm256_loadu_si256((const __m256i*)b);
    __m256i p16 = _mm256_maddubs_epi16(_mm256_abs_epi8(va), _mm256_sign_epi8(vb, va));
    return hsum_epi32(_mm256_madd_epi16(p16, _mm256_set1_epi16(1)));
}

/* QuantizeActivationQ8KAvx2 (RT/Q4KDotKernel.cs:148-209). */
int cpub_quantize_q8k(const float* src, int n, int8_t* quants, float* scales, int16_t* bsums) {
    if (n % 256) return ORC_ERR_SIZE;
    const __m256 absmask = _mm256_castsi256_ps(_mm256_set1_epi32(0x7fffffff));
    const __m256 lo = _mm256_set1_ps(-127.0f), hi = _mm256_set1_ps(127.0f);
    for (int b = 0; b < n / 256; b++) {
        const float* x = src + (size_t)b * 256;
        __m256 mv = _mm256_setzero_ps();
        for (int i = 0; i < 256; i += 8) mv = _mm256_max_ps(mv, _mm256_and_ps(_mm256_loadu_ps(x + i), absmask));
        __m128 m4 = _mm_max_ps(_mm256_castps256_ps128(mv), _mm256_extractf128_ps(mv, 1));
        float e[4];
        _mm_storeu_ps(e, m4);
        float a01 = e[0] > e[1] ? e[0] : e[1];
        float a23 = e[2] > e[3] ? e[2] : e[3];
        float absmax = a01 > a23 ? a01 : a23;
        float scale = absmax / 127.0f;
        scales[b] = scale;
        float inverse = scale > 0.0f ? 1.0f / scale : 0.0f;
        __m256 inv = _mm256_set1_ps(inverse);
        for (int g = 0; g < 16; g++) {
            __m256 x0 = _mm256_loadu_ps(x + g * 16), x1 = _mm256_loadu_ps(x + g * 16 + 8);
            __m256 r0 = _mm256_min_ps(hi, _mm256_max_ps(lo, _mm256_round_ps(_mm256_mul_ps(x0, inv),
                                                                              _MM_FROUND_TO_NEAREST_INT |
                                                                                  _MM_FROUND_NO_EXC)));
            __m256 r1 = _mm256_min_ps(hi, _mm256_max_ps(lo, _mm256_round_ps(_mm256_mul_ps(x1, inv),
                                                                              _MM_FROUND_TO_NEAREST_INT |
                                                                                  _MM_FROUND_NO_EXC)));
            __m256i i0 = _mm256_cvttps_epi32(r0), i1 = _mm256_cvttps_epi32(r1);
            bsums[(size_t)b * 16 + g] = (int16_t)hsum_epi32(_mm256_add_epi32(i0, i1));
            int32_t t[16];
            _mm256_storeu_si256((__m256i*)t, i0);
            _mm256_storeu_si256((__m256i*)(t + 8), i1);
            for (int k = 0; k < 16; k++) quants[(size_t)b * 256 + g * 16 + k] = (int8_t)t[k];
        }
    }
    return ORC_OK;
}

int cpub_quantize_q8_0(const float* src, int n, int8_t* quants, float* scales) {
    /* The reference's Q8DotKernel.Quantize is scalar (RT/Q8DotKernel.cs:42-91). */
    return orc_quantize_q8_0(src, n, quants, scales);
}

/* ---------------------------------------------------------------- threaded projections */

typedef struct {
    const uint8_t* blocks;
    const uint8_t* blocks2; /* gate/up: the up matrix */
    const int8_t* q;
    const float* s;
    const int16_t* b;
    const float* bias;
    float* out;
    float* out2;
    int spr;
    int out_dim;
} proj_ctx;

static void q4k_chunk(int start, int end, void* vctx) {
    proj_ctx* c = (proj_ctx*)vctx;
    for (int o = start; o < end; o++) {
        const uint8_t* row = c->blocks + (size_t)o * c->spr * ORC_Q4K_BYTES;
        float sum = 0.0f;
        for (int sb = 0; sb < c->spr; sb++) {
            sum += q4k_dot_avx2(row + (size_t)sb * ORC_Q4K_BYTES, c->q + sb * 256, c->s[sb], c->b + sb * 16);
        }
        c->out[o] = c->bias == NULL ? sum : c->bias[o] + sum;
    }
}

static void q4k_gate_up_chunk(int start, int end, void* vctx) {
    proj_ctx* c = (proj_ctx*)vctx;
    for (int g = start; g < end; g++) {
        int is_up = g >= c->out_dim;
        int row = is_up ? g - c->out_dim : g;
        const uint8_t* rp = (is_up ? c->blocks2 : c->blocks) + (size_t)row * c->spr * ORC_Q4K_BYTES;
        float sum = 0.0f;
        for (int sb = 0; sb < c->spr; sb++) {
            sum += q4k_dot_avx2(rp + (size_t)sb * ORC_Q4K_BYTES, c->q + sb * 256, c->s[sb], c->b + sb * 16);
        }
        if (is_up) c->out2[row] = sum;
        else c->out[row] = sum;
    }
}

static void q6k_chunk(int start, int end, void* vctx) {
    proj_ctx* c = (proj_ctx*)vctx;
    for (int o = start; o < end; o++) {
        const uint8_t* row = c->blocks + (size_t)o * c->spr * ORC_Q6K_BYTES;
        float sum = 0.0f;
        for (int sb = 0; sb < c->spr; sb++) {
            sum += q6k_dot_avx2(row + (size_t)sb * ORC_Q6K_BYTES, c->q + sb * 256, c->s[sb], c->b + sb * 16);
        }
        c->out[o] = c->bias == NULL ? sum : c->bias[o] + sum;
    }
}

typedef struct {
    const int8_t* wq;
    const float* ws;
    const int8_t* aq;
    const float* as;
    const float* bias;
    float* out;
    int in;
} q8_ctx;

static void q8_chunk(int start, int end, void* vctx) {
    q8_ctx* c = (q8_ctx*)vctx;
    int bpr = c->in / 32;
    for (int o = start; o < end; o++) {
        const int8_t* w = c->wq + (size_t)o * c->in;
        const float* ws = c->ws + (size_t)o * bpr;
        float r = 0.0f;
        for (int blk = 0; blk < bpr; blk++) {
            r += ws[blk] * c->as[blk] * (float)q8_block_dot_avx2(w + blk * 32, c->aq + blk * 32);
        }
        c->out[o] = c->bias == NULL ? r : c->bias[o] + r;
    }
}

/* Q4KDotKernel.ProjectParallel (RT/Q4KDotKernel.cs:485-552): quantize once, then row bands. */
int cpub_q4k_project_parallel(const float* input, const uint8_t* blocks, int in, int out, const float* bias,
                              float* output, int8_t* q, float* s, int16_t* b) {
    int rc = cpub_quantize_q8k(input, in, q, s, b);
    if (rc) return rc;
    proj_ctx c = {blocks, NULL, q, s, b, bias, output, NULL, in / 256, out};
    parallel_for(out, q4k_chunk, &c);
    return ORC_OK;
}

int cpub_q4k_project_prequantized_parallel(const uint8_t* blocks, int in, int out, const float* bias,
                                           float* output, const int8_t* q, const float* s, const int16_t* b) {
    proj_ctx c = {blocks, NULL, q, s, b, bias, output, NULL, in / 256, out};
    parallel_for(out, q4k_chunk, &c);
    return ORC_OK;
}

/* Q4KDotKernel.ProjectGateUpParallel (RT/Q4KDotKernel.cs:563-645). */
int cpub_q4k_project_gate_up(const float* input, const uint8_t* gate, const uint8_t* up, int in, int out_dim,
                             float* gate_out, float* up_out, int8_t* q, float* s, int16_t* b) {
    int rc = cpub_quantize_q8k(input, in, q, s, b);
    if (rc) return rc;
    proj_ctx c = {gate, up, q, s, b, NULL, gate_out, up_out, in / 256, out_dim};
    parallel_for(2 * out_dim, q4k_gate_up_chunk, &c);
    return ORC_OK;
}

/* Q6KDotKernel.ProjectParallel (RT/Q6KDotKernel.cs:314-381). */
int cpub_q6k_project_parallel(const float* input, const uint8_t* blocks, int in, int out, const float* bias,
                              float* output, int8_t* q, float* s, int16_t* b) {
    int rc = cpub_quantize_q8k(input, in, q, s, b);
    if (rc) return rc;
    proj_ctx c = {blocks, NULL, q, s, b, bias, output, NULL, in / 256, out};
    parallel_for(out, q6k_chunk, &c);
    return ORC_OK;
}

/* Q8DotKernel.ProjectParallel (RT/Q8DotKernel.cs:252-330). */
int cpub_q8_project_parallel(const float* input, const int8_t* wq, const float* ws, int in, int out,
                             const float* bias, float* output, int8_t* in_q, float* in_s) {
    int rc = cpub_quantize_q8_0(input, in, in_q, in_s);
    if (rc) return rc;
    q8_ctx c = {wq, ws, in_q, in_s, bias, output, in};
    parallel_for(out, q8_chunk, &c);
    return ORC_OK;
}

/* ---------------------------------------------------------------- batched projections (prefill, experts) */

#define CPUB_WS_TILE 64 /* Q4KDotKernel.WeightStationaryTile (RT/Q4KDotKernel.cs:809) */

typedef struct {
    const uint8_t* blocks;
    const int8_t* q;
    const float* s;
    const int16_t* b;
    const float* bias;
    float* out;
    int spr;
    int in;
    int out_dim;
    int rows;
} batched_ctx;

/* WeightStationaryChunk (RT/Q4KDotKernel.cs:894-955): per output, per 64-row tile, each super-block's d, dmin and
 * scales/mins decoded once and contracted against every row of the tile; acc[t] += q8s * (d*main - dmin*min) in
 * ascending super-block order, then output = biasO + acc[t]. */
static void q4k_ws_chunk(int start, int end, void* vctx) {
    batched_ctx* c = (batched_ctx*)vctx;
    float acc[CPUB_WS_TILE];
    for (int o = start; o < end; o++) {
        const uint8_t* row = c->blocks + (size_t)o * c->spr * ORC_Q4K_BYTES;
        const float bias_o = c->bias == NULL ? 0.0f : c->bias[o];
        for (int t0 = 0; t0 < c->rows; t0 += CPUB_WS_TILE) {
            const int tile = c->rows - t0 < CPUB_WS_TILE ? c->rows - t0 : CPUB_WS_TILE;
            for (int t = 0; t < tile; t++) acc[t] = 0.0f;
            for (int sb = 0; sb < c->spr; sb++) {
                const uint8_t* blk = row + (size_t)sb * ORC_Q4K_BYTES;
                const float d = orc_half_to_float(rd16(blk));
                const float dmin = orc_half_to_float(rd16(blk + 2));
                uint8_t sc[8], m[8];
                orc_unpack_q4k_scales_mins(blk + 4, sc, m);
                for (int t = 0; t < tile; t++) {
                    const size_t n = (size_t)(t0 + t);
                    const int32_t main_acc = q4k_main_dot_avx2(blk + 16, c->q + n * c->in + sb * 256, sc);
                    const int16_t* bs = c->b + n * c->spr * 16 + sb * 16;
                    int32_t min_acc = 0;
                    for (int j = 0; j < 8; j++) min_acc += m[j] * (bs[2 * j] + bs[2 * j + 1]);
                    acc[t] += c->s[n * c->spr + sb] * (d * (float)main_acc - dmin * (float)min_acc);
                }
            }
            for (int t = 0; t < tile; t++) c->out[(size_t)(t0 + t) * c->out_dim + o] = bias_o + acc[t];
        }
    }
}

/* Q6KDotKernel.ProjectBatchedChunk (RT/Q6KDotKernel.cs:477-510): per output, rows innermost, each row's
 * sum += Dot(...) in ascending super-block order; output = biasO + sum. */
static void q6k_batched_chunk(int start, int end, void* vctx) {
    batched_ctx* c = (batched_ctx*)vctx;
    for (int o = start; o < end; o++) {
        const uint8_t* row = c->blocks + (size_t)o * c->spr * ORC_Q6K_BYTES;
        const float bias_o = c->bias == NULL ? 0.0f : c->bias[o];
        for (int n = 0; n < c->rows; n++) {
            const size_t nn = (size_t)n;
            float sum = 0.0f;
            for (int sb = 0; sb < c->spr; sb++)
                sum += q6k_dot_avx2(row + (size_t)sb * ORC_Q6K_BYTES, c->q + nn * c->in + sb * 256,
                                    c->s[nn * c->spr + sb], c->b + nn * c->spr * 16 + sb * 16);
            c->out[nn * c->out_dim + o] = bias_o + sum;
        }
    }
}

/* Per-row QuantizeActivationQ8K on the calling thread (RT/Q4KDotKernel.cs:718-725, :856-863), then For over the
 * outputs. */
static int batched_project(int type, const float* x, int rows, const uint8_t* blocks, int in, int out,
                           const float* bias, float* y, int8_t* q, float* s, int16_t* b) {
    if (rows <= 0 || in <= 0 || out <= 0) return ORC_ERR_RANGE;
    if (in % 256) return ORC_ERR_SIZE;
    const int spr = in / 256;
    for (int n = 0; n < rows; n++) {
        int rc = cpub_quantize_q8k(x + (size_t)n * in, in, q + (size_t)n * in, s + (size_t)n * spr,
                                   b + (size_t)n * spr * 16);
        if (rc) return rc;
    }
    batched_ctx c = {blocks, q, s, b, bias, y, spr, in, out, rows};
    if (type == 12) parallel_for_all(out, q4k_ws_chunk, &c);
    else if (type == 14) parallel_for_all(out, q6k_batched_chunk, &c);
    else return ORC_ERR_RANGE;
    return ORC_OK;
}

/* Q4KDotKernel.ProjectBatchedWeightStationary (RT/Q4KDotKernel.cs:819-893). */
int cpub_q4k_project_batched_ws(const float* x, int rows, const uint8_t* blocks, int in, int out, const float* bias,
                                float* y, int8_t* q, float* s, int16_t* b) {
    return batched_project(12, x, rows, blocks, in, out, bias, y, q, s, b);
}

/* Q6KDotKernel.ProjectBatched (RT/Q6KDotKernel.cs:403-475). */
int cpub_q6k_project_batched(const float* x, int rows, const uint8_t* blocks, int in, int out, const float* bias,
                             float* y, int8_t* q, float* s, int16_t* b) {
    return batched_project(14, x, rows, blocks, in, out, bias, y, q, s, b);
}

/* DecodeSwiGluBatchedDispatched (RT/CachedFeedForwardBlock.cs:328-348) with BatchedQuantProjection.Dispatch for each
 * projection (Q4_K weight-stationary, Q6_K batched): gate, SiLU (the oracle's 1 / (1 + expf(-g)) form), up,
 * gate * up, down. Scratch: g, u [rows][d_ff]; q [rows][max(d_model, d_ff)], s, b to match. */
static int swiglu_batched(const float* x, int rows, const uint8_t* gate, const uint8_t* up, const uint8_t* down,
                          int gate_type, int down_type, int d_model, int d_ff, float* y, float* g, float* u, int8_t* q,
                          float* s, int16_t* b) {
    int rc = batched_project(gate_type, x, rows, gate, d_model, d_ff, NULL, g, q, s, b);
    if (rc) return rc;
    for (size_t i = 0; i < (size_t)rows * d_ff; i++) {
        const float sig = 1.0f / (1.0f + expf(-g[i]));
        g[i] = g[i] * sig;
    }
    if ((rc = batched_project(gate_type, x, rows, up, d_model, d_ff, NULL, u, q, s, b))) return rc;
    for (size_t i = 0; i < (size_t)rows * d_ff; i++) u[i] = g[i] * u[i];
    return batched_project(down_type, u, rows, down, d_ff, d_model, NULL, y, q, s, b);
}

/* MoeFeedForwardBlock.DecodeBatched after routing (RT/MoeFeedForwardBlock.cs:187-241): for each expert in order,
 * its tokens (first matching slot, tokens ascending) gathered, the batched SwiGLU, outputs stashed at (token, slot);
 * then each token's slots combined in slot order. Same grouping and combine as the oracle's orc_moe_ffn_batched. */
int cpub_moe_ffn_batched(int n_experts, const uint8_t* const* gate, const uint8_t* const* up,
                         const uint8_t* const* down, int gate_type, int down_type, const float* x, int rows,
                         int d_model, int d_ff, int top_k, const int* idx, const float* w, float* y) {
    if (!gate || !up || !down || !x || !idx || !w || !y) return ORC_ERR_NULL;
    if (n_experts <= 0 || rows <= 0 || top_k <= 0) return ORC_ERR_RANGE;
    if (d_model % 256 || d_ff % 256) return ORC_ERR_SIZE;
    const size_t P = (size_t)rows * top_k;
    const int kmax = d_model > d_ff ? d_model : d_ff;
    int* row_buf = (int*)malloc(sizeof(int) * (size_t)rows);
    int* slot_buf = (int*)malloc(sizeof(int) * (size_t)rows);
    int* have = (int*)calloc(P, sizeof(int));
    float* gathered = (float*)malloc(sizeof(float) * (size_t)rows * d_model);
    float* expert_out = (float*)malloc(sizeof(float) * (size_t)rows * d_model);
    float* slot_out = (float*)malloc(sizeof(float) * P * d_model);
    float* g = (float*)malloc(sizeof(float) * (size_t)rows * d_ff);
    float* u = (float*)malloc(sizeof(float) * (size_t)rows * d_ff);
    int8_t* q = (int8_t*)malloc((size_t)rows * kmax);
    float* s = (float*)malloc(sizeof(float) * (size_t)rows * (kmax / 256));
    int16_t* b = (int16_t*)malloc(sizeof(int16_t) * (size_t)rows * (kmax / 16));
    int rc = (row_buf && slot_buf && have && gathered && expert_out && slot_out && g && u && q && s && b) ? ORC_OK
                                                                                                      : ORC_ERR_SIZE;
    for (int e = 0; e < n_experts && !rc; e++) {
        int count = 0;
        for (int n = 0; n < rows; n++)
            for (int j = 0; j < top_k; j++)
                if (idx[n * top_k + j] == e) {
                    row_buf[count] = n;
                    slot_buf[count] = j;
                    count++;
                    break;
                }
        if (count == 0) continue;
        for (int c = 0; c < count; c++)
            memcpy(gathered + (size_t)c * d_model, x + (size_t)row_buf[c] * d_model, sizeof(float) * d_model);
        rc = swiglu_batched(gathered, count, gate[e], up[e], down[e], gate_type, down_type, d_model, d_ff,
                            expert_out, g, u, q, s, b);
        for (int c = 0; c < count && !rc; c++) {
            const size_t slot = (size_t)row_buf[c] * top_k + slot_buf[c];
            memcpy(slot_out + slot * d_model, expert_out + (size_t)c * d_model, sizeof(float) * d_model);
            have[slot] = 1;
        }
    }
    for (int n = 0; n < rows && !rc; n++) {
        float* dst = y + (size_t)n * d_model;
        for (int d = 0; d < d_model; d++) dst[d] = 0.0f;
        for (int j = 0; j < top_k; j++) {
            const size_t slot = (size_t)n * top_k + j;
            if (!have[slot]) continue;
            const float wj = w[slot];
            const float* src = slot_out + slot * d_model;
            for (int d = 0; d < d_model; d++) dst[d] += wj * src[d];
        }
    }
    free(row_buf);
    free(slot_buf);
    free(have);
    free(gathered);
    free(expert_out);
    free(slot_out);
    free(g);
    free(u);
    free(q);
    free(s);
    free(b);
    return rc;
}

/* Compiler and flags this file was built with (for the baseline's report). */
const char* cpub_build_info(void) {
#ifdef CPUB_FLAGS
    return "gcc " __VERSION__ "; " CPUB_FLAGS;
#else
    return "gcc " __VERSION__;
#endif
}

int cpub_has_avx2(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
}
