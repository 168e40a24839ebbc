// api.cpp — the C ABI of libovfq (declared in include/ovfq.h).
//
// Host responsibilities: argument validation before any device work (the reference throws before work,
// RT/Q4KDotKernel.cs:77-97), weight residency in HBM, activation quantisation scratch, staging of host
// buffers for the synchronous entry points, and dispatch to the kernels in quant.hip / project.hip.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/ovfq.h"
#include "ovfq_launch.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int ok() {
    g_last_error.clear();
    return OVFQ_OK;
}

#define HIP_TRY(expr)                                                                                  \
    do {                                                                                               \
        hipError_t _e = (expr);                                                                        \
        if (_e != hipSuccess) return fail(OVFQ_ERR_HIP, "%s failed: %s", #expr, hipGetErrorString(_e)); \
    } while (0)

// A growable device buffer owned by a context.
struct DevBuf {
    void* p = nullptr;
    size_t cap = 0;
};

}  // namespace

struct ovfq_ctx {
    int device = 0;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    int batched_kernel = OVFQ_BATCHED_AUTO;  // ovfq_ctx_set_batched_kernel
    std::mutex mu;
    // Activation quantisation scratch (Q8_K / Q8_0) and host-call staging.
    DevBuf act_q, act_s, act_b, x_stage, y_stage, y2_stage, bias_stage;
    // Routed-MoE scratch (plan, gate/up/intermediate/expert outputs, host staging), carved from one buffer.
    DevBuf moe;
    // Page-locked host arenas of the host-pointer entry points (hipHostMalloc): inputs go up, outputs come down.
    DevBuf h_up, h_down;
    // Scratch buffers replaced by larger ones. A HIP graph captured from _dev calls keeps the addresses it
    // was recorded with, so a superseded buffer stays allocated until the context is destroyed.
    std::vector<void*> retired;
    size_t retired_bytes = 0;
    // Live weights created on this context (ovfq_ctx_destroy refuses while any remain).
    int live_weights = 0;
};

// One device allocation holding every expert sliced from a 3-D GGUF expert tensor; the last expert weight
// destroyed frees it. Reference counts change under the owning context's mutex.
struct SharedPlane {
    void* p = nullptr;
    int refs = 0;
};

struct ovfq_weight {
    ovfq_ctx* ctx = nullptr;
    int type = 0;
    int in = 0;
    int out = 0;
    void* blocks = nullptr;  // Q4_K/Q6_K blocks or Q8_0 quant plane
    float* scales = nullptr; // Q8_0 scale plane
    size_t nbytes = 0;       // resident bytes (blocks + scales)
    void* mfma = nullptr;    // MFMA-ready copy (ovfq_weight_prepare_mfma), or NULL
    SharedPlane* shared = nullptr; // set for expert slices: blocks/scales point into shared->p
};

namespace {

// Grows `b` to at least `bytes`. The old buffer is not freed: queued work and any HIP graph captured from
// earlier calls may still address it, so it is kept in `retired` until ovfq_ctx_destroy. Capacities at least
// double on growth, which bounds the retired bytes by the live buffer's size.
int ensure(ovfq_ctx* c, DevBuf& b, size_t bytes) {
    if (b.cap >= bytes) return OVFQ_OK;
    size_t cap = bytes < 4096 ? 4096 : bytes;
    if (cap < 2 * b.cap) cap = 2 * b.cap;
    cap = (cap + 255) & ~size_t(255);
    void* p = nullptr;
    HIP_TRY(hipMalloc(&p, cap));
    if (b.p) {
        c->retired.push_back(b.p);
        c->retired_bytes += b.cap;
    }
    b.p = p;
    b.cap = cap;
    return OVFQ_OK;
}

// Replaces the page-locked arena `b` by one of at least `bytes` (doubling). The caller has made sure that no queued
// copy still reads or writes the old arena.
int host_grow(DevBuf& b, size_t bytes) {
    size_t cap = bytes < 65536 ? 65536 : bytes;
    if (cap < 2 * b.cap) cap = 2 * b.cap;
    cap = (cap + 4095) & ~size_t(4095);
    void* p = nullptr;
    HIP_TRY(hipHostMalloc(&p, cap, hipHostMallocDefault));
    if (b.p) (void)hipHostFree(b.p);
    b.p = p;
    b.cap = cap;
    return OVFQ_OK;
}

// The staging of one host-pointer call (made under the context lock). The caller's buffers are ordinary pageable
// memory; copying them through the context's page-locked arenas lets the DMA engines move them directly, where the
// runtime's pageable path stages every copy through buffers of its own and blocks the host on each. up() copies an
// input into the up arena and enqueues its upload; down() enqueues an output's download into the down arena;
// finish() waits for the stream and copies the outputs to the caller. An arena too small for a call is grown after a
// wait (and then fits the next call of that size).
struct HostIO {
    static constexpr int kMaxOuts = 8;
    struct Out {
        void* dst;
        size_t off, n;
    };
    ovfq_ctx* c;
    size_t up_off = 0, down_off = 0;
    Out outs[kMaxOuts];
    int n_outs = 0;

    explicit HostIO(ovfq_ctx* ctx) : c(ctx) {}

    static size_t round(size_t n) { return (n + 255) & ~size_t(255); }

    int up(void* dev_dst, const void* src, size_t n) {
        if (up_off + n > c->h_up.cap) {
            HIP_TRY(hipStreamSynchronize(c->stream));  // uploads already queued read the old arena
            int rc = host_grow(c->h_up, up_off + n);
            if (rc) return rc;
            up_off = 0;
        }
        char* p = static_cast<char*>(c->h_up.p) + up_off;
        memcpy(p, src, n);
        HIP_TRY(hipMemcpyAsync(dev_dst, p, n, hipMemcpyHostToDevice, c->stream));
        up_off += round(n);
        return OVFQ_OK;
    }

    int down(void* dst, const void* dev_src, size_t n) {
        if (down_off + n > c->h_down.cap || n_outs == kMaxOuts) {
            const size_t need = down_off + n;
            int rc = flush();
            if (rc) return rc;
            if (n > c->h_down.cap && (rc = host_grow(c->h_down, need))) return rc;
        }
        HIP_TRY(hipMemcpyAsync(static_cast<char*>(c->h_down.p) + down_off, dev_src, n, hipMemcpyDeviceToHost,
                               c->stream));
        outs[n_outs++] = Out{dst, down_off, n};
        down_off += round(n);
        return OVFQ_OK;
    }

    // Waits for the stream and hands the downloaded outputs to the caller.
    int flush() {
        HIP_TRY(hipStreamSynchronize(c->stream));
        for (int i = 0; i < n_outs; i++) memcpy(outs[i].dst, static_cast<char*>(c->h_down.p) + outs[i].off, outs[i].n);
        n_outs = 0;
        down_off = 0;
        return OVFQ_OK;
    }

    int finish() { return flush(); }
};

static_assert(ovfq::kNoAllocMaxElems == OVFQ_NOALLOC_MAX_ELEMS, "header and library disagree on the fixed scratch");
static_assert(ovfq::kHeadsMax == OVFQ_MAX_HEADS, "header and library disagree on the head count");

bool valid_type(int t) { return t == OVFQ_TYPE_Q4_K || t == OVFQ_TYPE_Q6_K || t == OVFQ_TYPE_Q8_0; }

size_t block_bytes_per_row(int type, int in) {
    if (type == OVFQ_TYPE_Q4_K) return (size_t)(in / OVFQ_QK) * OVFQ_Q4K_BYTES;
    if (type == OVFQ_TYPE_Q6_K) return (size_t)(in / OVFQ_QK) * OVFQ_Q6K_BYTES;
    return (size_t)in;  // Q8_0 quant plane
}

bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

// Shape checks of the weight constructors (RT/Q4KWeight.cs:46-62, RT/Q8Weight.cs:25-42).
int check_weight_shape(int type, int in, int out) {
    if (!valid_type(type)) return fail(OVFQ_ERR_TYPE, "unsupported weight type %d", type);
    if (in <= 0) return fail(OVFQ_ERR_RANGE, "inputSize (%d) must be positive", in);
    if (out <= 0) return fail(OVFQ_ERR_RANGE, "outputSize (%d) must be positive", out);
    if (type == OVFQ_TYPE_Q8_0) {
        if (in % OVFQ_Q8_BLOCK) return fail(OVFQ_ERR_SIZE, "inputSize (%d) must be a multiple of 32", in);
        if (in / OVFQ_Q8_BLOCK > 4000) return fail(OVFQ_ERR_SIZE, "Q8_0 inputSize (%d) above 128000", in);
    } else if (in % OVFQ_QK) {
        return fail(OVFQ_ERR_SIZE, "inputSize (%d) must be a multiple of 256", in);
    }
    if ((int64_t)in * out > (int64_t)1 << 40) return fail(OVFQ_ERR_SIZE, "weight too large");
    return OVFQ_OK;
}

int weight_create(ovfq_ctx* ctx, int type, const void* blocks, size_t nbytes, const float* q8_scales, int in,
                  int out, ovfq_weight** res, hipMemcpyKind kind) {
    if (!ctx) return fail(OVFQ_ERR_NULL, "ctx is NULL");
    if (!blocks) return fail(OVFQ_ERR_NULL, "blocks is NULL");
    if (!res) return fail(OVFQ_ERR_NULL, "out is NULL");
    int rc = check_weight_shape(type, in, out);
    if (rc) return rc;
    const size_t expected = block_bytes_per_row(type, in) * (size_t)out;
    if (nbytes < expected)
        return fail(OVFQ_ERR_SIZE, "blocks region (%zu B) is smaller than the expected %zu B", nbytes, expected);
    if (type == OVFQ_TYPE_Q8_0 && !q8_scales) return fail(OVFQ_ERR_NULL, "Q8_0 weight needs a scale plane");
    std::lock_guard<std::mutex> lk(ctx->mu);
    HIP_TRY(hipSetDevice(ctx->device));
    ovfq_weight* w = new ovfq_weight();
    w->ctx = ctx;
    w->type = type;
    w->in = in;
    w->out = out;
    hipError_t e = hipMalloc(&w->blocks, expected);
    if (e != hipSuccess) {
        delete w;
        return fail(OVFQ_ERR_HIP, "hipMalloc(%zu) failed: %s", expected, hipGetErrorString(e));
    }
    e = hipMemcpyAsync(w->blocks, blocks, expected, kind, ctx->stream);
    size_t scale_bytes = 0;
    if (e == hipSuccess && type == OVFQ_TYPE_Q8_0) {
        scale_bytes = (size_t)out * (in / OVFQ_Q8_BLOCK) * sizeof(float);
        e = hipMalloc(&w->scales, scale_bytes);
        if (e == hipSuccess) e = hipMemcpyAsync(w->scales, q8_scales, scale_bytes, kind, ctx->stream);
    }
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        if (w->blocks) (void)hipFree(w->blocks);
        if (w->scales) (void)hipFree(w->scales);
        delete w;
        return fail(OVFQ_ERR_HIP, "weight upload failed: %s", hipGetErrorString(e));
    }
    w->nbytes = expected + scale_bytes;
    ctx->live_weights++;
    *res = w;
    return ok();
}

// Quantises `rows` activation rows of length `in` for weight type `type` into the context scratch.
int quantize_into_scratch(ovfq_ctx* c, int type, const float* x_dev, int rows, int in, ovfq::ActQ* act) {
    const size_t n = (size_t)rows * in;
    int rc = ensure(c, c->act_q, n);
    if (rc) return rc;
    if (type == OVFQ_TYPE_Q8_0) {
        rc = ensure(c, c->act_s, n / 32 * sizeof(float));
        if (rc) return rc;
        HIP_TRY(ovfq::launch_quantize_q8_0(x_dev, (int64_t)(n / 32), (int8_t*)c->act_q.p, (float*)c->act_s.p,
                                           c->stream));
        *act = ovfq::ActQ{(const int8_t*)c->act_q.p, (const float*)c->act_s.p, nullptr};
    } else {
        rc = ensure(c, c->act_s, n / 256 * sizeof(float));
        if (rc) return rc;
        // the int16 bsums, then the same sums as fp16 (read by the tiled Q4_K kernels)
        rc = ensure(c, c->act_b, n / 16 * 2 * sizeof(int16_t));
        if (rc) return rc;
        int16_t* b = (int16_t*)c->act_b.p;
        uint16_t* bh = (uint16_t*)(b + n / 16);
        HIP_TRY(ovfq::launch_quantize_q8k(x_dev, (int64_t)(n / 256), (int8_t*)c->act_q.p, (float*)c->act_s.p, b,
                                          c->stream, bh));
        *act = ovfq::ActQ{(const int8_t*)c->act_q.p, (const float*)c->act_s.p, b, bh};
    }
    return OVFQ_OK;
}

// Decode-kernel selection knob for experiments: OVFQ_GEMV_DISABLE=1 routes M = 1 through the general kernel.
bool gemv_enabled() {
    static const bool on = [] {
        const char* v = getenv("OVFQ_GEMV_DISABLE");
        return !(v && *v == '1');
    }();
    return on;
}

// The small-M MFMA kernel serves M >= 3 unless OVFQ_SMALL_KERNEL=general (for measurements). M = 2 takes the
// multi-row decode kernel, or the general kernel where that cannot run: the small-M kernel was slower than the
// general one at M = 2 on MI355X for every Llama-3-8B shape.
bool small_mfma_enabled(int rows) {
    static const bool general = [] {
        const char* v = getenv("OVFQ_SMALL_KERNEL");
        return v && !strcmp(v, "general");
    }();
    return rows >= 3 && !general;
}

// Batched K-quant launch of rows >= 3: the 64-row-tiled MFMA kernel (true), else the small-M kernel where it takes
// the shape, else the general kernel. OVFQ_BATCHED_SMALL / _TILED force a kernel; automatic is the shape rule of
// mfma_tiled_preferred, and M >= 32 where the small-M kernel cannot run (input sizes past 16384).
bool use_tiled_mfma(const ovfq_ctx* c, int type, const ovfq::ProjJob* jobs, int count, int in, int rows) {
    if (!ovfq::mfma_supported(type) || rows < 3) return false;
    if (c->batched_kernel == OVFQ_BATCHED_TILED) return true;
    if (!small_mfma_enabled(rows) || !ovfq::mfma_small_supported(type, in)) return rows >= ovfq::kMfmaMinRows;
    if (c->batched_kernel == OVFQ_BATCHED_SMALL) return false;
    int o_tiles = 0;
    long out_rows = 0;
    for (int i = 0; i < count; i++) {
        o_tiles += (jobs[i].n_rows + 63) / 64;
        out_rows += jobs[i].n_rows;
    }
    return ovfq::mfma_tiled_preferred(type, rows, o_tiles, out_rows);
}

// Few activation rows: the multi-row decode kernel (each weight block unpacked once, one int8 dot per row). Its
// cost grows by about one block dot per row, the small-M MFMA kernel's hardly at all (MI355X, graph replay, us,
// multi-row / previous kernel): 2 rows 14336x4096 Q4_K 10.8 / 13.7, Q6_K 4096x14336 16.6 / 19.5; 4 rows 13.0 /
// 14.9; 8 rows 17.8 / 16.3. A fused q/k/v launch (three weights, which the small-M kernel runs one by one) is
// 7.0 / 19.1 at 3 rows and 10.1 / 20.0 at 8. Automatic: up to 4 rows, and up to 8 for three or more weights.
// A gate/up-shaped Q4_K pair (`pair_out` output rows each) tall enough for the expert-stream kernel takes that kernel
// from 3 rows (MI355X, us, multi-row / stream with its Q8_K launch, 2x14336x4096: 2 rows 17.2 / 20.7, 3 rows
// 20.1 / 19.4, 4 rows 22.9 / 19.6).
bool use_gemv_rows(const ovfq_ctx* c, int type, int in, int rows, int count, int pair_out = 0) {
    if ((type != OVFQ_TYPE_Q4_K && type != OVFQ_TYPE_Q6_K) || !ovfq::gemv_rows_supported(in, rows)) return false;
    // Decode rows of 16384 < K <= 32768, past the one-row kernel (which is faster wherever it runs: MI355X, us, one-row
    // / multi-row kernel at M = 1: 4096x4096 Q4_K 4.8 / 5.5, 4096x14336 Q6_K 14.0 / 14.3). At K = 28672 it
    // replaces the general kernel: 8192 rows Q4_K 31.1 -> 28.7, Q6_K 51.7 -> 40.4.
    if (rows == 1) return gemv_enabled() && !ovfq::gemv_supported(in);
    if (c->batched_kernel == OVFQ_BATCHED_ROWS) return true;
    if (c->batched_kernel != OVFQ_BATCHED_AUTO) return false;
    if (count == 2 && pair_out > 0 && rows >= 3 && small_mfma_enabled(rows) &&
        ovfq::stream_pair_preferred(type, in, pair_out))
        return false;
    return rows <= 4 || count >= 3;
}

// Whether the projection launch quantises its fp32 input itself instead of a separate Q8_K / Q8_0 launch: one row on
// a decode kernel (K <= 8192), or up to 64 super-blocks of rows on the multi-row decode kernel.
bool quantize_in_launch(const ovfq_ctx* c, int type, int in, int rows, int count, int pair_out = 0) {
    if (type == OVFQ_TYPE_Q8_0) return rows == 1 && gemv_enabled() && ovfq::q8_0_gemv_quantize_inside(in);
    if (rows == 1 && ovfq::gemv_supported(in)) return gemv_enabled() && ovfq::gemv_quantize_inside(in);
    return use_gemv_rows(c, type, in, rows, count, pair_out) && ovfq::gemv_rows_quantize_inside(in, rows);
}

// One launch for `count` weights sharing an activation: either the fp32 activation x (quantised inside the
// decode kernel) or an already-quantised `act`.
int launch_projection(ovfq_ctx* c, const ovfq_weight* const* ws, int count, const float* const* biases,
                      float* const* ys, int rows, ovfq::ActQ act, const float* x = nullptr) {
    ovfq::ProjJob jobs[ovfq::kMaxJobs];
    for (int i = 0; i < count; i++) {
        jobs[i].w = static_cast<const uint8_t*>(ws[i]->blocks);
        jobs[i].ws = ws[i]->scales;
        jobs[i].bias = biases ? biases[i] : nullptr;
        jobs[i].y = ys[i];
        jobs[i].n_rows = ws[i]->out;
        jobs[i].pre = static_cast<const uint8_t*>(ws[i]->mfma);
    }
    const int type = ws[0]->type;
    const int in = ws[0]->in;
    const int pair_out = count == 2 && ws[0]->out == ws[1]->out ? ws[0]->out : 0;
    if (x && rows > 1 && !use_gemv_rows(c, type, in, rows, count, pair_out))
        return fail(OVFQ_ERR_SIZE, "in-launch quantisation of %d rows needs the multi-row decode kernel", rows);
    // Every kernel below reads either the fp32 input (decode kernels that quantise it) or the quantised activation.
    if (!x && (!act.q || !act.s)) return fail(OVFQ_ERR_NULL, "projection launch without a quantised activation");
    if (type == OVFQ_TYPE_Q8_0) {
        // The int8-MFMA kernel from 8 rows; for inputs up to 8192 from 6 rows, and from 4 rows for 8192 outputs or
        // more. Its time is flat up to 16 rows (one 16-row tile, one-wave workgroups of 16 outputs), the row
        // kernel's grows by a pass over the weights per row (MI355X, graph replay, us, row kernel / MFMA kernel):
        // 4096x4096 at 4 rows 21.6 / 25.7, 16 rows 63.6 / 25.8, 64 rows 235 / 46.0, 512 rows - / 52.0; 14336x4096 at
        // 4 rows 43.0 / 31.6, 16 rows 149 / 31.6; 4096x14336 at 16 rows 164 / 84.3, 24 rows 234 / 122, 512 rows - /
        // 168. OVFQ_Q8_MFMA_MIN_ROWS sets a plain row bound instead (measurements).
        static const int q8_mfma_min = [] {
            const char* v = getenv("OVFQ_Q8_MFMA_MIN_ROWS");
            return v && *v ? atoi(v) : 0;
        }();
        long outs = 0;
        for (int i = 0; i < count; i++) outs += jobs[i].n_rows;
        bool q8_mfma = q8_mfma_min > 0 ? rows >= q8_mfma_min
                                       : rows >= 8 || (in <= 8192 && (rows >= 6 || (rows >= 4 && outs >= 8192)));
        if (c->batched_kernel == OVFQ_BATCHED_TILED) q8_mfma = rows >= 2;
        else if (c->batched_kernel != OVFQ_BATCHED_AUTO) q8_mfma = false;
        // The decode GEMV over 1 .. 8 rows where rows * K fits its LDS copy (it loads each block once for all rows:
        // 4096x4096 at 2 / 4 rows 7.2 / 7.8 us against the row kernel's 14.1 / 21.5 and the MFMA kernel's 25.6 / 25.8;
        // 14336x4096 at 4 rows 16.6 against 43.1 / 31.9). One row always takes it where it runs (the batched-kernel
        // choice is for 2 or more rows, and the caller may have left the quantisation to it); forced SMALL sends
        // 2 .. 8 rows to the row kernel, forced TILED to the MFMA kernel.
        const bool q8_choice = c->batched_kernel == OVFQ_BATCHED_AUTO || c->batched_kernel == OVFQ_BATCHED_ROWS;
        const bool q8_rows = gemv_enabled() && ovfq::q8_0_gemv_rows_supported(in, rows) && (rows == 1 || q8_choice);
        if (x && !q8_rows) return fail(OVFQ_ERR_SIZE, "in-launch Q8_0 quantisation needs the decode kernel");
        if (q8_rows)
            HIP_TRY(ovfq::launch_q8_0_gemv(jobs, count, in, rows, x, act, c->stream));
        else if (q8_mfma && ovfq::q8_0_mfma_supported(in, rows))
            HIP_TRY(ovfq::launch_project_q8_0_mfma(jobs, count, in, rows, act, c->stream));
        else
            HIP_TRY(ovfq::launch_project_q8_0(jobs, count, in, rows, act, c->stream));
    } else if (rows == 1 && gemv_enabled() && ovfq::gemv_supported(in)) {
        HIP_TRY(ovfq::launch_gemv_kquant(type, jobs, count, in, x, act, c->stream));
    } else if (use_gemv_rows(c, type, in, rows, count, pair_out)) {
        HIP_TRY(ovfq::launch_gemv_rows_kquant(type, jobs, count, in, rows, x, act, c->stream));
    } else if (use_tiled_mfma(c, type, jobs, count, in, rows)) {
        HIP_TRY(ovfq::launch_project_mfma(type, jobs, count, in, rows, act, c->stream));
    } else if (small_mfma_enabled(rows) && ovfq::mfma_small_supported(type, in)) {
        // Few rows: 16-row MFMA tiles with super-block-parallel waves; a gate/up-shaped pair shares one launch.
        const bool pair = count == 2 && jobs[0].n_rows == jobs[1].n_rows;
        for (int i = 0; i < count; i += pair ? 2 : 1) {
            const uint8_t* w0 = jobs[i].w;
            const uint8_t* w1 = pair ? jobs[i + 1].w : nullptr;
            ovfq::GroupLaunch L{};
            L.w0 = &w0;
            L.w1 = pair ? &w1 : nullptr;
            L.bias0 = jobs[i].bias;
            L.bias1 = pair ? jobs[i + 1].bias : nullptr;
            L.y0 = jobs[i].y;
            L.y1 = pair ? jobs[i + 1].y : nullptr;
            L.n_rows = jobs[i].n_rows;
            L.in = in;
            L.experts = 1;
            L.rows = rows;
            L.act = act;
            HIP_TRY(ovfq::launch_mfma_small(type, L, c->stream));
        }
    } else {
        HIP_TRY(ovfq::launch_project_kquant(type, jobs, count, in, rows, act, c->stream));
    }
    return OVFQ_OK;
}

int check_weight(const ovfq_ctx* ctx, const ovfq_weight* w) {
    if (!w) return fail(OVFQ_ERR_NULL, "weight is NULL");
    if (w->ctx != ctx) return fail(OVFQ_ERR_SIZE, "weight belongs to another context");
    return OVFQ_OK;
}

int check_rows(int rows) {
    if (rows <= 0) return fail(OVFQ_ERR_RANGE, "rows (%d) must be positive", rows);
    if (rows > 65536) return fail(OVFQ_ERR_RANGE, "rows (%d) above 65536", rows);
    return OVFQ_OK;
}

// An activation or output plane of `rows` x `cols` elements must stay below 2^31 elements, the length limit of
// the reference's spans (its scratch and outputs are Span<T>); the kernels index such planes with 32-bit
// offsets.
int check_plane(int64_t rows, int64_t cols, const char* what) {
    if (rows * cols >= ((int64_t)1 << 31))
        return fail(OVFQ_ERR_SIZE, "%s of %lld x %lld elements exceeds 2^31 - 1", what, (long long)rows,
                    (long long)cols);
    return OVFQ_OK;
}

// Device pointers handed to the _dev entry points must keep the kernels' 4-byte (quants/bsums) alignment.
// Carves 256-byte-aligned pieces off a base pointer.
struct Carver {
    char* p;
    size_t used = 0;
    template <class T>
    T* take(size_t bytes) {
        T* r = reinterpret_cast<T*>(p ? p + used : nullptr);
        used += (bytes + 255) & ~size_t(255);
        return r;
    }
};

bool rc_align(const void* p) { return p && !aligned(p, 4); }

int check_dev_align(const void* p, const char* name) {
    if (p && !aligned(p, 4)) return fail(OVFQ_ERR_SIZE, "%s must be 4-byte aligned", name);
    return OVFQ_OK;
}

}  // namespace

extern "C" {

const char* ovfq_last_error(void) { return g_last_error.c_str(); }

const char* ovfq_version(void) { return "ovfq 0.1 (gfx950)"; }

int ovfq_ctx_create(int device, ovfq_ctx** out) {
    if (!out) return fail(OVFQ_ERR_NULL, "out is NULL");
    int n = 0;
    HIP_TRY(hipGetDeviceCount(&n));
    if (device < 0 || device >= n) return fail(OVFQ_ERR_RANGE, "device %d out of range (%d devices)", device, n);
    HIP_TRY(hipSetDevice(device));
    // The allocation-free entry point's fixed scratch: resolve this device's copy once, with it current.
    HIP_TRY(ovfq::noalloc_scratch_init(device));
    ovfq_ctx* c = new ovfq_ctx();
    c->device = device;
    hipError_t e = hipStreamCreateWithFlags(&c->own_stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete c;
        return fail(OVFQ_ERR_HIP, "hipStreamCreate failed: %s", hipGetErrorString(e));
    }
    c->stream = c->own_stream;
    *out = c;
    return ok();
}

int ovfq_ctx_destroy(ovfq_ctx* c) {
    if (!c) return fail(OVFQ_ERR_NULL, "ctx is NULL");
    {
        std::lock_guard<std::mutex> lk(c->mu);
        // A weight locks its context when destroyed, so the context must outlive every weight made on it.
        if (c->live_weights > 0)
            return fail(OVFQ_ERR_STATE, "context still owns %d weight(s): destroy them first", c->live_weights);
        (void)hipSetDevice(c->device);
        (void)hipStreamSynchronize(c->stream);
        DevBuf* bufs[] = {&c->act_q,   &c->act_s,   &c->act_b,      &c->x_stage,
                          &c->y_stage, &c->y2_stage, &c->bias_stage, &c->moe};
        for (DevBuf* b : bufs)
            if (b->p) (void)hipFree(b->p);
        for (void* p : c->retired) (void)hipFree(p);
        if (c->h_up.p) (void)hipHostFree(c->h_up.p);
        if (c->h_down.p) (void)hipHostFree(c->h_down.p);
        if (c->own_stream) (void)hipStreamDestroy(c->own_stream);
    }
    delete c;
    return ok();
}

int ovfq_ctx_set_stream(ovfq_ctx* c, void* stream) {
    if (!c) return fail(OVFQ_ERR_NULL, "ctx is NULL");
    std::lock_guard<std::mutex> lk(c->mu);
    HIP_TRY(hipSetDevice(c->device));
    HIP_TRY(hipStreamSynchronize(c->stream));
    c->stream = static_cast<hipStream_t>(stream);
    return ok();
}

int ovfq_ctx_reset_stream(ovfq_ctx* c) {
    if (!c) return fail(OVFQ_ERR_NULL, "ctx is NULL");
    std::lock_guard<std::mutex> lk(c->mu);
    HIP_TRY(hipSetDevice(c->device));
    HIP_TRY(hipStreamSynchronize(c->stream));
    c->stream = c->own_stream;
    return ok();
}

int ovfq_ctx_release_retired(ovfq_ctx* c) {
    if (!c) return fail(OVFQ_ERR_NULL, "ctx is NULL");
    std::lock_guard<std::mutex> lk(c->mu);
    HIP_TRY(hipSetDevice(c->device));
    // queued work may still read a superseded buffer
    HIP_TRY(hipStreamSynchronize(c->stream));
    hipError_t first = hipSuccess;
    for (void* p : c->retired) {
        hipError_t e = hipFree(p);
        if (first == hipSuccess) first = e;
    }
    c->retired.clear();
    c->retired_bytes = 0;
    if (first != hipSuccess) return fail(OVFQ_ERR_HIP, "hipFree failed: %s", hipGetErrorString(first));
    return ok();
}

int ovfq_ctx_scratch_bytes(ovfq_ctx* c, size_t* live, size_t* retired) {
    if (!c) return fail(OVFQ_ERR_NULL, "ctx is NULL");
    std::lock_guard<std::mutex> lk(c->mu);
    const DevBuf* bufs[] = {&c->act_q, &c->act_s, &c->act_b, &c->x_stage, &c->y_stage, &c->y2_stage, &c->bias_stage,
                            &c->moe};
    size_t n = 0;
    for (const DevBuf* b : bufs) n += b->cap;
    if (live) *live = n;
    if (retired) *retired = c->retired_bytes;
    return ok();
}

int ovfq_ctx_set_batched_kernel(ovfq_ctx* c, int kernel) {
    if (!c) return fail(OVFQ_ERR_NULL, "ctx is NULL");
    if (kernel != OVFQ_BATCHED_AUTO && kernel != OVFQ_BATCHED_SMALL && kernel != OVFQ_BATCHED_TILED &&
        kernel != OVFQ_BATCHED_ROWS)
        return fail(OVFQ_ERR_RANGE, "unknown batched kernel choice %d", kernel);
    std::lock_guard<std::mutex> lk(c->mu);
    c->batched_kernel = kernel;
    return ok();
}

int ovfq_ctx_synchronize(ovfq_ctx* c) {
    if (!c) return fail(OVFQ_ERR_NULL, "ctx is NULL");
    std::lock_guard<std::mutex> lk(c->mu);
    HIP_TRY(hipSetDevice(c->device));
    HIP_TRY(hipStreamSynchronize(c->stream));
    return ok();
}

int ovfq_weight_create(ovfq_ctx* ctx, int type, const void* blocks, size_t nbytes, const float* q8_scales,
                       int input_size, int output_size, ovfq_weight** out) {
    return weight_create(ctx, type, blocks, nbytes, q8_scales, input_size, output_size, out,
                         hipMemcpyHostToDevice);
}

int ovfq_weight_create_from_device(ovfq_ctx* ctx, int type, const void* blocks, size_t nbytes,
                                   const float* q8_scales, int input_size, int output_size, ovfq_weight** out) {
    return weight_create(ctx, type, blocks, nbytes, q8_scales, input_size, output_size, out,
                         hipMemcpyDeviceToDevice);
}

// GGUF tensor types whose resident form is the Q8_0 planes: Q8_0 itself (de-interleaved) and the 5-bit types, which
// the reference's loader decodes to F32 and requantises to Q8_0 (LD/GgufLlamaLoader.cs:665-680).
bool gguf_as_q8(int type) { return type == OVFQ_TYPE_Q8_0 || type == OVFQ_TYPE_Q5_0 || type == OVFQ_TYPE_Q5_K; }

// Source bytes per 32 weights of such a tensor: 34 for Q8_0 (fp16 d + 32 int8); 22 for Q5_0 (a block) and for Q5_K
// (176 bytes per 256).
size_t gguf_bytes_per_32(int type) { return type == OVFQ_TYPE_Q8_0 ? 34 : 22; }

// Shape checks of a GGUF tensor that becomes Q8_0 planes: the resident Q8_0 weight's, and whole Q5_K super-blocks.
int check_gguf_q8_shape(int type, int in, int out) {
    int rc = check_weight_shape(OVFQ_TYPE_Q8_0, in, out);
    if (rc) return rc;
    if (type == OVFQ_TYPE_Q5_K && in % OVFQ_QK)
        return fail(OVFQ_ERR_SIZE, "Q5_K inputSize (%d) must be a multiple of 256", in);
    return OVFQ_OK;
}

hipError_t launch_gguf_to_q8(int type, const void* src, int64_t n_blocks, int8_t* q, float* s, hipStream_t st) {
    if (type == OVFQ_TYPE_Q8_0) return ovfq::launch_q8_0_deinterleave(src, n_blocks, q, s, st);
    return ovfq::launch_q5_to_q8_0(src, type == OVFQ_TYPE_Q5_K, n_blocks, q, s, st);
}

static int weight_create_gguf(ovfq_ctx* ctx, int type, const void* src, size_t nbytes, int in, int out,
                              ovfq_weight** res, bool host) {
    if (!gguf_as_q8(type))
        return weight_create(ctx, type, src, nbytes, nullptr, in, out, res,
                             host ? hipMemcpyHostToDevice : hipMemcpyDeviceToDevice);
    if (!ctx) return fail(OVFQ_ERR_NULL, "ctx is NULL");
    if (!src) return fail(OVFQ_ERR_NULL, "gguf_bytes is NULL");
    if (!res) return fail(OVFQ_ERR_NULL, "out is NULL");
    int rc = check_gguf_q8_shape(type, in, out);
    if (rc) return rc;
    const int64_t n_blocks = (int64_t)out * (in / OVFQ_Q8_BLOCK);
    const size_t gguf_len = (size_t)n_blocks * gguf_bytes_per_32(type);
    if (nbytes < gguf_len)
        return fail(OVFQ_ERR_SIZE, "GGUF region (%zu B) is smaller than the expected %zu B", nbytes, gguf_len);
    if (!host && type == OVFQ_TYPE_Q8_0 && !aligned(src, 2))
        return fail(OVFQ_ERR_SIZE, "device gguf_bytes must be 2-byte aligned");
    std::lock_guard<std::mutex> lk(ctx->mu);
    HIP_TRY(hipSetDevice(ctx->device));
    ovfq_weight* w = new ovfq_weight();
    w->ctx = ctx;
    w->type = OVFQ_TYPE_Q8_0;
    w->in = in;
    w->out = out;
    void* staged = nullptr;
    hipError_t e = hipMalloc(&w->blocks, (size_t)n_blocks * OVFQ_Q8_BLOCK);
    if (e == hipSuccess) e = hipMalloc(&w->scales, (size_t)n_blocks * sizeof(float));
    const void* dsrc = src;
    if (e == hipSuccess && host) {
        e = hipMalloc(&staged, gguf_len);
        if (e == hipSuccess) e = hipMemcpyAsync(staged, src, gguf_len, hipMemcpyHostToDevice, ctx->stream);
        dsrc = staged;
    }
    if (e == hipSuccess)
        e = launch_gguf_to_q8(type, dsrc, n_blocks, static_cast<int8_t*>(w->blocks), w->scales, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (staged) (void)hipFree(staged);
    if (e != hipSuccess) {
        if (w->blocks) (void)hipFree(w->blocks);
        if (w->scales) (void)hipFree(w->scales);
        delete w;
        return fail(OVFQ_ERR_HIP, "GGUF upload to Q8_0 failed: %s", hipGetErrorString(e));
    }
    w->nbytes = (size_t)n_blocks * (OVFQ_Q8_BLOCK + sizeof(float));
    ctx->live_weights++;
    *res = w;
    return ok();
}

int ovfq_weight_create_gguf(ovfq_ctx* ctx, int type, const void* gguf_bytes, size_t nbytes, int input_size,
                            int output_size, ovfq_weight** out) {
    return weight_create_gguf(ctx, type, gguf_bytes, nbytes, input_size, output_size, out, true);
}

int ovfq_weight_create_gguf_dev(ovfq_ctx* ctx, int type, const void* gguf_bytes, size_t nbytes, int input_size,
                                int output_size, ovfq_weight** out) {
    return weight_create_gguf(ctx, type, gguf_bytes, nbytes, input_size, output_size, out, false);
}

// GgufLlamaLoader.LoadExperts (LD/GgufLlamaLoader.cs:600-690) for Q4_K / Q6_K / Q8_0: a 3-D expert tensor
// [ne0 = in, ne1 = out, ne2 = n_experts] (expert axis slowest) -> one weight per expert. All experts live in one
// device allocation, each slice starting on a 256-byte boundary (expert e at e * stride); Q4_K/Q6_K bytes are
// copied verbatim, Q8_0 blocks de-interleaved per expert into quant planes [E][stride_q] then scale planes
// [E][stride_s].
static int experts_gguf_impl(ovfq_ctx* ctx, int type, const void* src, size_t nbytes, int in, int out,
                             int n_experts, ovfq_weight** res, bool host) {
    if (!ctx) return fail(OVFQ_ERR_NULL, "ctx is NULL");
    if (!src) return fail(OVFQ_ERR_NULL, "gguf_bytes is NULL");
    if (!res) return fail(OVFQ_ERR_NULL, "out is NULL");
    const bool q8 = gguf_as_q8(type);
    int rc = q8 ? check_gguf_q8_shape(type, in, out) : check_weight_shape(type, in, out);
    if (rc) return rc;
    if (n_experts <= 0 || n_experts > OVFQ_MAX_EXPERT_SLICES)
        return fail(OVFQ_ERR_RANGE, "n_experts (%d) must be in [1, %d]", n_experts, OVFQ_MAX_EXPERT_SLICES);
    const int64_t blocks_per_expert = (int64_t)out * (in / OVFQ_Q8_BLOCK);
    const size_t src_expert =
        q8 ? (size_t)blocks_per_expert * gguf_bytes_per_32(type) : block_bytes_per_row(type, in) * (size_t)out;
    if (nbytes / (size_t)n_experts < src_expert)
        return fail(OVFQ_ERR_SIZE, "expert tensor region (%zu B) is smaller than the expected %d x %zu B", nbytes,
                    n_experts, src_expert);
    if (!host && type == OVFQ_TYPE_Q8_0 && !aligned(src, 2))
        return fail(OVFQ_ERR_SIZE, "device gguf_bytes must be 2-byte aligned");
    auto pad = [](size_t b) { return (b + 255) & ~size_t(255); };
    const size_t q_bytes = q8 ? (size_t)out * in : src_expert;
    const size_t s_bytes = q8 ? (size_t)blocks_per_expert * sizeof(float) : 0;
    const size_t q_stride = pad(q_bytes), s_stride = pad(s_bytes);
    const size_t E = (size_t)n_experts;
    const hipMemcpyKind kind = host ? hipMemcpyHostToDevice : hipMemcpyDeviceToDevice;
    std::lock_guard<std::mutex> lk(ctx->mu);
    HIP_TRY(hipSetDevice(ctx->device));
    char* base = nullptr;
    void* staged = nullptr;
    hipError_t e = hipMalloc((void**)&base, E * (q_stride + s_stride));
    if (e == hipSuccess && !q8) {
        for (size_t x = 0; x < E && e == hipSuccess; x++)
            e = hipMemcpyAsync(base + x * q_stride, static_cast<const char*>(src) + x * src_expert, src_expert, kind,
                               ctx->stream);
    } else if (e == hipSuccess) {
        const char* dsrc = static_cast<const char*>(src);
        if (host) {
            e = hipMalloc(&staged, E * src_expert);
            if (e == hipSuccess) e = hipMemcpyAsync(staged, src, E * src_expert, hipMemcpyHostToDevice, ctx->stream);
            dsrc = static_cast<const char*>(staged);
        }
        float* scales = reinterpret_cast<float*>(base + E * q_stride);
        for (size_t x = 0; x < E && e == hipSuccess; x++)
            e = launch_gguf_to_q8(type, dsrc + x * src_expert, blocks_per_expert,
                                  reinterpret_cast<int8_t*>(base + x * q_stride),
                                  reinterpret_cast<float*>(reinterpret_cast<char*>(scales) + x * s_stride), ctx->stream);
    }
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (staged) (void)hipFree(staged);
    if (e != hipSuccess) {
        if (base) (void)hipFree(base);
        return fail(OVFQ_ERR_HIP, "expert tensor upload failed: %s", hipGetErrorString(e));
    }
    SharedPlane* sp = new SharedPlane();
    sp->p = base;
    sp->refs = n_experts;
    for (size_t x = 0; x < E; x++) {
        ovfq_weight* w = new ovfq_weight();
        w->ctx = ctx;
        w->type = q8 ? OVFQ_TYPE_Q8_0 : type;
        w->in = in;
        w->out = out;
        w->blocks = base + x * q_stride;
        w->scales = q8 ? reinterpret_cast<float*>(base + E * q_stride + x * s_stride) : nullptr;
        w->nbytes = q_bytes + s_bytes;
        w->shared = sp;
        res[x] = w;
    }
    ctx->live_weights += n_experts;
    return ok();
}

int ovfq_weight_create_experts_gguf(ovfq_ctx* ctx, int type, const void* gguf_bytes, size_t nbytes, int input_size,
                                    int output_size, int n_experts, ovfq_weight** out) {
    return experts_gguf_impl(ctx, type, gguf_bytes, nbytes, input_size, output_size, n_experts, out, true);
}

int ovfq_weight_create_experts_gguf_dev(ovfq_ctx* ctx, int type, const void* gguf_bytes, size_t nbytes,
                                        int input_size, int output_size, int n_experts, ovfq_weight** out) {
    return experts_gguf_impl(ctx, type, gguf_bytes, nbytes, input_size, output_size, n_experts, out, false);
}

int ovfq_weight_destroy(ovfq_weight* w) {
    if (!w) return fail(OVFQ_ERR_NULL, "weight is NULL");
    {
        std::lock_guard<std::mutex> lk(w->ctx->mu);
        (void)hipSetDevice(w->ctx->device);
        (void)hipStreamSynchronize(w->ctx->stream);
        if (w->shared) {
            if (--w->shared->refs == 0) {
                (void)hipFree(w->shared->p);
                delete w->shared;
            }
        } else {
            if (w->blocks) (void)hipFree(w->blocks);
            if (w->scales) (void)hipFree(w->scales);
        }
        if (w->mfma) (void)hipFree(w->mfma);
        w->ctx->live_weights--;
    }
    delete w;
    return ok();
}

int ovfq_weight_prepare_mfma(ovfq_ctx* ctx, ovfq_weight* w) {
    if (!ctx) return fail(OVFQ_ERR_NULL, "ctx is NULL");
    int rc = check_weight(ctx, w);
    if (rc) return rc;
    if (w->type != OVFQ_TYPE_Q4_K && w->type != OVFQ_TYPE_Q6_K)
        return fail(OVFQ_ERR_TYPE, "an MFMA-ready copy exists for K-quant weights only");
    // Q4_K operands cost a few packed multiplies per dword to build in registers; streaming them prepared
    // (3.7x the bytes) measured slower, so Q4_K weights keep the GGUF-operand path.
    if (w->type == OVFQ_TYPE_Q4_K) return ok();
    std::lock_guard<std::mutex> lk(ctx->mu);
    if (w->mfma) return ok();
    HIP_TRY(hipSetDevice(ctx->device));
    void* pre = nullptr;
    hipError_t e = hipMalloc(&pre, ovfq::mfma_prepared_bytes(w->in, w->out));
    if (e == hipSuccess)
        e = ovfq::launch_mfma_prepare(w->type, static_cast<const uint8_t*>(w->blocks), w->in, w->out,
                                      static_cast<uint8_t*>(pre), ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        if (pre) (void)hipFree(pre);
        return fail(OVFQ_ERR_HIP, "MFMA-ready copy failed: %s", hipGetErrorString(e));
    }
    w->mfma = pre;
    return ok();
}

int ovfq_weight_info(const ovfq_weight* w, int* type, int* input_size, int* output_size, size_t* byte_count,
                     const void** device_blocks) {
    if (!w) return fail(OVFQ_ERR_NULL, "weight is NULL");
    if (type) *type = w->type;
    if (input_size) *input_size = w->in;
    if (output_size) *output_size = w->out;
    if (byte_count) *byte_count = w->nbytes;
    if (device_blocks) *device_blocks = w->blocks;
    return ok();
}

static int decode_row_impl(ovfq_ctx* ctx, const ovfq_weight* w, int row, float* dst, bool host) {
    if (!ctx) return fail(OVFQ_ERR_NULL, "ctx is NULL");
    int rc = check_weight(ctx, w);
    if (rc) return rc;
    if (!dst) return fail(OVFQ_ERR_NULL, "dst is NULL");
    if (row < 0 || row >= w->out) return fail(OVFQ_ERR_RANGE, "row %d out of range [0, %d)", row, w->out);
    std::lock_guard<std::mutex> lk(ctx->mu);
    HIP_TRY(hipSetDevice(ctx->device));
    float* d = dst;
    if (host) {
        rc = ensure(ctx, ctx->y_stage, (size_t)w->in * 4);
        if (rc) return rc;
        d = (float*)ctx->y_stage.p;
    }
    HIP_TRY(ovfq::launch_decode_row(w->type, w->blocks, w->scales, w->in, row, d, ctx->stream));
    if (host) {
        HostIO io(ctx);
        if ((rc = io.down(dst, d, (size_t)w->in * 4)) || (rc = io.finish())) return rc;
    }
    return ok();
}

int ovfq_weight_decode_row(ovfq_ctx* ctx, const ovfq_weight* w, int row, float* dst) {
    return decode_row_impl(ctx, w, row, dst, true);
}

int ovfq_weight_decode_row_dev(ovfq_ctx* ctx, const ovfq_weight* w, int row, float* dst) {
    return decode_row_impl(ctx, w, row, dst, false);
}

// ---------------------------------------------------------------------------------------- quantisation

static int quantize_impl(ovfq_ctx* ctx, bool k_quant, const float* x, int rows, int k, int8_t* q, float* s,
                         int16_t* b, bool host) {
    if (!ctx) return fail(OVFQ_ERR_NULL, "ctx is NULL");
    if (!x || !q || !s || (k_quant && !b)) return fail(OVFQ_ERR_NULL, "a source or scratch pointer is NULL");
    int rc = check_rows(rows);
    if (rc) return rc;
    const int blk = k_quant ? OVFQ_QK : OVFQ_Q8_BLOCK;
    if (k <= 0 || k % blk)
        return fail(OVFQ_ERR_SIZE, "Source length (%d) must be a multiple of %d.", k, blk);
    if ((rc = check_plane(rows, k, "activation"))) return rc;
    if (!host) {
        if ((rc = check_dev_align(x, "x")) || (rc = check_dev_align(q, "quants")) ||
            (rc = check_dev_align(s, "scales")) || (rc = check_dev_align(b, "bsums")))
            return rc;
    }
    const size_t n = (size_t)rows * k;
    std::lock_guard<std::mutex> lk(ctx->mu);
    HIP_TRY(hipSetDevice(ctx->device));
    const float* xd = x;
    int8_t* qd = q;
    float* sd = s;
    int16_t* bd = b;
    HostIO io(ctx);
    if (host) {
        if ((rc = ensure(ctx, ctx->x_stage, n * 4))) return rc;
        if ((rc = ensure(ctx, ctx->y_stage, n))) return rc;
        if ((rc = ensure(ctx, ctx->y2_stage, n / blk * 4))) return rc;
        if (k_quant && (rc = ensure(ctx, ctx->bias_stage, n / 16 * 2))) return rc;
        if ((rc = io.up(ctx->x_stage.p, x, n * 4))) return rc;
        xd = (const float*)ctx->x_stage.p;
        qd = (int8_t*)ctx->y_stage.p;
        sd = (float*)ctx->y2_stage.p;
        bd = (int16_t*)ctx->bias_stage.p;
    }
    if (k_quant) {
        HIP_TRY(ovfq::launch_quantize_q8k(xd, (int64_t)(n / OVFQ_QK), qd, sd, bd, ctx->stream));
    } else {
        HIP_TRY(ovfq::launch_quantize_q8_0(xd, (int64_t)(n / OVFQ_Q8_BLOCK), qd, sd, ctx->stream));
    }
    if (host) {
        if ((rc = io.down(q, qd, n)) || (rc = io.down(s, sd, n / blk * 4)) ||
            (k_quant && (rc = io.down(b, bd, n / 16 * 2))) || (rc = io.finish()))
            return rc;
    }
    return ok();
}

int ovfq_quantize_q8k(ovfq_ctx* ctx, const float* x, int rows, int k, int8_t* q, float* s, int16_t* b) {
    return quantize_impl(ctx, true, x, rows, k, q, s, b, true);
}
int ovfq_quantize_q8k_dev(ovfq_ctx* ctx, const float* x, int rows, int k, int8_t* q, float* s, int16_t* b) {
    return quantize_impl(ctx, true, x, rows, k, q, s, b, false);
}
int ovfq_quantize_q8_0(ovfq_ctx* ctx, const float* x, int rows, int k, int8_t* q, float* s) {
    return quantize_impl(ctx, false, x, rows, k, q, s, nullptr, true);
}
int ovfq_quantize_q8_0_dev(ovfq_ctx* ctx, const float* x, int rows, int k, int8_t* q, float* s) {
    return quantize_impl(ctx, false, x, rows, k, q, s, nullptr, false);
}

// ---------------------------------------------------------------------------------------- projections

// Shared body of the fused (same activation) projections: count weights, one quantisation, one launch.
static int project_impl(ovfq_ctx* ctx, int count, const ovfq_weight* const* ws, const float* x, int rows,
                        const float* const* biases, float* const* ys, bool host) {
    if (!ctx) return fail(OVFQ_ERR_NULL, "ctx is NULL");
    if (count < 1 || count > ovfq::kMaxJobs) return fail(OVFQ_ERR_RANGE, "count (%d) must be in [1, 4]", count);
    if (!ws || !ys) return fail(OVFQ_ERR_NULL, "weights / outputs array is NULL");
    if (!x) return fail(OVFQ_ERR_NULL, "input is NULL");
    int rc = check_rows(rows);
    if (rc) return rc;
    for (int i = 0; i < count; i++) {
        if ((rc = check_weight(ctx, ws[i]))) return rc;
        if (!ys[i]) return fail(OVFQ_ERR_NULL, "output %d is NULL", i);
        if (ws[i]->type != ws[0]->type) return fail(OVFQ_ERR_TYPE, "fused weights must share a type");
        if (ws[i]->in != ws[0]->in) return fail(OVFQ_ERR_SIZE, "fused weights must share inputSize");
        if (!host && (rc = check_dev_align(ys[i], "output"))) return rc;
        if ((rc = check_plane(rows, ws[i]->out, "output"))) return rc;
    }
    if (!host && (rc = check_dev_align(x, "input"))) return rc;
    const int in = ws[0]->in;
    if ((rc = check_plane(rows, in, "activation"))) return rc;
    std::lock_guard<std::mutex> lk(ctx->mu);
    HIP_TRY(hipSetDevice(ctx->device));
    const float* xd = x;
    const float* bd[ovfq::kMaxJobs] = {nullptr, nullptr, nullptr, nullptr};
    float* yd[ovfq::kMaxJobs];
    size_t y_off[ovfq::kMaxJobs];
    HostIO io(ctx);
    if (host) {
        size_t ytotal = 0, btotal = 0;
        for (int i = 0; i < count; i++) {
            y_off[i] = ytotal;
            ytotal += (size_t)rows * ws[i]->out;
            if (biases && biases[i]) btotal += ws[i]->out;
        }
        if ((rc = ensure(ctx, ctx->x_stage, (size_t)rows * in * 4))) return rc;
        if ((rc = ensure(ctx, ctx->y_stage, ytotal * 4))) return rc;
        if (btotal && (rc = ensure(ctx, ctx->bias_stage, btotal * 4))) return rc;
        if ((rc = io.up(ctx->x_stage.p, x, (size_t)rows * in * 4))) return rc;
        xd = (const float*)ctx->x_stage.p;
        size_t boff = 0;
        for (int i = 0; i < count; i++) {
            yd[i] = (float*)ctx->y_stage.p + y_off[i];
            if (biases && biases[i]) {
                float* bdst = (float*)ctx->bias_stage.p + boff;
                if ((rc = io.up(bdst, biases[i], (size_t)ws[i]->out * 4))) return rc;
                bd[i] = bdst;
                boff += ws[i]->out;
            }
        }
    } else {
        for (int i = 0; i < count; i++) {
            yd[i] = ys[i];
            bd[i] = biases ? biases[i] : nullptr;
        }
    }
    if (quantize_in_launch(ctx, ws[0]->type, in, rows, count,
                           count == 2 && ws[0]->out == ws[1]->out ? ws[0]->out : 0)) {
        // Decode: the Q8_K quantisation happens inside the projection launch.
        if ((rc = launch_projection(ctx, ws, count, bd, yd, rows, ovfq::ActQ{nullptr, nullptr, nullptr}, xd)))
            return rc;
    } else {
        ovfq::ActQ act;
        if ((rc = quantize_into_scratch(ctx, ws[0]->type, xd, rows, in, &act))) return rc;
        if ((rc = launch_projection(ctx, ws, count, bd, yd, rows, act))) return rc;
    }
    if (host) {
        for (int i = 0; i < count; i++)
            if ((rc = io.down(ys[i], yd[i], (size_t)rows * ws[i]->out * 4))) return rc;
        if ((rc = io.finish())) return rc;
    }
    return ok();
}

int ovfq_project(ovfq_ctx* ctx, const ovfq_weight* w, const float* x, int rows, const float* bias, float* y) {
    const float* biases[1] = {bias};
    float* ys[1] = {y};
    return project_impl(ctx, 1, &w, x, rows, biases, ys, true);
}

int ovfq_project_dev(ovfq_ctx* ctx, const ovfq_weight* w, const float* x, int rows, const float* bias,
                     float* y) {
    const float* biases[1] = {bias};
    float* ys[1] = {y};
    return project_impl(ctx, 1, &w, x, rows, biases, ys, false);
}

int ovfq_project_noalloc_dev(ovfq_ctx* ctx, const ovfq_weight* w, const float* x, int rows, const float* bias,
                             float* y) {
    if (!ctx) return fail(OVFQ_ERR_NULL, "ctx is NULL");
    int rc = check_weight(ctx, w);
    if (rc) return rc;
    if (!x || !y) return fail(OVFQ_ERR_NULL, "input or output is NULL");
    if ((rc = check_rows(rows))) return rc;
    if ((rc = check_dev_align(x, "input")) || (rc = check_dev_align(y, "output"))) return rc;
    if ((rc = check_plane(rows, w->out, "output"))) return rc;
    const int in = w->in;
    if ((int64_t)rows * in > ovfq::kNoAllocMaxElems)
        return fail(OVFQ_ERR_SIZE, "rows x inputSize (%lld) above the fixed scratch's %lld elements",
                    (long long)rows * in, (long long)ovfq::kNoAllocMaxElems);
    std::lock_guard<std::mutex> lk(ctx->mu);
    HIP_TRY(hipSetDevice(ctx->device));
    const ovfq_weight* ws[1] = {w};
    const float* bs[1] = {bias};
    float* ys[1] = {y};
    if (quantize_in_launch(ctx, w->type, in, rows, 1)) {
        if ((rc = launch_projection(ctx, ws, 1, bs, ys, rows, ovfq::ActQ{nullptr, nullptr, nullptr}, x))) return rc;
        return ok();
    }
    // The activation's quantised form goes to this device's fixed scratch (resolved when a context was created
    // on it): quants, then scales, then (Q8_K) bsums, each 256-byte aligned. The quantiser writes every byte
    // the projection reads, so nothing is cleared first.
    const bool q80 = w->type == OVFQ_TYPE_Q8_0;
    const size_t n = (size_t)rows * in;
    auto carve = [&](Carver& cv, int8_t** q, float** s, int16_t** b) {
        *q = cv.take<int8_t>(n);
        *s = cv.take<float>(n / (q80 ? OVFQ_Q8_BLOCK : OVFQ_QK) * sizeof(float));
        *b = q80 ? nullptr : cv.take<int16_t>(n / OVFQ_GROUP * sizeof(int16_t));
    };
    int8_t* q;
    float* s;
    int16_t* b;
    Carver sizing{nullptr};
    carve(sizing, &q, &s, &b);
    if (sizing.used > ovfq::kNoAllocScratchBytes)  // cannot happen up to kNoAllocMaxElems; checked all the same
        return fail(OVFQ_ERR_SIZE, "fixed scratch too small (%zu B needed)", sizing.used);
    char* base = static_cast<char*>(ovfq::noalloc_scratch(ctx->device));
    if (!base) return fail(OVFQ_ERR_HIP, "fixed scratch of device %d is not resolved", ctx->device);
    Carver cv{base};
    carve(cv, &q, &s, &b);
    if (q80)
        HIP_TRY(ovfq::launch_quantize_q8_0(x, (int64_t)(n / OVFQ_Q8_BLOCK), q, s, ctx->stream));
    else
        HIP_TRY(ovfq::launch_quantize_q8k(x, (int64_t)(n / OVFQ_QK), q, s, b, ctx->stream));
    if ((rc = launch_projection(ctx, ws, 1, bs, ys, rows, ovfq::ActQ{q, s, b}))) return rc;
    return ok();
}

int ovfq_project_gate_up(ovfq_ctx* ctx, const ovfq_weight* gate, const ovfq_weight* up, const float* x,
                         float* gate_out, float* up_out) {
    if (gate && up && (gate->out != up->out || gate->in != up->in))
        return fail(OVFQ_ERR_SIZE, "gate and up must have the same shape");
    const ovfq_weight* ws[2] = {gate, up};
    float* ys[2] = {gate_out, up_out};
    return project_impl(ctx, 2, ws, x, 1, nullptr, ys, true);
}

int ovfq_project_gate_up_dev(ovfq_ctx* ctx, const ovfq_weight* gate, const ovfq_weight* up, const float* x,
                             float* gate_out, float* up_out) {
    if (gate && up && (gate->out != up->out || gate->in != up->in))
        return fail(OVFQ_ERR_SIZE, "gate and up must have the same shape");
    const ovfq_weight* ws[2] = {gate, up};
    float* ys[2] = {gate_out, up_out};
    return project_impl(ctx, 2, ws, x, 1, nullptr, ys, false);
}

int ovfq_project_multi(ovfq_ctx* ctx, int count, const ovfq_weight* const* weights, const float* x, int rows,
                       const float* const* biases, float* const* ys) {
    return project_impl(ctx, count, weights, x, rows, biases, ys, true);
}

int ovfq_project_multi_dev(ovfq_ctx* ctx, int count, const ovfq_weight* const* weights, const float* x, int rows,
                           const float* const* biases, float* const* ys) {
    return project_impl(ctx, count, weights, x, rows, biases, ys, false);
}

static int prequant_impl(ovfq_ctx* ctx, const ovfq_weight* w, const int8_t* q, const float* s, const int16_t* b,
                         int rows, const float* bias, float* y, bool host) {
    if (!ctx) return fail(OVFQ_ERR_NULL, "ctx is NULL");
    int rc = check_weight(ctx, w);
    if (rc) return rc;
    const bool kq = w->type != OVFQ_TYPE_Q8_0;
    if (!q || !s || (kq && !b) || !y) return fail(OVFQ_ERR_NULL, "activation scratch or output is NULL");
    if ((rc = check_rows(rows))) return rc;
    if ((rc = check_plane(rows, w->in, "activation")) || (rc = check_plane(rows, w->out, "output"))) return rc;
    if (!host) {
        if ((rc = check_dev_align(q, "quants")) || (rc = check_dev_align(s, "scales")) ||
            (rc = check_dev_align(b, "bsums")) || (rc = check_dev_align(y, "output")))
            return rc;
    }
    const size_t n = (size_t)rows * w->in;
    const int blk = kq ? OVFQ_QK : OVFQ_Q8_BLOCK;
    std::lock_guard<std::mutex> lk(ctx->mu);
    HIP_TRY(hipSetDevice(ctx->device));
    ovfq::ActQ act{q, s, b};
    const float* bd = bias;
    float* yd = y;
    HostIO io(ctx);
    if (host) {
        if ((rc = ensure(ctx, ctx->act_q, n))) return rc;
        if ((rc = ensure(ctx, ctx->act_s, n / blk * 4))) return rc;
        if (kq && (rc = ensure(ctx, ctx->act_b, n / 16 * 2))) return rc;
        if ((rc = ensure(ctx, ctx->y_stage, (size_t)rows * w->out * 4))) return rc;
        if (bias && (rc = ensure(ctx, ctx->bias_stage, (size_t)w->out * 4))) return rc;
        if ((rc = io.up(ctx->act_q.p, q, n)) || (rc = io.up(ctx->act_s.p, s, n / blk * 4)) ||
            (kq && (rc = io.up(ctx->act_b.p, b, n / 16 * 2))))
            return rc;
        if (bias) {
            if ((rc = io.up(ctx->bias_stage.p, bias, (size_t)w->out * 4))) return rc;
            bd = (const float*)ctx->bias_stage.p;
        }
        act = ovfq::ActQ{(const int8_t*)ctx->act_q.p, (const float*)ctx->act_s.p,
                         kq ? (const int16_t*)ctx->act_b.p : nullptr};
        yd = (float*)ctx->y_stage.p;
    }
    const ovfq_weight* ws[1] = {w};
    const float* bs[1] = {bd};
    float* ys[1] = {yd};
    if ((rc = launch_projection(ctx, ws, 1, bs, ys, rows, act))) return rc;
    if (host && ((rc = io.down(y, yd, (size_t)rows * w->out * 4)) || (rc = io.finish()))) return rc;
    return ok();
}

int ovfq_project_prequantized(ovfq_ctx* ctx, const ovfq_weight* w, const int8_t* q, const float* s,
                              const int16_t* b, int rows, const float* bias, float* y) {
    return prequant_impl(ctx, w, q, s, b, rows, bias, y, true);
}

int ovfq_project_prequantized_dev(ovfq_ctx* ctx, const ovfq_weight* w, const int8_t* q, const float* s,
                                  const int16_t* b, int rows, const float* bias, float* y) {
    return prequant_impl(ctx, w, q, s, b, rows, bias, y, false);
}

int ovfq_project_multi_prequantized_dev(ovfq_ctx* ctx, int count, const ovfq_weight* const* ws, const int8_t* q,
                                        const float* s, const int16_t* b, int rows, const float* const* biases,
                                        float* const* ys) {
    if (!ctx) return fail(OVFQ_ERR_NULL, "ctx is NULL");
    if (count < 1 || count > ovfq::kMaxJobs) return fail(OVFQ_ERR_RANGE, "count (%d) must be in [1, 4]", count);
    if (!ws || !ys) return fail(OVFQ_ERR_NULL, "weights / outputs array is NULL");
    if (!q || !s || !b) return fail(OVFQ_ERR_NULL, "activation is NULL");
    int rc;
    for (int i = 0; i < count; i++) {
        if ((rc = check_weight(ctx, ws[i]))) return rc;
        if (!ys[i]) return fail(OVFQ_ERR_NULL, "output %d is NULL", i);
        if (ws[i]->type == OVFQ_TYPE_Q8_0) return fail(OVFQ_ERR_TYPE, "Q8_K activations need K-quant weights");
        if (ws[i]->type != ws[0]->type) return fail(OVFQ_ERR_TYPE, "fused weights must share a type");
        if (ws[i]->in != ws[0]->in) return fail(OVFQ_ERR_SIZE, "fused weights must share inputSize");
        if ((rc = check_dev_align(ys[i], "output"))) return rc;
    }
    if ((rc = check_rows(rows))) return rc;
    if ((rc = check_plane(rows, ws[0]->in, "activation"))) return rc;
    for (int i = 0; i < count; i++)
        if ((rc = check_plane(rows, ws[i]->out, "output"))) return rc;
    if ((rc = check_dev_align(q, "quants")) || (rc = check_dev_align(s, "scales")) || (rc = check_dev_align(b, "bsums")))
        return rc;
    std::lock_guard<std::mutex> lk(ctx->mu);
    HIP_TRY(hipSetDevice(ctx->device));
    if ((rc = launch_projection(ctx, ws, count, biases, ys, rows, ovfq::ActQ{q, s, b}))) return rc;
    return ok();
}

// ---------------------------------------------------------------------------------------- per-head Q8_0 Wo

static int heads_impl(ovfq_ctx* ctx, int H, const ovfq_weight* const* wo, const float* x, int rows, const float* bias,
                      float* y, bool host) {
    if (!ctx) return fail(OVFQ_ERR_NULL, "ctx is NULL");
    if (!wo) return fail(OVFQ_ERR_NULL, "head weight array is NULL");
    if (!x || !y) return fail(OVFQ_ERR_NULL, "input or output is NULL");
    if (H < 1 || H > ovfq::kHeadsMax) return fail(OVFQ_ERR_RANGE, "n_heads (%d) must be in [1, %d]", H, ovfq::kHeadsMax);
    int rc;
    for (int h = 0; h < H; h++) {
        if ((rc = check_weight(ctx, wo[h]))) return rc;
        if (wo[h]->type != OVFQ_TYPE_Q8_0) return fail(OVFQ_ERR_TYPE, "head %d: per-head Wo must be Q8_0", h);
        if (wo[h]->in != wo[0]->in || wo[h]->out != wo[0]->out)
            return fail(OVFQ_ERR_SIZE, "head %d: every head's Wo must be [d_model][head_dim] of one shape", h);
    }
    const int hd = wo[0]->in, dm = wo[0]->out, K = H * hd;
    if (hd > ovfq::kHeadsMaxDim) return fail(OVFQ_ERR_SIZE, "head_dim (%d) above %d", hd, ovfq::kHeadsMaxDim);
    if ((rc = check_rows(rows))) return rc;
    if ((rc = check_plane(rows, K, "activation")) || (rc = check_plane(rows, dm, "output"))) return rc;
    if (!host && ((rc = check_dev_align(x, "input")) || (rc = check_dev_align(y, "output")) ||
                  (rc = check_dev_align(bias, "bias"))))
        return rc;
    // Batches from 32 rows: the int8-MFMA kernel streams each head's Wo once per 16-64 activation rows; fewer rows take
    // the decode kernel, one launch per 8 rows. MI355X, Llama-3-8B Wo (32 x 4096x128), graph replay, us, MFMA / per-8
    // launches: 9 rows 36.9 / 19.5, 16 rows 37.6 / 28.7, 32 rows 46.4 / 47.7, 64 rows 64.7 / 89.2, 512 rows 73.3 /
    // 628.8. OVFQ_HEADS_MFMA_MIN_ROWS sets the switch (measurements).
    static const int heads_mfma_min = [] {
        const char* v = getenv("OVFQ_HEADS_MFMA_MIN_ROWS");
        return v && *v ? atoi(v) : 32;
    }();
    bool mfma = rows >= heads_mfma_min && ovfq::q8_0_heads_mfma_supported(H, hd, rows);
    if (ctx->batched_kernel == OVFQ_BATCHED_TILED) mfma = ovfq::q8_0_heads_mfma_supported(H, hd, rows);
    else if (ctx->batched_kernel != OVFQ_BATCHED_AUTO) mfma = false;
    // rows per decode launch: as many as the LDS copy of the activation and the head values allow (up to 8)
    int R = 0;
    for (int r = rows < ovfq::kHeadsMaxRows ? rows : ovfq::kHeadsMaxRows; r >= 1 && !R && !mfma; r--)
        if (ovfq::q8_0_heads_supported(H, hd, r)) R = r;
    if (!R && !mfma) return fail(OVFQ_ERR_SIZE, "n_heads x head_dim (%d) too large for one launch", K);
    std::lock_guard<std::mutex> lk(ctx->mu);
    HIP_TRY(hipSetDevice(ctx->device));
    const float* xd = x;
    const float* bd = bias;
    float* yd = y;
    HostIO io(ctx);
    if (host) {
        if ((rc = ensure(ctx, ctx->x_stage, (size_t)rows * K * 4)) || (rc = ensure(ctx, ctx->y_stage, (size_t)rows * dm * 4)))
            return rc;
        if (bias && (rc = ensure(ctx, ctx->bias_stage, (size_t)dm * 4))) return rc;
        if ((rc = io.up(ctx->x_stage.p, x, (size_t)rows * K * 4))) return rc;
        if (bias && (rc = io.up(ctx->bias_stage.p, bias, (size_t)dm * 4))) return rc;
        xd = (const float*)ctx->x_stage.p;
        bd = bias ? (const float*)ctx->bias_stage.p : nullptr;
        yd = (float*)ctx->y_stage.p;
    }
    const int8_t* wq[ovfq::kHeadsMax];
    const float* ws[ovfq::kHeadsMax];
    for (int h = 0; h < H; h++) {
        wq[h] = static_cast<const int8_t*>(wo[h]->blocks);
        ws[h] = wo[h]->scales;
    }
    ovfq::ActQ act{nullptr, nullptr, nullptr};
    if (mfma) {
        if ((rc = quantize_into_scratch(ctx, OVFQ_TYPE_Q8_0, xd, rows, K, &act))) return rc;
        HIP_TRY(ovfq::launch_q8_0_heads_mfma(wq, ws, H, hd, dm, rows, bd, act, yd, ctx->stream));
        if (host && ((rc = io.down(y, yd, (size_t)rows * dm * 4)) || (rc = io.finish()))) return rc;
        return ok();
    }
    // One launch per R rows; the Q8_0 quantisation of the heads' inputs runs inside it when the rows are short, else
    // once for all rows beforehand.
    const bool inside = ovfq::q8_0_heads_quantize_inside(H, hd, R);
    if (!inside && (rc = quantize_into_scratch(ctx, OVFQ_TYPE_Q8_0, xd, rows, K, &act))) return rc;
    for (int r0 = 0; r0 < rows; r0 += R) {
        const int n = rows - r0 < R ? rows - r0 : R;
        const ovfq::ActQ a = inside ? ovfq::ActQ{nullptr, nullptr, nullptr}
                                    : ovfq::ActQ{act.q + (size_t)r0 * K, act.s + (size_t)r0 * (K / OVFQ_Q8_BLOCK), nullptr};
        HIP_TRY(ovfq::launch_q8_0_heads(wq, ws, H, hd, dm, n, bd, inside ? xd + (size_t)r0 * K : nullptr, a,
                                        yd + (size_t)r0 * dm, ctx->stream));
    }
    if (host && ((rc = io.down(y, yd, (size_t)rows * dm * 4)) || (rc = io.finish()))) return rc;
    return ok();
}

int ovfq_project_heads_q8_0(ovfq_ctx* ctx, int n_heads, const ovfq_weight* const* wo, const float* x, int rows,
                            const float* bias, float* y) {
    return heads_impl(ctx, n_heads, wo, x, rows, bias, y, true);
}

int ovfq_project_heads_q8_0_dev(ovfq_ctx* ctx, int n_heads, const ovfq_weight* const* wo, const float* x, int rows,
                                const float* bias, float* y) {
    return heads_impl(ctx, n_heads, wo, x, rows, bias, y, false);
}

// ---------------------------------------------------------------------------------------- routed MoE

static int topk_impl(ovfq_ctx* ctx, const float* logits, int rows, int n_experts, int top_k, int normalize, int* idx,
                     float* w, bool host) {
    if (!ctx) return fail(OVFQ_ERR_NULL, "ctx is NULL");
    if (!logits || !idx || !w) return fail(OVFQ_ERR_NULL, "logits / expert_indices / expert_weights is NULL");
    if (n_experts < 1) return fail(OVFQ_ERR_SIZE, "Router logits cannot be empty (n_experts = %d)", n_experts);
    if (n_experts > OVFQ_MAX_EXPERTS)
        return fail(OVFQ_ERR_SIZE, "n_experts (%d) above %d", n_experts, OVFQ_MAX_EXPERTS);
    if (top_k < 1) return fail(OVFQ_ERR_RANGE, "top_k (%d) must be positive", top_k);
    if (rows < 1) return fail(OVFQ_ERR_RANGE, "rows (%d) must be positive", rows);
    if (check_plane(rows, n_experts, "logits") || check_plane(rows, top_k, "expert_indices")) return OVFQ_ERR_SIZE;
    if (!host && (rc_align(logits) || rc_align(idx) || rc_align(w)))
        return fail(OVFQ_ERR_SIZE, "device pointers must be 4-byte aligned");
    const int k = top_k < n_experts ? top_k : n_experts;
    std::lock_guard<std::mutex> lk(ctx->mu);
    HIP_TRY(hipSetDevice(ctx->device));
    if (!host) {
        HIP_TRY(ovfq::launch_moe_topk(logits, rows, n_experts, k, top_k, normalize, idx, w, ctx->stream));
        return ok();
    }
    const size_t lb = (size_t)rows * n_experts * 4, ob = (size_t)rows * top_k * 4;
    int rc;
    if ((rc = ensure(ctx, ctx->moe, ((lb + 255) & ~size_t(255)) + 2 * ((ob + 255) & ~size_t(255))))) return rc;
    char* base = static_cast<char*>(ctx->moe.p);
    float* dl = reinterpret_cast<float*>(base);
    int* di = reinterpret_cast<int*>(base + ((lb + 255) & ~size_t(255)));
    float* dw = reinterpret_cast<float*>(base + ((lb + 255) & ~size_t(255)) + ((ob + 255) & ~size_t(255)));
    HostIO io(ctx);
    // slots past min(top_k, n_experts) keep the caller's values
    if ((rc = io.up(dl, logits, lb)) || (rc = io.up(di, idx, ob)) || (rc = io.up(dw, w, ob))) return rc;
    HIP_TRY(ovfq::launch_moe_topk(dl, rows, n_experts, k, top_k, normalize, di, dw, ctx->stream));
    if ((rc = io.down(idx, di, ob)) || (rc = io.down(w, dw, ob)) || (rc = io.finish())) return rc;
    return ok();
}

int ovfq_moe_select_topk(ovfq_ctx* ctx, const float* logits, int rows, int n_experts, int top_k, int normalize,
                         int* expert_indices, float* expert_weights) {
    return topk_impl(ctx, logits, rows, n_experts, top_k, normalize, expert_indices, expert_weights, true);
}

int ovfq_moe_select_topk_dev(ovfq_ctx* ctx, const float* logits, int rows, int n_experts, int top_k, int normalize,
                             int* expert_indices, float* expert_weights) {
    return topk_impl(ctx, logits, rows, n_experts, top_k, normalize, expert_indices, expert_weights, false);
}

// With `logits` (router logits [rows][E]) the routing is computed here (MoeRouter.SelectTopK) and written to idx / w
// ([rows][k], outputs); without, idx / w are the caller's routing (inputs).
static int moe_impl(ovfq_ctx* ctx, int E, const ovfq_weight* const* gate, const ovfq_weight* const* up,
                    const ovfq_weight* const* down, const float* x, int rows, int k, const int* idx, const float* w,
                    float* y, bool host, const float* logits = nullptr, int normalize = 0) {
    if (!ctx) return fail(OVFQ_ERR_NULL, "ctx is NULL");
    if (!gate || !up || !down) return fail(OVFQ_ERR_NULL, "expert weight arrays are NULL");
    if (!x || !idx || !w || !y) return fail(OVFQ_ERR_NULL, "x / expert_indices / expert_weights / y is NULL");
    const bool route = logits != nullptr;
    if (E < 1 || E > OVFQ_MAX_EXPERTS) return fail(OVFQ_ERR_RANGE, "n_experts (%d) must be in [1, %d]", E, OVFQ_MAX_EXPERTS);
    int rc;
    if ((rc = check_rows(rows))) return rc;
    if (k < 1 || k > E) return fail(OVFQ_ERR_RANGE, "top_k (%d) must be in [1, n_experts]", k);
    for (int e = 0; e < E; e++) {
        if (!gate[e] || !up[e] || !down[e]) return fail(OVFQ_ERR_NULL, "expert %d has a NULL weight", e);
        if ((rc = check_weight(ctx, gate[e])) || (rc = check_weight(ctx, up[e])) || (rc = check_weight(ctx, down[e])))
            return rc;
    }
    const int gt = gate[0]->type, dt = down[0]->type;
    const int dmodel = gate[0]->in, dff = gate[0]->out;
    for (int e = 0; e < E; e++) {
        if (gate[e]->type == OVFQ_TYPE_Q8_0 || down[e]->type == OVFQ_TYPE_Q8_0)
            return fail(OVFQ_ERR_TYPE, "expert weights must be Q4_K or Q6_K");
        if (gate[e]->type != gt || up[e]->type != gt || down[e]->type != dt)
            return fail(OVFQ_ERR_TYPE, "gate/up experts must share one type and down experts another");
        if (gate[e]->in != dmodel || up[e]->in != dmodel || gate[e]->out != dff || up[e]->out != dff ||
            down[e]->in != dff || down[e]->out != dmodel)
            return fail(OVFQ_ERR_SIZE, "expert %d shapes differ (gate/up [d_ff][d_model], down [d_model][d_ff])", e);
    }
    if (!host && (rc_align(x) || rc_align(idx) || rc_align(w) || rc_align(y) || (route && rc_align(logits))))
        return fail(OVFQ_ERR_SIZE, "device pointers must be 4-byte aligned");
    // token rows and (token, slot) pair rows of the activation, gate/up and expert-output planes
    if ((rc = check_plane(rows, dmodel, "activation")) || (rc = check_plane((int64_t)rows * k, dff, "gate/up output")) ||
        (rc = check_plane((int64_t)rows * k, dmodel, "expert output")) ||
        (route && (rc = check_plane(rows, E, "router logits"))))
        return rc;
    const size_t P = (size_t)rows * k;
    std::lock_guard<std::mutex> lk(ctx->mu);
    HIP_TRY(hipSetDevice(ctx->device));
    // scratch layout (sizes first, then the pointers into one buffer)
    // Many pairs per expert: the batched int8-MFMA kernel over expert groups (64-row tiles, operand build amortised
    // over the tile); few: the small-M kernel (16-row tiles, super-block-parallel waves). Measured on MI355X with 8
    // Mixtral-shaped experts, top-2: small-M wins at 8 pairs per expert on average (304 vs 352 us), the grouped
    // kernel from 12 (354 vs 365 us; 64 tokens 362 vs 469 us).
    static const int grouped_min = [] {
        const char* v = getenv("OVFQ_MOE_GROUPED_MIN_PAIRS");
        return v && *v ? atoi(v) : 12;
    }();
    // the small-M kernel keeps a row's block values in LDS (d_model, d_ff <= 16384); past that, always grouped
    const bool small_ok = ovfq::mfma_small_supported(gt, dmodel) && ovfq::mfma_small_supported(dt, dff);
    const bool grouped_big = !small_ok || ctx->batched_kernel == OVFQ_BATCHED_TILED ||
                             (ctx->batched_kernel == OVFQ_BATCHED_AUTO && P >= (size_t)grouped_min * E);
    const int max_tiles = (int)((P + ovfq::kGroupedTileRows - 1) / ovfq::kGroupedTileRows) + E;
    auto carve = [&](Carver& c, int** off, int** prow, int** pof, float** pw, float** g, float** u, int8_t** iq,
                     float** is, int16_t** ib, float** out, float** hx, int** hidx, float** hw, float** hy,
                     float** hl) {
        *off = c.take<int>((size_t)(E + 2 + max_tiles) * 4);  // expert_off[E + 1], tile count, tile list
        *prow = c.take<int>(P * 4);
        *pof = c.take<int>(P * 4);
        *pw = c.take<float>(P * 4);
        *g = c.take<float>(P * dff * 4);
        *u = c.take<float>(P * dff * 4);
        *iq = c.take<int8_t>(P * dff);
        *is = c.take<float>(P * (dff / OVFQ_QK) * 4);
        *ib = c.take<int16_t>(P * (dff / 16) * 2);
        *out = c.take<float>(P * dmodel * 4);
        if (host) {
            *hx = c.take<float>((size_t)rows * dmodel * 4);
            *hidx = c.take<int>(P * 4);
            *hw = c.take<float>(P * 4);
            *hy = c.take<float>((size_t)rows * dmodel * 4);
            if (route) *hl = c.take<float>((size_t)rows * E * 4);
        }
    };
    int *off, *prow, *pof, *hidx = nullptr;
    float *pw, *g, *u, *is, *out, *hx = nullptr, *hw = nullptr, *hy = nullptr, *hl = nullptr;
    int8_t* iq;
    int16_t* ib;
    Carver sizing{nullptr};
    carve(sizing, &off, &prow, &pof, &pw, &g, &u, &iq, &is, &ib, &out, &hx, &hidx, &hw, &hy, &hl);
    if ((rc = ensure(ctx, ctx->moe, sizing.used))) return rc;
    Carver c{static_cast<char*>(ctx->moe.p)};
    carve(c, &off, &prow, &pof, &pw, &g, &u, &iq, &is, &ib, &out, &hx, &hidx, &hw, &hy, &hl);
    const float* xd = x;
    const float* ld = logits;
    int* idxd = const_cast<int*>(idx);  // written only when routing here (then the caller's output)
    float* wd = const_cast<float*>(w);
    float* yd = y;
    HostIO io(ctx);
    if (host) {
        if ((rc = io.up(hx, x, (size_t)rows * dmodel * 4))) return rc;
        if (route) {
            if ((rc = io.up(hl, logits, (size_t)rows * E * 4))) return rc;
            ld = hl;
        } else {
            if ((rc = io.up(hidx, idx, P * 4)) || (rc = io.up(hw, w, P * 4))) return rc;
        }
        xd = hx;
        idxd = hidx;
        wd = hw;
        yd = hy;
    }
    // the grouping plan and the Q8_K quantisation of x share one launch (neither depends on the other)
    const size_t n_x = (size_t)rows * dmodel;
    if ((rc = ensure(ctx, ctx->act_q, n_x)) || (rc = ensure(ctx, ctx->act_s, n_x / OVFQ_QK * sizeof(float))) ||
        (rc = ensure(ctx, ctx->act_b, n_x / 16 * sizeof(int16_t))))
        return rc;
    const ovfq::ActQ act{(const int8_t*)ctx->act_q.p, (const float*)ctx->act_s.p, (const int16_t*)ctx->act_b.p};
    int* tile_count = off + E + 1;
    int* tiles = off + E + 2;
    if (route)
        HIP_TRY(ovfq::launch_moe_route_plan(ld, rows, k, E, normalize, idxd, wd, off, prow, pof,
                                            ovfq::kGroupedTileRows, grouped_big ? tiles : nullptr, tile_count, xd,
                                            (int64_t)(n_x / OVFQ_QK), (int8_t*)ctx->act_q.p, (float*)ctx->act_s.p,
                                            (int16_t*)ctx->act_b.p, ctx->stream));
    else
        HIP_TRY(ovfq::launch_moe_plan(idxd, rows, k, E, off, prow, pof, ovfq::kGroupedTileRows,
                                      grouped_big ? tiles : nullptr, tile_count, xd, (int64_t)(n_x / OVFQ_QK),
                                      (int8_t*)ctx->act_q.p, (float*)ctx->act_s.p, (int16_t*)ctx->act_b.p,
                                      ctx->stream));
    const uint8_t* gw[OVFQ_MAX_EXPERTS];
    const uint8_t* uw[OVFQ_MAX_EXPERTS];
    const uint8_t* dw[OVFQ_MAX_EXPERTS];
    for (int e = 0; e < E; e++) {
        gw[e] = static_cast<const uint8_t*>(gate[e]->blocks);
        uw[e] = static_cast<const uint8_t*>(up[e]->blocks);
        dw[e] = static_cast<const uint8_t*>(down[e]->blocks);
    }
    ovfq::GroupLaunch L{};
    L.w0 = gw;
    L.w1 = uw;
    L.y0 = g;
    L.y1 = u;
    L.n_rows = dff;
    L.in = dmodel;
    L.experts = E;
    L.rows = rows;
    L.expert_off = off;
    L.pair_row = prow;
    L.act = act;
    L.pairs = (int)P;
    if (grouped_big)
        HIP_TRY(ovfq::launch_mfma_grouped(gt, L, tiles, tile_count, max_tiles, ctx->stream));
    else
        HIP_TRY(ovfq::launch_mfma_small(gt, L, ctx->stream));
    ovfq::GroupLaunch D{};
    D.w0 = dw;
    D.y0 = out;
    D.n_rows = dmodel;
    D.in = dff;
    D.experts = E;
    D.rows = (int)P;
    D.expert_off = off;
    D.pair_row = nullptr;  // the intermediate is already pair-major
    D.act = ovfq::ActQ{iq, is, ib};
    D.pairs = (int)P;
    // With top-1 / top-2 and the down projection on the small-M path (the expert-stream or small-M kernel), the
    // combine is folded into it: each token output gets at most two float-atomic adds onto zero, whose sum does not
    // depend on their order, so it is the combine kernel's (0 + w0 o0) + w1 o1 exactly. The zeroing and the per-pair
    // weights go in the gate * up launch.
    // Float atomics on the output need ordinary device memory: a _dev caller's y that is host-mapped (or not known to
    // HIP) keeps the separate combine launch. The host entry points write into the context's own device staging.
    bool y_device = host;
    if (!host) {
        hipPointerAttribute_t attr{};
        if (hipPointerGetAttributes(&attr, y) == hipSuccess)
            y_device = attr.type == hipMemoryTypeDevice;
        else
            (void)hipGetLastError();  // an unregistered host pointer: clear the sticky error
    }
    ovfq::MoeFold fold{};
    if (k <= 2 && !grouped_big && y_device) {
        fold = ovfq::MoeFold{yd, (int64_t)rows * dmodel, pof, wd, (int)P, pw};
        D.comb = yd;
        D.comb_tok = prow;
        D.comb_w = pw;
    }
    HIP_TRY(ovfq::launch_gate_up_q8k(g, u, off, E, (int)P, dff, false, iq, is, ib, ctx->stream, fold));
    if (grouped_big)
        HIP_TRY(ovfq::launch_mfma_grouped(dt, D, tiles, tile_count, max_tiles, ctx->stream));
    else
        HIP_TRY(ovfq::launch_mfma_small(dt, D, ctx->stream));
    if (!D.comb) HIP_TRY(ovfq::launch_moe_combine(out, pof, wd, rows, k, dmodel, yd, ctx->stream));
    if (host) {
        if ((rc = io.down(y, yd, (size_t)rows * dmodel * 4))) return rc;
        if (route && ((rc = io.down(const_cast<int*>(idx), idxd, P * 4)) ||
                      (rc = io.down(const_cast<float*>(w), wd, P * 4))))
            return rc;
        if ((rc = io.finish())) return rc;
    }
    return ok();
}

// ---------------------------------------------------------------------------------------- gated FFN

static int ffn_impl(ovfq_ctx* ctx, const ovfq_weight* gate, const ovfq_weight* up, const ovfq_weight* down,
                    const float* x, int rows, int activation, float* y, bool host) {
    if (!ctx) return fail(OVFQ_ERR_NULL, "ctx is NULL");
    if (activation != OVFQ_FFN_SWIGLU && activation != OVFQ_FFN_GEGLU)
        return fail(OVFQ_ERR_RANGE, "activation %d is neither OVFQ_FFN_SWIGLU (3) nor OVFQ_FFN_GEGLU (4)", activation);
    if (!gate || !up || !down) return fail(OVFQ_ERR_NULL, "gate / up / down is NULL");
    if (!x || !y) return fail(OVFQ_ERR_NULL, "x / y is NULL");
    int rc;
    if ((rc = check_weight(ctx, gate)) || (rc = check_weight(ctx, up)) || (rc = check_weight(ctx, down))) return rc;
    if ((rc = check_rows(rows))) return rc;
    if (gate->type == OVFQ_TYPE_Q8_0 || down->type == OVFQ_TYPE_Q8_0)
        return fail(OVFQ_ERR_TYPE, "the fused FFN takes Q4_K / Q6_K weights");
    if (up->type != gate->type) return fail(OVFQ_ERR_TYPE, "gate and up must share a type");
    const int dmodel = gate->in, dff = gate->out;
    if (up->in != dmodel || up->out != dff || down->in != dff || down->out != dmodel)
        return fail(OVFQ_ERR_SIZE, "shapes must be gate/up [d_ff][d_model] and down [d_model][d_ff]");
    if (!host && (rc_align(x) || rc_align(y))) return fail(OVFQ_ERR_SIZE, "device pointers must be 4-byte aligned");
    if ((rc = check_plane(rows, dmodel, "activation")) || (rc = check_plane(rows, dff, "gate/up output"))) return rc;
    std::lock_guard<std::mutex> lk(ctx->mu);
    HIP_TRY(hipSetDevice(ctx->device));
    const size_t R = (size_t)rows;
    auto carve = [&](Carver& c, float** g, float** u, int8_t** iq, float** is, int16_t** ib, float** hx, float** hy) {
        *g = c.take<float>(R * dff * 4);
        *u = c.take<float>(R * dff * 4);
        *iq = c.take<int8_t>(R * dff);
        *is = c.take<float>(R * (dff / OVFQ_QK) * 4);
        *ib = c.take<int16_t>(R * (dff / 16) * 2);
        if (host) {
            *hx = c.take<float>(R * dmodel * 4);
            *hy = c.take<float>(R * dmodel * 4);
        }
    };
    float *g, *u, *is, *hx = nullptr, *hy = nullptr;
    int8_t* iq;
    int16_t* ib;
    Carver sizing{nullptr};
    carve(sizing, &g, &u, &iq, &is, &ib, &hx, &hy);
    if ((rc = ensure(ctx, ctx->moe, sizing.used))) return rc;
    Carver c{static_cast<char*>(ctx->moe.p)};
    carve(c, &g, &u, &iq, &is, &ib, &hx, &hy);
    const float* xd = x;
    float* yd = y;
    HostIO io(ctx);
    if (host) {
        if ((rc = io.up(hx, x, R * dmodel * 4))) return rc;
        xd = hx;
        yd = hy;
    }
    // gate/up (one launch; for one or a few short rows the Q8_K quantisation runs inside it)
    const ovfq_weight* gu[2] = {gate, up};
    float* gu_out[2] = {g, u};
    if (quantize_in_launch(ctx, gate->type, dmodel, rows, 2, gate->out == up->out ? gate->out : 0)) {
        if ((rc = launch_projection(ctx, gu, 2, nullptr, gu_out, rows, ovfq::ActQ{nullptr, nullptr, nullptr}, xd)))
            return rc;
    } else {
        ovfq::ActQ act;
        if ((rc = quantize_into_scratch(ctx, gate->type, xd, rows, dmodel, &act))) return rc;
        if ((rc = launch_projection(ctx, gu, 2, nullptr, gu_out, rows, act))) return rc;
    }
    // act(gate) * up, quantised to Q8_K for the down projection
    HIP_TRY(ovfq::launch_gate_up_q8k(g, u, nullptr, 0, rows, dff, activation == OVFQ_FFN_GEGLU, iq, is, ib,
                                     ctx->stream));
    const ovfq_weight* dw[1] = {down};
    float* dy[1] = {yd};
    if ((rc = launch_projection(ctx, dw, 1, nullptr, dy, rows, ovfq::ActQ{iq, is, ib}))) return rc;
    if (host && ((rc = io.down(y, yd, R * dmodel * 4)) || (rc = io.finish()))) return rc;
    return ok();
}

int ovfq_ffn_swiglu(ovfq_ctx* ctx, const ovfq_weight* gate, const ovfq_weight* up, const ovfq_weight* down,
                    const float* x, int rows, float* y) {
    return ffn_impl(ctx, gate, up, down, x, rows, OVFQ_FFN_SWIGLU, y, true);
}

int ovfq_ffn_swiglu_dev(ovfq_ctx* ctx, const ovfq_weight* gate, const ovfq_weight* up, const ovfq_weight* down,
                        const float* x, int rows, float* y) {
    return ffn_impl(ctx, gate, up, down, x, rows, OVFQ_FFN_SWIGLU, y, false);
}

int ovfq_ffn_gated(ovfq_ctx* ctx, const ovfq_weight* gate, const ovfq_weight* up, const ovfq_weight* down,
                   const float* x, int rows, int activation, float* y) {
    return ffn_impl(ctx, gate, up, down, x, rows, activation, y, true);
}

int ovfq_ffn_gated_dev(ovfq_ctx* ctx, const ovfq_weight* gate, const ovfq_weight* up, const ovfq_weight* down,
                       const float* x, int rows, int activation, float* y) {
    return ffn_impl(ctx, gate, up, down, x, rows, activation, y, false);
}

int ovfq_moe_ffn(ovfq_ctx* ctx, int n_experts, const ovfq_weight* const* gate, const ovfq_weight* const* up,
                 const ovfq_weight* const* down, const float* x, int rows, int top_k, const int* expert_indices,
                 const float* expert_weights, float* y) {
    return moe_impl(ctx, n_experts, gate, up, down, x, rows, top_k, expert_indices, expert_weights, y, true);
}

int ovfq_moe_ffn_dev(ovfq_ctx* ctx, int n_experts, const ovfq_weight* const* gate, const ovfq_weight* const* up,
                     const ovfq_weight* const* down, const float* x, int rows, int top_k, const int* expert_indices,
                     const float* expert_weights, float* y) {
    return moe_impl(ctx, n_experts, gate, up, down, x, rows, top_k, expert_indices, expert_weights, y, false);
}

int ovfq_moe_ffn_routed(ovfq_ctx* ctx, int n_experts, const ovfq_weight* const* gate, const ovfq_weight* const* up,
                        const ovfq_weight* const* down, const float* x, int rows, const float* router_logits,
                        int top_k, int normalize, int* expert_indices, float* expert_weights, float* y) {
    if (!router_logits) return fail(OVFQ_ERR_NULL, "router_logits is NULL");
    return moe_impl(ctx, n_experts, gate, up, down, x, rows, top_k, expert_indices, expert_weights, y, true,
                    router_logits, normalize);
}

int ovfq_moe_ffn_routed_dev(ovfq_ctx* ctx, int n_experts, const ovfq_weight* const* gate,
                            const ovfq_weight* const* up, const ovfq_weight* const* down, const float* x, int rows,
                            const float* router_logits, int top_k, int normalize, int* expert_indices,
                            float* expert_weights, float* y) {
    if (!router_logits) return fail(OVFQ_ERR_NULL, "router_logits is NULL");
    return moe_impl(ctx, n_experts, gate, up, down, x, rows, top_k, expert_indices, expert_weights, y, false,
                    router_logits, normalize);
}

// ---------------------------------------------------------------------------------------- weight encoders

static int encode_impl(ovfq_ctx* ctx, int type, const float* w, int in, int out, void* dst, float* scales) {
    if (!ctx) return fail(OVFQ_ERR_NULL, "ctx is NULL");
    if (!w || !dst || (type == OVFQ_TYPE_Q8_0 && !scales)) return fail(OVFQ_ERR_NULL, "source or destination is NULL");
    int rc = check_weight_shape(type, in, out);
    if (rc) return rc;
    if ((rc = check_dev_align(w, "weights")) || (rc = check_dev_align(dst, "dst"))) return rc;
    std::lock_guard<std::mutex> lk(ctx->mu);
    HIP_TRY(hipSetDevice(ctx->device));
    const int64_t n = (int64_t)in * out;
    if (type == OVFQ_TYPE_Q4_K) {
        HIP_TRY(ovfq::launch_encode_q4k(w, n / OVFQ_QK, (uint8_t*)dst, ctx->stream));
    } else if (type == OVFQ_TYPE_Q6_K) {
        HIP_TRY(ovfq::launch_encode_q6k(w, n / OVFQ_QK, (uint8_t*)dst, ctx->stream));
    } else {
        HIP_TRY(ovfq::launch_quantize_q8_0(w, n / OVFQ_Q8_BLOCK, (int8_t*)dst, scales, ctx->stream));
    }
    return ok();
}

int ovfq_quantize_weight_q4k_dev(ovfq_ctx* ctx, const float* w, int in, int out, uint8_t* dst) {
    return encode_impl(ctx, OVFQ_TYPE_Q4_K, w, in, out, dst, nullptr);
}
int ovfq_quantize_weight_q6k_dev(ovfq_ctx* ctx, const float* w, int in, int out, uint8_t* dst) {
    return encode_impl(ctx, OVFQ_TYPE_Q6_K, w, in, out, dst, nullptr);
}
int ovfq_quantize_weight_q8_0_dev(ovfq_ctx* ctx, const float* w, int in, int out, int8_t* q, float* s) {
    return encode_impl(ctx, OVFQ_TYPE_Q8_0, w, in, out, q, s);
}

}  // extern "C"
