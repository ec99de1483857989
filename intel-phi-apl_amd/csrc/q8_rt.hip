/* q8_rt.hip: the C-ABI of include/q8_rt.h over HIP: the GPU context behind struct rt, weight
 * upload, the queue of a round, and the host-pointer and device-pointer products.
 *
 * The reference's products ran on the card's team out of the card's memory (src/card/rt.c:
 * 205-285); here the weights are HBM-resident handles and a round is: every distinct x into
 * one pinned staging buffer, one copy kernel to HBM, one launch per product on the runtime's
 * stream storing its y into pinned host memory, one wait on a completion flag. */
#include <hip/hip_runtime.h>

#include <errno.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include <chrono>
#include <unordered_map>
#include <vector>

#include "../../include/q8_rt.h"
#include "q8_device.h"
#include "q8_wait.h"

#define HIPCHECK(call)                                                                                                 \
    do {                                                                                                               \
        hipError_t e_ = (call);                                                                                        \
        if (e_ != hipSuccess) {                                                                                        \
            fprintf(stderr, "q8_rt: %s failed: %s (%s:%d)\n", #call, hipGetErrorString(e_), __FILE__, __LINE__);       \
            abort();                                                                                                   \
        }                                                                                                              \
    } while (0)

/* Q8_ABORT_EXIT=n (1..125), read by rt_init: a caller's mistake ends the process with _exit(n)
 * instead of abort(), for test harnesses that check the message of an expected failure in a child
 * process without a SIGABRT. */
static int abort_exit = 0;

/* A caller's mistake (a bad shape, an unregistered handle, a misaligned address): the reason on
 * stderr, then abort(), as the reference's entry points fail, before anything is launched. */
[[noreturn]] static void failv(const char *fn, const char *fmt, va_list ap)
{
    fprintf(stderr, "q8_rt: %s: ", fn);
    vfprintf(stderr, fmt, ap);
    fputc('\n', stderr);
    fflush(stderr);
    if (abort_exit >= 1 && abort_exit <= 125)
        _exit(abort_exit);
    abort();
}

[[noreturn]] __attribute__((format(printf, 2, 3))) static void failf(const char *fn, const char *fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    failv(fn, fmt, ap);
}

[[noreturn]] static void fail(const char *fn, const char *why) { failf(fn, "%s", why); }

/* The device scratch of rt_gemm_dev_noalloc: the matrix-core product's K-split partials, at most
 * Q8_GEMM_PART_MAX floats (32 MiB), in a static array of every GPU the library runs on, so that the
 * product allocates nothing. Host code never names it: rt_init asks for its address on the device
 * (hipGetSymbolAddress) and keeps that in the runtime. */
static __device__ __align__(256) float scratch[Q8_GEMM_PART_MAX];

namespace {

/* a registered weight handle: its shape, and whether the library allocated it (rt_q8_upload and
 * the like) or only registered a caller's buffer (rt_q8_repack_dev) */
struct matrix {
    long rows, cols;
    bool owned;
};

struct ktrec {
    int kind;
    long rows, cols, t, grid;
    char name[64];
};

struct job {
    const void *w;
    long rows, cols, t;
    const float *x;
    float *y;
    size_t x_off, y_off; /* floats, in the staging buffers */
};

struct ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    /* the settings, from the environment at rt_init or from their setters; nothing reads the
     * environment on a product call */
    int exact = 0;          /* Q8_EXACT, rt_set_exact */
    int epi_apart = 0;      /* rt_set_epi_apart */
    double wait_s = Q8_WAIT_DEFAULT_S; /* Q8_WAIT_S: every host wait's deadline */
    size_t upload_chunk = (size_t)64 << 20; /* Q8_UPLOAD_CHUNK, rt_set_upload_chunk */
    q8_gemm_opts gemm_opts = {0, 0};        /* rt_gemm_force */
    int x_direct = 1;       /* rt_set_x_direct */
    /* staging for the host-pointer products, in floats: pinned x and y, x's copy in HBM */
    float *hx = nullptr, *hy = nullptr, *dx = nullptr;
    size_t x_cap = 0, y_cap = 0;
    /* the completion flag of the host-pointer calls (pinned) and the last number set in it */
    unsigned *flag = nullptr;
    unsigned flag_seq = 0;
    /* scratch for the fused pair when it runs as two products (exact mode, t >= 5): G and U */
    float *scratch = nullptr;
    size_t scratch_cap = 0;
    /* the epilogues run apart: the normed x, or the product before the residual is added */
    float *epi = nullptr;
    size_t epi_cap = 0;
    /* the matrix-core product's K-split partials */
    float *part = nullptr;
    /* a matrix-core round's partials, every product's */
    float *rpart = nullptr;
    size_t rpart_cap = 0;
    /* the device address of `scratch` on this runtime's GPU (rt_gemm_dev_noalloc's partials) */
    float *noalloc_part = nullptr;
    /* the greedy next token's candidates */
    void *amax = nullptr;
    size_t amax_cap = 0;
    /* buffers replaced by larger ones: a recorded graph may still use them, so they live
     * until rt_fini */
    std::vector<void *> retired;
    std::unordered_map<const void *, matrix> weights;
    job queue[RT_BATCH];
    int queued = 0;
    /* weight upload staging: two pinned host chunks and two device chunks of whole 16-row groups,
     * an event per chunk slot (the slot's copy and repack are done); allocated on the first upload */
    uint8_t *up_host[2] = {nullptr, nullptr}, *up_dev[2] = {nullptr, nullptr};
    hipEvent_t up_done[2] = {nullptr, nullptr};
    size_t up_cap = 0;
    /* the host-pointer calls' phases (rt_host_timing): microseconds summed over the calls */
    int htime_on = 0;
    double ht[RT_HT_PHASES] = {};
    double ht_t2 = 0.0; /* the current call's end of launching: wait_done sets it */
    long hcalls = 0;
    /* kernel timing (rt_ktime): one event pair per recorded product */
    int ktime_on = 0;
    std::vector<hipEvent_t> kt_events;
    std::vector<ktrec> kt;
};

constexpr size_t KT_MAX = 16384;

/* The runtimes alive, in the order rt_init set them up; rt_q8_row takes no struct rt
 * (src/card/rt.h:85) and uses the last of them. */
std::vector<ctx *> live;
ctx *current = nullptr;

/* the host's clock, for the host-pointer calls' phases */
double now_us()
{
    return std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

ctx *get(struct rt *R, const char *fn)
{
    if (!R || !R->chain)
        fail(fn, "rt_init has not run on this struct rt");
    return (ctx *)R->chain;
}

/* w must be a handle the registry holds (from an upload, or a buffer rt_q8_repack_dev wrote), used
 * as its own shape or a prefix of its whole 16-row groups: anything else (a host pointer left by an
 * engine still on its own repack, an address inside a matrix, a freed handle) aborts here, before
 * a kernel could read it */
void check_shape(ctx *c, const char *fn, const void *w, long rows, long cols)
{
    if (!w)
        fail(fn, "w is NULL");
    if (rows <= 0 || cols <= 0 || rows % Q8_GROUP || cols % Q8_BLOCK)
        failf(fn, "rows %ld must be a positive multiple of 16 and cols %ld of 32", rows, cols);
    auto it = c->weights.find(w);
    if (it == c->weights.end())
        failf(fn, "w %p is not a weight handle (rt_q8_upload, rt_q8_upload_fd, rt_q8_upload_packed, rt_gguf_upload or rt_q8_repack_dev make them)", w);
    if (it->second.cols != cols || rows > it->second.rows)
        failf(fn, "w was uploaded as %ld x %ld, used as %ld x %ld (only a prefix of whole 16-row groups may be used)", it->second.rows, it->second.cols,
              rows, cols);
}

void check_dev_ptr(const char *fn, const void *p, const char *what)
{
    if (!p || ((uintptr_t)p & 15))
        failf(fn, "%s must be a 16-byte aligned device address", what);
}

/* Waits, each bounded by the runtime's deadline (q8_wait_until): the stream idle, an event done.
 * A HIP error seen while polling (a kernel that failed) stops the process with the call's name. */
void sync_stream(ctx *c, const char *what)
{
    q8_wait_until(
        [&] {
            const hipError_t e = hipStreamQuery(c->stream);
            if (e == hipErrorNotReady)
                return false;
            if (e != hipSuccess) {
                fprintf(stderr, "q8_rt: %s: the stream reports %s\n", what, hipGetErrorString(e));
                abort();
            }
            return true;
        },
        c->wait_s, what);
}

void sync_event(ctx *c, hipEvent_t ev, const char *what)
{
    q8_wait_until(
        [&] {
            const hipError_t e = hipEventQuery(ev);
            if (e == hipErrorNotReady)
                return false;
            if (e != hipSuccess) {
                fprintf(stderr, "q8_rt: %s: the event reports %s\n", what, hipGetErrorString(e));
                abort();
            }
            return true;
        },
        c->wait_s, what);
}

/* *p = a pinned host buffer of n floats (the old one freed: no call is in flight when it grows) */
void grow_pinned(float **p, size_t n)
{
    if (*p)
        HIPCHECK(hipHostFree(*p));
    HIPCHECK(hipHostMalloc((void **)p, n * sizeof(float), hipHostMallocDefault));
}

void reserve_staging(ctx *c, size_t nx, size_t ny)
{
    if (nx > c->x_cap) {
        size_t n = nx + nx / 2 + 4096;
        grow_pinned(&c->hx, n);
        if (c->dx)
            HIPCHECK(hipFree(c->dx));
        HIPCHECK(hipMalloc((void **)&c->dx, n * sizeof(float)));
        c->x_cap = n;
    }
    if (ny > c->y_cap) {
        size_t n = ny + ny / 2 + 4096;
        grow_pinned(&c->hy, n);
        c->y_cap = n;
    }
}

/* Workspace is allocated on demand, never while the stream is being recorded into a graph:
 * a product of a new, larger size must run once before a graph records it. */
void no_capture(ctx *c, const char *what)
{
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    HIPCHECK(hipStreamIsCapturing(c->stream, &st));
    if (st != hipStreamCaptureStatusNone)
        failf(what, "must grow while a graph is being recorded: run a product of this size once before rt_graph_begin");
}

float *reserve_scratch(ctx *c, size_t n)
{
    if (n > c->scratch_cap) {
        no_capture(c, "the fused pair's scratch");
        if (c->scratch)
            c->retired.push_back(c->scratch);
        HIPCHECK(hipMalloc((void **)&c->scratch, n * sizeof(float)));
        c->scratch_cap = n;
    }
    return c->scratch;
}

float *reserve_epi(ctx *c, size_t n)
{
    if (n > c->epi_cap) {
        no_capture(c, "the epilogue's workspace");
        if (c->epi)
            c->retired.push_back(c->epi);
        HIPCHECK(hipMalloc((void **)&c->epi, n * sizeof(float)));
        c->epi_cap = n;
    }
    return c->epi;
}

/* the matrix-core rounds' workspace, at least need floats (grown outside graph capture) */
float *reserve_rpart(ctx *c, size_t need)
{
    if (need > c->rpart_cap) {
        no_capture(c, "a matrix-core round's partial sums");
        if (c->rpart)
            c->retired.push_back(c->rpart);
        HIPCHECK(hipMalloc((void **)&c->rpart, need * sizeof(float)));
        c->rpart_cap = need;
    }
    return c->rpart;
}

void reserve_gemm(ctx *c, long rows, long cols, long t)
{
    if (!c->part && q8_gemm_part_floats(rows, cols, t, c->gemm_opts) > 0) {
        no_capture(c, "the matrix-core product's partial sums");
        HIPCHECK(hipMalloc((void **)&c->part, (size_t)Q8_GEMM_PART_MAX * sizeof(float)));
    }
    if (q8_gemm_part_floats(rows, cols, t, c->gemm_opts) > Q8_GEMM_PART_MAX)
        fail("the matrix-core product", "its K-split partials exceed the workspace (a planning error)");
}

/* Whether a product of t tokens runs on the matrix cores (every 64-token launch of it, the last
 * one too, however few tokens it holds, so that a token's bits do not depend on t), else on the
 * decode kernels, which take at most 4 tokens a launch. */
bool on_matrix_cores(long t) { return t >= 5; }

/* Y = X W^T for t >= 5 tokens on the matrix cores, 64 at a time; res != NULL: Y = res + X W^T (res
 * may be Y), added in the matrix-core product's store or partial sum. part != NULL: the K-split
 * partials go there (at most Q8_GEMM_PART_MAX floats) instead of the runtime's workspace, and
 * nothing is allocated. */
void gemm_tokens(ctx *c, const void *w, long rows, long cols, const float *x, long xs, long t, float *y, const float *res = nullptr,
                 float *part = nullptr)
{
    const q8_stream_t s = (q8_stream_t)c->stream;
    for (long k = 0; k < t; k += 64) {
        const long n = t - k < 64 ? t - k : 64;
        if (part) {
            if (q8_gemm_part_floats(rows, cols, n, c->gemm_opts) > Q8_GEMM_PART_MAX)
                failf("rt_gemm_dev_noalloc", "the K-split partials of %ld x %ld at %ld tokens exceed the %ld-float scratch", rows, cols, n,
                      (long)Q8_GEMM_PART_MAX);
        } else {
            reserve_gemm(c, rows, cols, n);
        }
        q8_launch_gemm_mfma(s, w, rows, cols, x + k * xs, xs, n, y + k * rows, part ? part : c->part, res ? res + k * rows : nullptr,
                            c->gemm_opts);
    }
}

void launched(const char *what)
{
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        fprintf(stderr, "q8_rt: launch of %s failed: %s\n", what, hipGetErrorString(e));
        abort(); /* a HIP failure, not a caller's mistake */
    }
}

/* Y = X W^T (w1 NULL) or SiLU(X W0^T) * (X W1^T), device pointers, on the stream. part != NULL (a
 * single product only): the matrix-core product's partials go there, and nothing is allocated. */
void product(ctx *c, const void *w0, const void *w1, long rows, long cols, const float *x, long xs, long t, float *y, float *part = nullptr)
{
    q8_stream_t s = (q8_stream_t)c->stream;
    if (c->ktime_on && c->kt.size() < KT_MAX) {
        const size_t i = c->kt.size();
        const int kind = c->exact ? RT_K_EXACT : (on_matrix_cores(t) ? RT_K_GEMM : RT_K_GEMV) + (w1 ? 1 : 0);
        c->kt.push_back(ktrec{kind, rows, cols, t, 0, {0}});
        q8_time_next(c->kt_events[2 * i], c->kt_events[2 * i + 1], c->kt.back().name, &c->kt.back().grid);
    }
    if (c->exact) {
        if (!w1) {
            q8_launch_exact(s, w0, rows, cols, x, xs, t, y);
        } else {
            float *g = reserve_scratch(c, (size_t)(2 * rows * t));
            q8_launch_exact(s, w0, rows, cols, x, xs, t, g);
            q8_launch_exact(s, w1, rows, cols, x, xs, t, g + rows * t);
            q8_launch_swiglu_ew(s, g, g + rows * t, rows * t, y);
        }
        launched("the reference-order product");
        return;
    }
    if (!on_matrix_cores(t)) {
        q8_launch_gemv(s, w0, w1, rows, cols, x, xs, t, y);
    } else if (!w1) {
        gemm_tokens(c, w0, rows, cols, x, xs, t, y, nullptr, part);
    } else {
        float *g = reserve_scratch(c, (size_t)(2 * rows * t));
        /* 64 tokens at a time, the gate and the up product as one round, their sums and the SwiGLU
         * in one launch: the same sums and SwiGLU as apart (below, where the round is refused) */
        const void *w2[2] = {w0, w1};
        const long r2[2] = {rows, rows};
        const long t0 = t < 64 ? t : 64;
        float *rp = reserve_rpart(c, (size_t)q8_gemm_round_part_floats(2, r2, cols, t0, c->gemm_opts));
        bool pair_done = true;
        for (long k = 0; k < t && pair_done; k += 64) {
            const long tk = t - k < 64 ? t - k : 64;
            float *y2[2] = {g, g + rows * tk};
            if (q8_launch_gemm_round(s, 2, w2, r2, cols, x + k * xs, xs, tk, y2, rp, (long)c->rpart_cap, c->gemm_opts, y + k * rows) != 0) {
                if (k > 0)
                    fail("the fused pair", "a later 64-token chunk refused its round (a planning error)");
                pair_done = false;
            }
        }
        if (pair_done) {
            launched("the fused pair");
            return;
        }
        gemm_tokens(c, w0, rows, cols, x, xs, t, g);
        gemm_tokens(c, w1, rows, cols, x, xs, t, g + rows * t);
        q8_launch_swiglu_ew(s, g, g + rows * t, rows * t, y);
    }
    launched("the product");
}

/* kernel timing for one launch about to be made: the record, or false when timing is off */
bool kt_begin(ctx *c, int kind, long rows, long cols, long t)
{
    if (!c->ktime_on || c->kt.size() >= KT_MAX)
        return false;
    const size_t i = c->kt.size();
    c->kt.push_back(ktrec{kind, rows, cols, t, 0, {0}});
    q8_time_next(c->kt_events[2 * i], c->kt_events[2 * i + 1], c->kt.back().name, &c->kt.back().grid);
    return true;
}

void kt_cancel(ctx *c)
{
    q8_time_next(nullptr, nullptr, nullptr, nullptr);
    c->kt.pop_back();
}

/* Y = X W^T (or the fused pair) with an epilogue: the RMS norm of x first (e.nw) or the residual
 * added to Y (e.res). Fused into the decode kernel where it takes the shape; else the norm apart
 * into the workspace and then the product, or the residual in the matrix-core product's store, or
 * the product into the workspace and then the add. */
void product_epi(ctx *c, const void *w0, const void *w1, long rows, long cols, const float *x, long xs, long t, float *y, q8_epi e)
{
    const q8_stream_t s = (q8_stream_t)c->stream;
    const bool apart = c->epi_apart != 0;
    if (!c->exact && t <= 4 && !apart) {
        const bool timed = kt_begin(c, RT_K_GEMV + (w1 ? 1 : 0), rows, cols, t);
        if (q8_launch_gemv_epi(s, w0, w1, rows, cols, x, xs, t, y, e) == 0) {
            launched("the product and its epilogue");
            return;
        }
        if (timed)
            kt_cancel(c);
    }
    if (e.nw) {
        float *xn = reserve_epi(c, (size_t)(t * cols));
        q8_launch_rmsnorm(s, x, xs, t, cols, e.nw, e.eps, xn);
        launched("the norm");
        product(c, w0, w1, rows, cols, xn, cols, t, y);
        return;
    }
    if (!c->exact && !w1 && !apart && on_matrix_cores(t)) {
        kt_begin(c, RT_K_GEMM, rows, cols, t);
        gemm_tokens(c, w0, rows, cols, x, xs, t, y, e.res);
        launched("the product and its residual");
        return;
    }
    float *tmp = reserve_epi(c, (size_t)(t * rows));
    product(c, w0, w1, rows, cols, x, xs, t, tmp);
    q8_launch_add(s, e.res, tmp, t * rows, y);
    launched("the residual add");
}

/* Products sharing x as one launch: at t <= 4 the decode round, from 5 tokens, 64 at a time, the
 * matrix-core round (one launch, each product on its own K split, so with its own launch's bits)
 * and one launch of their partial sums, in a workspace of its own grown to the
 * round. True when launched, false when the kernels do not take the shapes (the caller then runs
 * them one by one). */
bool round_launch(ctx *c, int n, const void *const *w, const long *rows, long cols, const float *x, long xs, long t, float *const *y)
{
    const bool timed = c->ktime_on && c->kt.size() < KT_MAX;
    if (timed) {
        long total = 0;
        for (int i = 0; i < n; i++)
            total += rows[i];
        const size_t k = c->kt.size();
        c->kt.push_back(ktrec{RT_K_ROUND, total, cols, t, 0, {0}});
        q8_time_next(c->kt_events[2 * k], c->kt_events[2 * k + 1], c->kt.back().name, &c->kt.back().grid);
    }
    int rc;
    if (t <= 4) {
        rc = q8_launch_gemv_round((q8_stream_t)c->stream, n, w, rows, cols, x, xs, t, y);
    } else {
        /* 64 tokens at a time (a token's bits do not depend on t) */
        float *rp = reserve_rpart(c, (size_t)q8_gemm_round_part_floats(n, rows, cols, t < 64 ? t : 64, c->gemm_opts));
        rc = 0;
        for (long k = 0; k < t && rc == 0; k += 64) {
            const long tk = t - k < 64 ? t - k : 64;
            float *yk[RT_BATCH];
            for (int i = 0; i < n; i++)
                yk[i] = y[i] + k * rows[i];
            rc = q8_launch_gemm_round((q8_stream_t)c->stream, n, w, rows, cols, x + k * xs, xs, tk, yk, rp, (long)c->rpart_cap, c->gemm_opts);
            if (rc != 0 && k > 0)
                fail("the round", "a later 64-token chunk refused its round (a planning error)");
        }
    }
    if (rc != 0) {
        if (timed) {
            q8_time_next(nullptr, nullptr, nullptr, nullptr);
            c->kt.pop_back();
        }
        return false;
    }
    launched("the round");
    return true;
}

/* Returns once every kernel queued on the runtime's stream so far is done and its stores are
 * visible to the host: a one-lane kernel queued last sets the pinned flag to this call's number
 * and the host polls it. Each kernel's end writes back its stores, and the flag's release store
 * follows them, so y in pinned memory is complete when the flag reads the number. This is 4.4 us a
 * call quicker than hipStreamSynchronize (18.4 against 14.0 us for a 4096x4096 rt_gemv). Every
 * 64th poll past the first 4096 also asks the stream, which reports a kernel that failed; the
 * wait ends at the runtime's deadline (q8_wait_until). */
void wait_done(ctx *c, const char *what)
{
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    HIPCHECK(hipStreamIsCapturing(c->stream, &st));
    if (st != hipStreamCaptureStatusNone)
        fail(what, "it waits for its result, so it cannot be recorded into a graph (use the _dev entry points)");
    const unsigned seq = ++c->flag_seq;
    q8_launch_flag((q8_stream_t)c->stream, c->flag, seq);
    launched("the completion flag");
    if (c->htime_on)
        c->ht_t2 = now_us();
    unsigned long polls = 0;
    q8_wait_until(
        [&] {
            if (__atomic_load_n(c->flag, __ATOMIC_ACQUIRE) == seq)
                return true;
            if (++polls > 4096 && (polls & 63) == 0) {
                const hipError_t e = hipStreamQuery(c->stream);
                if (e != hipSuccess && e != hipErrorNotReady) {
                    fprintf(stderr, "q8_rt: %s: the stream reports %s\n", what, hipGetErrorString(e));
                    abort();
                }
            }
            return false;
        },
        c->wait_s, what);
}

/* A round over host pointers: distinct x staged once, every product (those sharing x as one
 * launch), one wait. x goes to pinned memory on the host. When every product of the round is a
 * decode product (t <= 4, not exact) the kernels read x there directly (rt_set_x_direct, the
 * default: each workgroup reads all of x, and the L2 serves all but the first read of a line);
 * otherwise a copy kernel moves it to HBM first. One launch fewer a call: 14.1 against 15.6 us
 * for a 4096x4096 rt_gemv, 2.82 against 2.92 ms for the 9B token's 129 calls (one run each, from
 * C); the kernel itself waits ~1.7 us longer for x over the host link. The products store y
 * straight into pinned host memory, which the host reads after the wait. Asynchronous copies in
 * both directions cost more: 19.2 / 32.9 / 148.7 us against 17.6 / 24.3 / 126.6 us a call for
 * the 4096x4096, 12288x4096 and 151936x4096 GEMVs, 152 against 25 us at 4096x4096 with 4 tokens
 * (against the copy kernel). */
void run_round(ctx *c, job *jobs, int n, const char *what)
{
    const double t0 = c->htime_on ? now_us() : 0.0;
    size_t nx = 0, ny = 0;
    for (int i = 0; i < n; i++) {
        job &j = jobs[i];
        const size_t xlen = (size_t)(j.t * j.cols);
        j.x_off = (size_t)-1;
        for (int k = 0; k < i; k++)
            if (jobs[k].x == j.x && (size_t)(jobs[k].t * jobs[k].cols) == xlen) {
                j.x_off = jobs[k].x_off;
                break;
            }
        if (j.x_off == (size_t)-1) {
            j.x_off = nx;
            nx += (xlen + 63) / 64 * 64;
        }
        j.y_off = ny;
        ny += ((size_t)(j.t * j.rows) + 63) / 64 * 64;
    }
    reserve_staging(c, nx, ny);
    for (int i = 0; i < n; i++) {
        const job &j = jobs[i];
        bool first = true;
        for (int k = 0; k < i; k++)
            if (jobs[k].x_off == j.x_off)
                first = false;
        if (first)
            memcpy(c->hx + j.x_off, j.x, sizeof(float) * (size_t)(j.t * j.cols));
    }
    const double t1 = c->htime_on ? now_us() : 0.0;
    bool direct = c->x_direct && !c->exact;
    for (int i = 0; i < n; i++)
        direct = direct && jobs[i].t <= 4;
    const float *xb = c->dx;
    if (direct) {
        xb = c->hx;
    } else {
        q8_launch_copy((q8_stream_t)c->stream, c->dx, c->hx, (long)(nx / 4)); /* nx is a multiple of 64 floats */
        launched("the copy of x");
    }
    /* products that share x (and t): one round for the group */
    bool done[RT_BATCH] = {};
    for (int i = 0; i < n && !c->exact; i++) {
        if (done[i])
            continue;
        const void *w[RT_BATCH];
        long rows[RT_BATCH];
        float *y[RT_BATCH];
        int idx[RT_BATCH], k = 0;
        for (int j = i; j < n; j++)
            if (!done[j] && jobs[j].x_off == jobs[i].x_off && jobs[j].t == jobs[i].t && jobs[j].cols == jobs[i].cols) {
                w[k] = jobs[j].w, rows[k] = jobs[j].rows, y[k] = c->hy + jobs[j].y_off, idx[k++] = j;
            }
        if (k > 1 && round_launch(c, k, w, rows, jobs[i].cols, xb + jobs[i].x_off, jobs[i].cols, jobs[i].t, y))
            for (int j = 0; j < k; j++)
                done[idx[j]] = true;
    }
    for (int i = 0; i < n; i++) {
        const job &j = jobs[i];
        if (!done[i])
            product(c, j.w, nullptr, j.rows, j.cols, xb + j.x_off, j.cols, j.t, c->hy + j.y_off);
    }
    wait_done(c, what);
    const double t3 = c->htime_on ? now_us() : 0.0;
    for (int i = 0; i < n; i++)
        memcpy(jobs[i].y, c->hy + jobs[i].y_off, sizeof(float) * (size_t)(jobs[i].t * jobs[i].rows));
    if (c->htime_on) {
        const double t4 = now_us();
        c->ht[RT_HT_STAGE] += t1 - t0;
        c->ht[RT_HT_LAUNCH] += c->ht_t2 - t1;
        c->ht[RT_HT_WAIT] += t3 - c->ht_t2;
        c->ht[RT_HT_COPY_OUT] += t4 - t3;
        c->hcalls++;
    }
}

} // namespace

extern "C" {

int rt_init(struct rt *R, int threads)
{
    if (!R)
        return -1;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count < 1)
        return -1;
    const char *dev = getenv("Q8_DEVICE");
    const int device = dev ? atoi(dev) : 0;
    if (device < 0 || device >= count)
        return -1;
    if (hipSetDevice(device) != hipSuccess)
        return -1;
    ctx *c = new ctx;
    c->device = device;
    if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess || hipEventCreate(&c->ev0) != hipSuccess ||
        hipEventCreate(&c->ev1) != hipSuccess || hipHostMalloc((void **)&c->flag, 64, hipHostMallocDefault) != hipSuccess) {
        delete c;
        return -1;
    }
    __atomic_store_n(c->flag, 0u, __ATOMIC_RELEASE);
    /* this GPU's copy of the static scratch: its address, asked for once with the device current */
    if (hipGetSymbolAddress((void **)&c->noalloc_part, HIP_SYMBOL(scratch)) != hipSuccess || !c->noalloc_part) {
        (void)hipHostFree(c->flag);
        (void)hipEventDestroy(c->ev0);
        (void)hipEventDestroy(c->ev1);
        (void)hipStreamDestroy(c->stream);
        delete c;
        return -1;
    }
    /* the environment, read here once */
    const char *ex = getenv("Q8_EXACT");
    c->exact = ex && atoi(ex) != 0;
    const char *ws = getenv("Q8_WAIT_S");
    if (ws && atof(ws) > 0.0)
        c->wait_s = atof(ws);
    const char *uc = getenv("Q8_UPLOAD_CHUNK");
    if (uc && atol(uc) > 0)
        c->upload_chunk = (size_t)atol(uc);
    const char *ae = getenv("Q8_ABORT_EXIT");
    abort_exit = ae ? atoi(ae) : 0;
    /* R->team and R->frame belong to the caller, which creates its team before rt_init
     * (src/card/engine.c:249-250) and keeps using it for the primitives that are not products */
    R->gemm_chain = nullptr;
    R->chain = c;
    R->threads = threads;
    live.push_back(c);
    current = c;
    return 0;
}

void rt_fini(struct rt *R)
{
    if (!R || !R->chain)
        return;
    ctx *c = (ctx *)R->chain;
    sync_stream(c, "rt_fini");
    for (auto &kv : c->weights)
        if (kv.second.owned)
            HIPCHECK(hipFree((void *)kv.first));
    if (c->hx)
        HIPCHECK(hipHostFree(c->hx));
    if (c->hy)
        HIPCHECK(hipHostFree(c->hy));
    if (c->dx)
        HIPCHECK(hipFree(c->dx));
    if (c->flag)
        HIPCHECK(hipHostFree(c->flag));
    if (c->scratch)
        HIPCHECK(hipFree(c->scratch));
    if (c->part)
        HIPCHECK(hipFree(c->part));
    if (c->epi)
        HIPCHECK(hipFree(c->epi));
    if (c->rpart)
        HIPCHECK(hipFree(c->rpart));
    for (void *p : c->retired)
        HIPCHECK(hipFree(p));
    for (auto &e : c->kt_events)
        HIPCHECK(hipEventDestroy(e));
    if (c->amax)
        HIPCHECK(hipFree(c->amax));
    for (int k = 0; k < 2; k++) {
        if (c->up_host[k])
            HIPCHECK(hipHostFree(c->up_host[k]));
        if (c->up_dev[k])
            HIPCHECK(hipFree(c->up_dev[k]));
        if (c->up_done[k])
            HIPCHECK(hipEventDestroy(c->up_done[k]));
    }
    for (size_t i = 0; i < live.size(); i++)
        if (live[i] == c) {
            live.erase(live.begin() + (long)i);
            break;
        }
    current = live.empty() ? nullptr : live.back();
    HIPCHECK(hipEventDestroy(c->ev0));
    HIPCHECK(hipEventDestroy(c->ev1));
    HIPCHECK(hipStreamDestroy(c->stream));
    delete c;
    R->chain = nullptr;
}

void rt_gemv(struct rt *R, const void *w, long rows, long cols, const float *x, float *y)
{
    ctx *c = get(R, "rt_gemv");
    check_shape(c, "rt_gemv", w, rows, cols);
    if (!x || !y)
        fail("rt_gemv", "x and y must be host arrays");
    job j = {w, rows, cols, 1, x, y, 0, 0};
    run_round(c, &j, 1, "rt_gemv");
}

void rt_gemv_q(struct rt *R, const void *w, long rows, long cols, const float *x, float *y)
{
    ctx *c = get(R, "rt_gemv_q");
    check_shape(c, "rt_gemv_q", w, rows, cols);
    if (c->queued >= RT_BATCH)
        fail("rt_gemv_q", "more than RT_BATCH (8) products queued");
    c->queue[c->queued++] = job{w, rows, cols, 1, x, y, 0, 0};
}

void rt_gemm_q(struct rt *R, const void *w, long rows, long cols, const float *x, long t, float *y)
{
    ctx *c = get(R, "rt_gemm_q");
    check_shape(c, "rt_gemm_q", w, rows, cols);
    if (t < 1)
        fail("rt_gemm_q", "t must be at least 1");
    if (c->queued >= RT_BATCH)
        fail("rt_gemm_q", "more than RT_BATCH (8) products queued");
    c->queue[c->queued++] = job{w, rows, cols, t, x, y, 0, 0};
}

void rt_gemv_open(struct rt *R) { (void)get(R, "rt_gemv_open"); }

void rt_gemv_go(struct rt *R)
{
    ctx *c = get(R, "rt_gemv_go");
    if (c->queued)
        run_round(c, c->queue, c->queued, "rt_gemv_go");
    c->queued = 0;
}

void rt_gemm(struct rt *R, const void *w, long rows, long cols, const float *x, long t, float *y)
{
    ctx *c = get(R, "rt_gemm");
    check_shape(c, "rt_gemm", w, rows, cols);
    if (t < 1)
        fail("rt_gemm", "t must be at least 1");
    job j = {w, rows, cols, t, x, y, 0, 0};
    run_round(c, &j, 1, "rt_gemm");
}

long gemv_i_bytes(long rows, long cols) { return rows / Q8_GROUP * (cols / Q8_BLOCK) * 544; }

void gemv_i_repack(const uint8_t *q8, long rows, long cols, void *out)
{
    if (!q8 || !out || rows <= 0 || cols <= 0 || rows % Q8_GROUP || cols % Q8_BLOCK)
        fail("gemv_i_repack", "needs q8, out, rows a positive multiple of 16, cols of 32");
    const long nb = cols / Q8_BLOCK;
    uint8_t *o = (uint8_t *)out;
    for (long g = 0; g < rows / Q8_GROUP; g++) {
        uint8_t *grp = o + g * 17 * cols;
        for (int r = 0; r < Q8_GROUP; r++) {
            const uint8_t *src = q8 + (g * Q8_GROUP + r) * nb * Q8_BLOCK_BYTES;
            uint8_t *q = grp + r * cols, *d = grp + Q8_GROUP * cols + r * (cols / 16);
            for (long b = 0; b < nb; b++) {
                memcpy(q + b * Q8_BLOCK, src + b * Q8_BLOCK_BYTES + 2, Q8_BLOCK);
                memcpy(d + 2 * b, src + b * Q8_BLOCK_BYTES, 2);
            }
        }
    }
}

static const void *register_matrix(ctx *c, void *dev, long rows, long cols, bool owned = true)
{
    c->weights[dev] = matrix{rows, cols, owned};
    return dev;
}

extern "C++" {
/* Bytes of an upload chunk: the runtime's setting (64 MiB unless Q8_UPLOAD_CHUNK or
 * rt_set_upload_chunk says otherwise), at least one 16-row group. */
static size_t upload_chunk(const ctx *c, size_t group) { return c->upload_chunk < group ? group : c->upload_chunk; }

static void reserve_upload(ctx *c, size_t group)
{
    const size_t need = upload_chunk(c, group);
    if (c->up_cap >= need)
        return;
    no_capture(c, "the upload staging");
    sync_stream(c, "the upload staging");
    for (int k = 0; k < 2; k++) {
        if (c->up_host[k])
            HIPCHECK(hipHostFree(c->up_host[k]));
        if (c->up_dev[k])
            HIPCHECK(hipFree(c->up_dev[k]));
        HIPCHECK(hipHostMalloc((void **)&c->up_host[k], need, hipHostMallocDefault));
        HIPCHECK(hipMalloc((void **)&c->up_dev[k], need));
        if (!c->up_done[k])
            HIPCHECK(hipEventCreateWithFlags(&c->up_done[k], hipEventDisableTiming));
    }
    c->up_cap = need;
}

/* A new form S matrix of rows x cols from GGUF Q8_0 rows, chunk by chunk: read(dst, off, n) puts
 * the source's bytes [off, off + n) into a pinned chunk, which goes to HBM and is repacked there
 * (a run of whole 16-row groups is a form S matrix of its own, at the same byte offset) while the
 * host fills the other chunk. nullptr, with nothing left allocated, when HBM is full or a read
 * fails (*read_failed set). */
template <class Read>
static const void *upload_groups(ctx *c, const char *fn, long rows, long cols, Read read, bool *read_failed)
{
    no_capture(c, fn);
    const size_t bytes = (size_t)gemv_i_bytes(rows, cols), group = (size_t)gemv_i_bytes(Q8_GROUP, cols);
    reserve_upload(c, group);
    const size_t want = upload_chunk(c, group), per = (want < c->up_cap ? want : c->up_cap) / group * group;
    void *out = nullptr;
    if (hipMalloc(&out, bytes) != hipSuccess)
        return nullptr;
    int k = 0;
    for (size_t off = 0; off < bytes; off += per, k ^= 1) {
        const size_t n = bytes - off < per ? bytes - off : per;
        sync_event(c, c->up_done[k], fn); /* the slot's last copy has read its chunk */
        if (!read(c->up_host[k], off, n)) {
            sync_stream(c, fn);
            HIPCHECK(hipFree(out));
            *read_failed = true;
            return nullptr;
        }
        HIPCHECK(hipMemcpyAsync(c->up_dev[k], c->up_host[k], n, hipMemcpyHostToDevice, c->stream));
        q8_launch_repack((q8_stream_t)c->stream, c->up_dev[k], (long)(n / group) * Q8_GROUP, cols, (uint8_t *)out + off);
        launched("the repack");
        HIPCHECK(hipEventRecord(c->up_done[k], c->stream));
    }
    sync_stream(c, fn);
    return register_matrix(c, out, rows, cols);
}
} /* extern "C++" */

const void *rt_q8_upload(struct rt *R, const uint8_t *q8, long rows, long cols)
{
    ctx *c = get(R, "rt_q8_upload");
    if (!q8 || rows <= 0 || cols <= 0 || rows % Q8_GROUP || cols % Q8_BLOCK)
        fail("rt_q8_upload", "needs q8, rows a positive multiple of 16, cols of 32");
    bool bad = false;
    return upload_groups(
        c, "rt_q8_upload", rows, cols,
        [&](uint8_t *dst, size_t off, size_t n) {
            memcpy(dst, q8 + off, n);
            return true;
        },
        &bad);
}

const void *rt_q8_upload_fd(struct rt *R, int fd, uint64_t offset, long rows, long cols)
{
    ctx *c = get(R, "rt_q8_upload_fd");
    if (fd < 0 || rows <= 0 || cols <= 0 || rows % Q8_GROUP || cols % Q8_BLOCK)
        fail("rt_q8_upload_fd", "needs an open file, rows a positive multiple of 16, cols of 32");
    bool bad = false;
    const void *w = upload_groups(
        c, "rt_q8_upload_fd", rows, cols,
        [&](uint8_t *dst, size_t off, size_t n) {
            for (size_t got = 0; got < n;) {
                const ssize_t r = pread(fd, dst + got, n - got, (off_t)(offset + off + got));
                if (r <= 0)
                    return false;
                got += (size_t)r;
            }
            return true;
        },
        &bad);
    if (!w)
        errno = bad ? (errno ? errno : EIO) : ENOMEM;
    return w;
}

const void *rt_q8_upload_packed(struct rt *R, const void *packed, long rows, long cols)
{
    ctx *c = get(R, "rt_q8_upload_packed");
    if (!packed || rows <= 0 || cols <= 0 || rows % Q8_GROUP || cols % Q8_BLOCK)
        fail("rt_q8_upload_packed", "needs packed, rows a positive multiple of 16, cols of 32");
    const size_t bytes = (size_t)gemv_i_bytes(rows, cols);
    void *out = nullptr;
    if (hipMalloc(&out, bytes) != hipSuccess)
        return nullptr;
    HIPCHECK(hipMemcpyAsync(out, packed, bytes, hipMemcpyHostToDevice, c->stream));
    sync_stream(c, "rt_q8_upload_packed");
    return register_matrix(c, out, rows, cols);
}

void rt_q8_free(struct rt *R, const void *w)
{
    ctx *c = get(R, "rt_q8_free");
    auto it = c->weights.find(w);
    if (it == c->weights.end())
        fail("rt_q8_free", "w is not a handle from rt_q8_upload");
    if (!it->second.owned)
        fail("rt_q8_free", "w is a buffer of the caller's that rt_q8_repack_dev registered: free it with rt_dev_free");
    sync_stream(c, "rt_q8_free");
    HIPCHECK(hipFree((void *)w));
    c->weights.erase(it);
}

void rt_gemv_dev(struct rt *R, const void *w, long rows, long cols, const float *x, float *y)
{
    rt_gemm_dev(R, w, rows, cols, x, cols, 1, y);
}

void rt_gemm_dev(struct rt *R, const void *w, long rows, long cols, const float *x, long x_stride, long t, float *y)
{
    ctx *c = get(R, "rt_gemm_dev");
    check_shape(c, "rt_gemm_dev", w, rows, cols);
    check_dev_ptr("rt_gemm_dev", x, "x");
    check_dev_ptr("rt_gemm_dev", y, "y");
    if (t < 1 || x_stride < cols || x_stride % 4)
        fail("rt_gemm_dev", "t >= 1 and x_stride >= cols, a multiple of 4");
    product(c, w, nullptr, rows, cols, x, x_stride, t, y);
}

void rt_gemm_dev_noalloc(struct rt *R, const void *w, long rows, long cols, const float *x, long x_stride, long t, float *y)
{
    ctx *c = get(R, "rt_gemm_dev_noalloc");
    check_shape(c, "rt_gemm_dev_noalloc", w, rows, cols);
    check_dev_ptr("rt_gemm_dev_noalloc", x, "x");
    check_dev_ptr("rt_gemm_dev_noalloc", y, "y");
    if (t < 1 || x_stride < cols || x_stride % 4)
        fail("rt_gemm_dev_noalloc", "t >= 1 and x_stride >= cols, a multiple of 4");
    product(c, w, nullptr, rows, cols, x, x_stride, t, y, c->noalloc_part);
}

void rt_gemv_round_dev(struct rt *R, int n, const void *const *w, const long *rows, long cols, const float *x, long x_stride, long t, float *const *y)
{
    ctx *c = get(R, "rt_gemv_round_dev");
    if (n < 1 || n > RT_BATCH || !w || !rows || !y)
        fail("rt_gemv_round_dev", "needs 1..RT_BATCH (8) products");
    check_dev_ptr("rt_gemv_round_dev", x, "x");
    if (t < 1 || x_stride < cols || x_stride % 4)
        fail("rt_gemv_round_dev", "t >= 1 and x_stride >= cols, a multiple of 4");
    for (int i = 0; i < n; i++) {
        check_shape(c, "rt_gemv_round_dev", w[i], rows[i], cols);
        check_dev_ptr("rt_gemv_round_dev", y[i], "every y");
    }
    if (!c->exact && n > 1 && round_launch(c, n, w, rows, cols, x, x_stride, t, y))
        return;
    for (int i = 0; i < n; i++)
        product(c, w[i], nullptr, rows[i], cols, x, x_stride, t, y[i]);
}

void rt_gemv_swiglu_dev(struct rt *R, const void *wg, const void *wu, long rows, long cols, const float *x, long x_stride, long t, float *y)
{
    ctx *c = get(R, "rt_gemv_swiglu_dev");
    check_shape(c, "rt_gemv_swiglu_dev", wg, rows, cols);
    check_shape(c, "rt_gemv_swiglu_dev", wu, rows, cols);
    check_dev_ptr("rt_gemv_swiglu_dev", x, "x");
    check_dev_ptr("rt_gemv_swiglu_dev", y, "y");
    if (t < 1 || x_stride < cols || x_stride % 4)
        fail("rt_gemv_swiglu_dev", "t >= 1 and x_stride >= cols, a multiple of 4");
    product(c, wg, wu, rows, cols, x, x_stride, t, y);
}

static void check_rows(const char *fn, long cols, long x_stride, long t)
{
    if (t < 1 || x_stride < cols || x_stride % 4)
        fail(fn, "t >= 1 and x_stride >= cols, a multiple of 4");
}

void rt_rmsnorm_dev(struct rt *R, const float *x, long x_stride, long t, long cols, const float *nw, float eps, float *xn)
{
    ctx *c = get(R, "rt_rmsnorm_dev");
    check_dev_ptr("rt_rmsnorm_dev", x, "x");
    check_dev_ptr("rt_rmsnorm_dev", nw, "nw");
    check_dev_ptr("rt_rmsnorm_dev", xn, "xn");
    if (cols <= 0 || cols % 4)
        fail("rt_rmsnorm_dev", "cols must be a positive multiple of 4");
    check_rows("rt_rmsnorm_dev", cols, x_stride, t);
    q8_launch_rmsnorm((q8_stream_t)c->stream, x, x_stride, t, cols, nw, eps, xn);
    launched("the norm");
}

void rt_gemm_norm_dev(struct rt *R, const void *w, long rows, long cols, const float *x, long x_stride, long t, const float *nw, float eps, float *y)
{
    ctx *c = get(R, "rt_gemm_norm_dev");
    check_shape(c, "rt_gemm_norm_dev", w, rows, cols);
    check_dev_ptr("rt_gemm_norm_dev", x, "x");
    check_dev_ptr("rt_gemm_norm_dev", nw, "nw");
    check_dev_ptr("rt_gemm_norm_dev", y, "y");
    check_rows("rt_gemm_norm_dev", cols, x_stride, t);
    product_epi(c, w, nullptr, rows, cols, x, x_stride, t, y, q8_epi{nw, eps, nullptr});
}

void rt_gemv_swiglu_norm_dev(struct rt *R, const void *wg, const void *wu, long rows, long cols, const float *x, long x_stride, long t, const float *nw,
                             float eps, float *y)
{
    ctx *c = get(R, "rt_gemv_swiglu_norm_dev");
    check_shape(c, "rt_gemv_swiglu_norm_dev", wg, rows, cols);
    check_shape(c, "rt_gemv_swiglu_norm_dev", wu, rows, cols);
    check_dev_ptr("rt_gemv_swiglu_norm_dev", x, "x");
    check_dev_ptr("rt_gemv_swiglu_norm_dev", nw, "nw");
    check_dev_ptr("rt_gemv_swiglu_norm_dev", y, "y");
    check_rows("rt_gemv_swiglu_norm_dev", cols, x_stride, t);
    product_epi(c, wg, wu, rows, cols, x, x_stride, t, y, q8_epi{nw, eps, nullptr});
}

void rt_gemv_round_norm_dev(struct rt *R, int n, const void *const *w, const long *rows, long cols, const float *x, long x_stride, long t,
                            const float *nw, float eps, float *const *y)
{
    ctx *c = get(R, "rt_gemv_round_norm_dev");
    if (n < 1 || n > RT_BATCH || !w || !rows || !y)
        fail("rt_gemv_round_norm_dev", "needs 1..RT_BATCH (8) products");
    check_dev_ptr("rt_gemv_round_norm_dev", x, "x");
    check_dev_ptr("rt_gemv_round_norm_dev", nw, "nw");
    check_rows("rt_gemv_round_norm_dev", cols, x_stride, t);
    for (int i = 0; i < n; i++) {
        check_shape(c, "rt_gemv_round_norm_dev", w[i], rows[i], cols);
        check_dev_ptr("rt_gemv_round_norm_dev", y[i], "every y");
    }
    const q8_stream_t s = (q8_stream_t)c->stream;
    if (!c->exact && t <= 4 && !c->epi_apart) {
        long total = 0;
        for (int i = 0; i < n; i++)
            total += rows[i];
        const bool timed = kt_begin(c, RT_K_ROUND, total, cols, t);
        if (q8_launch_gemv_round_epi(s, n, w, rows, cols, x, x_stride, t, y, q8_epi{nw, eps, nullptr}) == 0) {
            launched("the round and its norm");
            return;
        }
        if (timed)
            kt_cancel(c);
    }
    float *xn = reserve_epi(c, (size_t)(t * cols));
    q8_launch_rmsnorm(s, x, x_stride, t, cols, nw, eps, xn);
    launched("the norm");
    if (!c->exact && n > 1 && round_launch(c, n, w, rows, cols, xn, cols, t, y))
        return;
    for (int i = 0; i < n; i++)
        product(c, w[i], nullptr, rows[i], cols, xn, cols, t, y[i]);
}

void rt_gemm_residual_dev(struct rt *R, const void *w, long rows, long cols, const float *x, long x_stride, long t, const float *r, float *y)
{
    ctx *c = get(R, "rt_gemm_residual_dev");
    check_shape(c, "rt_gemm_residual_dev", w, rows, cols);
    check_dev_ptr("rt_gemm_residual_dev", x, "x");
    check_dev_ptr("rt_gemm_residual_dev", r, "r");
    check_dev_ptr("rt_gemm_residual_dev", y, "y");
    check_rows("rt_gemm_residual_dev", cols, x_stride, t);
    product_epi(c, w, nullptr, rows, cols, x, x_stride, t, y, q8_epi{nullptr, 0.0f, r});
}

void *rt_dev_alloc(struct rt *R, long bytes)
{
    (void)get(R, "rt_dev_alloc");
    void *p = nullptr;
    if (bytes <= 0 || hipMalloc(&p, (size_t)bytes) != hipSuccess)
        return nullptr;
    return p;
}

void rt_dev_free(struct rt *R, void *p)
{
    ctx *c = get(R, "rt_dev_free");
    if (!p)
        return;
    auto it = c->weights.find(p);
    if (it != c->weights.end() && it->second.owned)
        fail("rt_dev_free", "p is a weight handle the library allocated: free it with rt_q8_free");
    /* every buffer rt_q8_repack_dev registered inside the allocation stops being a handle, the
     * allocation's start or an address inside it */
    hipDeviceptr_t base = nullptr;
    size_t size = 0;
    HIPCHECK(hipMemGetAddressRange(&base, &size, (hipDeviceptr_t)p));
    const uintptr_t lo = (uintptr_t)base, hi = lo + size;
    for (auto w = c->weights.begin(); w != c->weights.end();) {
        const uintptr_t a = (uintptr_t)w->first;
        if (!w->second.owned && a >= lo && a < hi)
            w = c->weights.erase(w);
        else
            ++w;
    }
    sync_stream(c, "rt_dev_free");
    HIPCHECK(hipFree(p));
}

void rt_dev_upload(struct rt *R, void *dst, const void *src, long bytes)
{
    ctx *c = get(R, "rt_dev_upload");
    HIPCHECK(hipMemcpyAsync(dst, src, (size_t)bytes, hipMemcpyHostToDevice, c->stream));
    sync_stream(c, "rt_dev_upload");
}

void rt_dev_download(struct rt *R, void *dst, const void *src, long bytes)
{
    ctx *c = get(R, "rt_dev_download");
    HIPCHECK(hipMemcpyAsync(dst, src, (size_t)bytes, hipMemcpyDeviceToHost, c->stream));
    sync_stream(c, "rt_dev_download");
}

void rt_dev_sync(struct rt *R)
{
    ctx *c = get(R, "rt_dev_sync");
    sync_stream(c, "rt_dev_sync");
}

void rt_q8_fill_dev(struct rt *R, void *dst, long rows, long cols, uint64_t seed, int dist, float mu, float sigma)
{
    ctx *c = get(R, "rt_q8_fill_dev");
    if (!dst || rows <= 0 || cols <= 0 || cols % Q8_BLOCK || ((uintptr_t)dst & 1))
        fail("rt_q8_fill_dev", "needs an even device address, rows > 0, cols a positive multiple of 32");
    q8_launch_fill((q8_stream_t)c->stream, dst, rows, cols, seed, dist, mu, sigma);
    launched("the fill");
}

void rt_q8_repack_dev(struct rt *R, const void *q8_dev, long rows, long cols, void *out_dev)
{
    ctx *c = get(R, "rt_q8_repack_dev");
    if (!q8_dev || !out_dev || rows <= 0 || cols <= 0 || rows % Q8_GROUP || cols % Q8_BLOCK || ((uintptr_t)out_dev & 31) || ((uintptr_t)q8_dev & 1))
        fail("rt_q8_repack_dev", "needs rows a positive multiple of 16, cols of 32, out 32-byte aligned");
    /* out_dev must not lie in a matrix the library allocated: its start or an address inside it */
    hipDeviceptr_t base = nullptr;
    size_t size = 0;
    HIPCHECK(hipMemGetAddressRange(&base, &size, (hipDeviceptr_t)out_dev));
    auto it = c->weights.find((const void *)base);
    if (it != c->weights.end() && it->second.owned)
        fail("rt_q8_repack_dev", "out_dev lies in a weight handle the library allocated");
    if ((uintptr_t)out_dev + (size_t)gemv_i_bytes(rows, cols) > (uintptr_t)base + size)
        fail("rt_q8_repack_dev", "out_dev's allocation ends before the repacked matrix does");
    q8_launch_repack((q8_stream_t)c->stream, q8_dev, rows, cols, out_dev);
    launched("the repack");
    register_matrix(c, out_dev, rows, cols, false);
}

void rt_f32_fill_dev(struct rt *R, float *dst, long n, uint64_t seed)
{
    ctx *c = get(R, "rt_f32_fill_dev");
    if (!dst || n <= 0)
        fail("rt_f32_fill_dev", "needs dst and n > 0");
    q8_launch_fill_f32((q8_stream_t)c->stream, dst, n, seed);
    launched("the fill");
}

void rt_q8_row(const void *w, long cols, long row, float *z)
{
    ctx *c = current;
    if (!c)
        fail("rt_q8_row", "rt_init has not run");
    auto it = c->weights.find(w);
    if (it == c->weights.end())
        fail("rt_q8_row", "w is not a handle from rt_q8_upload");
    if (cols != it->second.cols || row < 0 || row >= it->second.rows || !z)
        fail("rt_q8_row", "cols must be the matrix's and row one of its rows");
    reserve_staging(c, 64, (size_t)cols);
    /* the row index staged where x goes (one 16-byte copy), the row stored into pinned memory */
    long *dr = (long *)c->dx;
    ((long *)c->hx)[0] = row, ((long *)c->hx)[1] = 0;
    q8_launch_copy((q8_stream_t)c->stream, dr, c->hx, 1);
    launched("the copy of the row index");
    q8_launch_rows((q8_stream_t)c->stream, w, cols, it->second.rows, dr, 1, c->hy);
    launched("the row read");
    wait_done(c, "rt_q8_row");
    memcpy(z, c->hy, sizeof(float) * (size_t)cols);
}

void rt_q8_rows_dev(struct rt *R, const void *w, long cols, const long *rows, long n, float *z)
{
    ctx *c = get(R, "rt_q8_rows_dev");
    auto it = c->weights.find(w);
    if (it == c->weights.end())
        fail("rt_q8_rows_dev", "w is not a handle from rt_q8_upload");
    if (cols != it->second.cols || n < 1 || !rows)
        fail("rt_q8_rows_dev", "cols must be the matrix's and n >= 1");
    check_dev_ptr("rt_q8_rows_dev", z, "z");
    q8_launch_rows((q8_stream_t)c->stream, w, cols, it->second.rows, rows, n, z);
    launched("the row gather");
}

void rt_argmax_dev(struct rt *R, const float *a, long n, long *idx)
{
    ctx *c = get(R, "rt_argmax_dev");
    if (!a || !idx || n < 1)
        fail("rt_argmax_dev", "needs a, idx and n >= 1");
    const size_t need = (size_t)q8_argmax_chunks(n) * (sizeof(float) + sizeof(long)) + 64;
    if (need > c->amax_cap) {
        no_capture(c, "the next token's candidates");
        if (c->amax)
            c->retired.push_back(c->amax);
        HIPCHECK(hipMalloc(&c->amax, need));
        c->amax_cap = need;
    }
    const long nc = q8_argmax_chunks(n);
    long *ci = (long *)c->amax;
    float *cm = (float *)(ci + nc);
    q8_launch_argmax((q8_stream_t)c->stream, a, n, cm, ci, idx);
    launched("the next token");
}

void rt_dev_copy(struct rt *R, void *dst, const void *src, long bytes)
{
    ctx *c = get(R, "rt_dev_copy");
    if (!dst || !src || bytes <= 0 || bytes % 16 || ((uintptr_t)dst & 15) || ((uintptr_t)src & 15))
        fail("rt_dev_copy", "needs 16-byte aligned device addresses and bytes a positive multiple of 16");
    q8_launch_copy((q8_stream_t)c->stream, dst, src, bytes / 16);
    launched("the copy");
}

void rt_q8_read_dev(struct rt *R, const void *w0, const void *w1, long rows, long cols, const float *x, long x_stride, long t, unsigned *sink)
{
    ctx *c = get(R, "rt_q8_read_dev");
    check_shape(c, "rt_q8_read_dev", w0, rows, cols);
    if (w1)
        check_shape(c, "rt_q8_read_dev", w1, rows, cols);
    check_dev_ptr("rt_q8_read_dev", x, "x");
    check_dev_ptr("rt_q8_read_dev", sink, "sink");
    if (t < 1 || t > 16 || (t > 1 && (x_stride < cols || x_stride % 4)))
        fail("rt_q8_read_dev", "needs 1 to 16 tokens, x rows at least cols floats apart (a multiple of 4)");
    if (t >= 5) {
        if (w1)
            fail("rt_q8_read_dev", "at 5 to 16 tokens it reads one matrix (the fused pair runs as two products there)");
        const bool timed = kt_begin(c, RT_K_GEMM, rows, cols, t);
        if (q8_launch_read_gemm((q8_stream_t)c->stream, w0, rows, cols, x, x_stride, t, sink, c->gemm_opts) != 0) {
            if (timed)
                kt_cancel(c);
            fail("rt_q8_read_dev", "at 5 to 16 tokens it reads for the x-resident matrix-core kernel, which rt_gemm_force has switched off");
        }
        launched("the read");
        return;
    }
    const bool timed = kt_begin(c, w1 ? RT_K_GEMV_PAIR : RT_K_GEMV, rows, cols, t);
    if (q8_launch_read((q8_stream_t)c->stream, w0, w1, rows, cols, x, x_stride, t, sink) != 0) {
        if (timed)
            kt_cancel(c);
        failf("rt_q8_read_dev", "no read kernel for %ld x %ld%s at %ld tokens (the decode kernel's grids for the decode token's shapes at one "
              "token, and for the 9B verify shapes at 2 to 4)", rows, cols, w1 ? " (pair)" : "", t);
    }
    launched("the read");
}

void rt_prims_dev(struct rt *R, const int8_t *q, const float *x8, const float *c8, float *o8, long n8, const uint16_t *h, const float *xf,
                  const float *cf, float *of, long nf)
{
    ctx *c = get(R, "rt_prims_dev");
    if (n8 % 4)
        fail("rt_prims_dev", "n8 must be a multiple of 4");
    q8_launch_prims((q8_stream_t)c->stream, q, x8, c8, o8, n8, h, xf, cf, of, nf);
    launched("the primitive gate");
}

int rt_set_exact(struct rt *R, int exact)
{
    ctx *c = get(R, "rt_set_exact");
    const int old = c->exact;
    c->exact = exact != 0;
    return old;
}

int rt_set_epi_apart(struct rt *R, int apart)
{
    ctx *c = get(R, "rt_set_epi_apart");
    const int old = c->epi_apart;
    c->epi_apart = apart != 0;
    return old;
}

long rt_set_upload_chunk(struct rt *R, long bytes)
{
    ctx *c = get(R, "rt_set_upload_chunk");
    if (bytes <= 0)
        fail("rt_set_upload_chunk", "bytes must be positive");
    const long old = (long)c->upload_chunk;
    c->upload_chunk = (size_t)bytes;
    return old;
}

int rt_set_x_direct(struct rt *R, int direct)
{
    ctx *c = get(R, "rt_set_x_direct");
    const int old = c->x_direct;
    c->x_direct = direct != 0;
    return old;
}

void rt_gemm_force(struct rt *R, int streaming, int ks)
{
    ctx *c = get(R, "rt_gemm_force");
    if (ks < 0)
        fail("rt_gemm_force", "ks must be 0 (the planner's) or a split count");
    c->gemm_opts = q8_gemm_opts{ks, streaming != 0};
}

void rt_timer_start(struct rt *R)
{
    ctx *c = get(R, "rt_timer_start");
    HIPCHECK(hipEventRecord(c->ev0, c->stream));
}

float rt_timer_stop(struct rt *R)
{
    ctx *c = get(R, "rt_timer_stop");
    float ms = 0.0f;
    HIPCHECK(hipEventRecord(c->ev1, c->stream));
    sync_event(c, c->ev1, "rt_timer_stop");
    HIPCHECK(hipEventElapsedTime(&ms, c->ev0, c->ev1));
    return ms;
}

void rt_graph_begin(struct rt *R)
{
    ctx *c = get(R, "rt_graph_begin");
    if (c->ktime_on)
        fail("rt_graph_begin", "kernel timing is on: switch it off before recording");
    HIPCHECK(hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
}

void *rt_graph_end(struct rt *R)
{
    ctx *c = get(R, "rt_graph_end");
    hipGraph_t g = nullptr;
    hipGraphExec_t e = nullptr;
    HIPCHECK(hipStreamEndCapture(c->stream, &g));
    HIPCHECK(hipGraphInstantiate(&e, g, nullptr, nullptr, 0));
    HIPCHECK(hipGraphDestroy(g));
    return (void *)e;
}

void rt_graph_launch(struct rt *R, void *graph)
{
    ctx *c = get(R, "rt_graph_launch");
    HIPCHECK(hipGraphLaunch((hipGraphExec_t)graph, c->stream));
}

void rt_graph_free(struct rt *R, void *graph)
{
    ctx *c = get(R, "rt_graph_free");
    sync_stream(c, "rt_graph_free");
    HIPCHECK(hipGraphExecDestroy((hipGraphExec_t)graph));
}

void rt_host_timing(struct rt *R, int on)
{
    ctx *c = get(R, "rt_host_timing");
    c->htime_on = on != 0;
    for (double &v : c->ht)
        v = 0.0;
    c->hcalls = 0;
}

long rt_host_timing_read(struct rt *R, double *us)
{
    ctx *c = get(R, "rt_host_timing_read");
    if (!us)
        fail("rt_host_timing_read", "us is NULL");
    for (int k = 0; k < RT_HT_PHASES; k++)
        us[k] = c->ht[k];
    return c->hcalls;
}

void rt_ktime(struct rt *R, int on)
{
    ctx *c = get(R, "rt_ktime");
    if (on && c->kt_events.empty()) {
        c->kt_events.resize(2 * KT_MAX);
        c->kt.reserve(KT_MAX); /* the timing slot points into the last record: no reallocation */
        for (auto &e : c->kt_events)
            HIPCHECK(hipEventCreate(&e));
    }
    c->kt.clear();
    c->ktime_on = on != 0;
}

long rt_ktime_read(struct rt *R, int *kind, long *rows, long *cols, long *t, float *us, char *names, long *grid, long max)
{
    ctx *c = get(R, "rt_ktime_read");
    sync_stream(c, "rt_ktime_read");
    const long n = (long)c->kt.size() < max ? (long)c->kt.size() : max;
    for (long i = 0; i < n; i++) {
        float ms = 0.0f;
        HIPCHECK(hipEventElapsedTime(&ms, c->kt_events[2 * i], c->kt_events[2 * i + 1]));
        kind[i] = c->kt[i].kind;
        rows[i] = c->kt[i].rows;
        cols[i] = c->kt[i].cols;
        t[i] = c->kt[i].t;
        us[i] = 1000.0f * ms;
        if (names)
            memcpy(names + 64 * i, c->kt[i].name, 64);
        if (grid)
            grid[i] = c->kt[i].grid;
    }
    c->kt.clear();
    return n;
}

void rt_device_info(struct rt *R, char *name, long name_len, int *cus)
{
    ctx *c = get(R, "rt_device_info");
    hipDeviceProp_t p;
    HIPCHECK(hipGetDeviceProperties(&p, c->device));
    if (name && name_len > 0) {
        snprintf(name, (size_t)name_len, "%s (%s)", p.name, p.gcnArchName);
    }
    if (cus)
        *cus = p.multiProcessorCount;
}

} /* extern "C" */
