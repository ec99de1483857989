/* q8_rt.h: the Q8_0 weight products of the APL engine's runtime, on one MI355X (gfx950).
 *
 * Drop-in for the product half of the reference runtime ABI (src/card/rt.h:61-72) and its
 * load-time API (src/card/gemv.h:50-67): the same names, argument meanings, shapes and
 * output layouts. Only pointers and integers cross this interface; no HIP or torch types.
 *
 *   y = W x          rt_gemv        W [rows cols] Q8_0, x F32[cols], y F32[rows]
 *   Y = X W^T        rt_gemm        X F32[t cols] token-major, Y F32[t rows] token-major
 *
 * Q8_0 is the GGUF block: per 32 columns of a row, an IEEE binary16 scale d (2 bytes, little
 * endian) then 32 int8 q; the weight is d*q. A matrix is rows*cols/32 such 34-byte blocks,
 * row by row (src/card/gemv.c:25, 30-33).
 *
 * Weights live in HBM for the life of the process: rt_q8_upload copies a matrix's GGUF rows
 * to the GPU once and returns the handle that every later product takes as `w`, where the
 * reference took the address of its repacked form I copy (src/card/engine.c:303-316).
 * The device form ("form S", below) has the same size as GGUF and as form I, and, like form
 * I, a prefix of whole 16-row groups is the matrix of those rows: rt_gemv(R, w, 32768, ...)
 * on the handle of a 151936-row matrix is the product of its first 32768 rows.
 *
 * Form S, per 16-row group g (17*cols bytes, at g*17*cols from the handle):
 *   16*cols bytes   int8 q, row by row (row 16g+r at r*cols), columns in order
 *   cols bytes      binary16 d, row by row (row 16g+r at 16*cols + r*cols/16), blocks in order
 *
 * Shapes: rows % 16 == 0, cols % 32 == 0 (src/card/gemv.h:1-11), as the reference; cols % 4 == 0
 * also makes every row of x 16-byte aligned. A violation prints the reason and aborts: the
 * reference's entry points return nothing and do not fail partially.
 *
 * Threading: one host thread calls these, as only the card's main thread called the
 * reference's (src/card/rt.c:31-37, 274-285). The queue is a static of the library: not
 * reentrant, as the reference's is not (src/card/rt.c:216-226).
 *
 * Errors: every HIP call is checked; a failure prints the call and the HIP error and aborts.
 *
 * Waits: no call waits for the GPU without a deadline. A call that waits (for its y, a copy, the
 * stream) and sees no completion within Q8_WAIT_S seconds (60 when unset) prints what it waited
 * for and ends the process with _exit(3), as the reference's card does after about 60 s without
 * its host (src/card/link.c:17-32).
 *
 * Environment: read once, by rt_init (Q8_DEVICE, Q8_EXACT, Q8_WAIT_S, Q8_UPLOAD_CHUNK,
 * Q8_ABORT_EXIT), never on a product call; only Q8_EXACT changes a product's bits. */
#ifndef Q8_RT_H
#define Q8_RT_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

struct team;
struct gemm_chain;

/* The runtime's state, field for field the reference's (src/card/rt.h:19-26), so generated
 * code that reads R->frame, R->threads or R->last compiles unchanged. rt_init keeps the GPU
 * context (device, stream, staging buffers) behind `chain`; team and gemm_chain stay NULL. */
struct rt {
    struct team *team;
    char *frame;
    void *chain;
    struct gemm_chain *gemm_chain;
    int threads;
    int last;
};

/* ---- init (src/card/rt.h:38-39; rt.c:179-203) */

/* Once, before any product: selects the GPU (Q8_DEVICE, default 0), creates the stream and
 * the staging buffers, and reads the other settings from the environment (above). threads is
 * kept in R->threads and otherwise unused: the GPU grid replaces the team. 0, or -1 when the GPU
 * or its memory is not there. (Q8_ABORT_EXIT=n, 1..125: a caller's mistake ends the process with
 * _exit(n) instead of abort(), for harnesses that check the message in a child process.) */
int rt_init(struct rt *R, int threads);

/* Releases the stream, the staging buffers and every uploaded matrix. An addition: the
 * reference frees nothing before exit. */
void rt_fini(struct rt *R);

/* ---- products (src/card/rt.h:61-72; rt.c:205-285) */

/* y = W x. x, y host memory: x is staged in pinned host memory (the decode kernels read it there;
 * the matrix-core and reference-order products get a copy in HBM), the product stores y into
 * pinned host memory, y is copied out; returns when y is valid. (rt.c:205-214) */
void rt_gemv(struct rt *R, const void *w, long rows, long cols, const float *x, float *y);

/* Adjacent products: queue up to RT_BATCH, none reading another's result; rt_gemv_go runs them
 * all and returns when every y is valid. Queued products that share x copy it once and run as a
 * round (rt_gemv_round_dev, below).
 * (rt.h:63-69; rt.c:251-265, 274-285) */
#define RT_BATCH 8
void rt_gemv_q(struct rt *R, const void *w, long rows, long cols, const float *x, float *y);
/* Opens the round before x is ready (rt.c:267-272). Reads nothing ahead: on the MI355X a read of the
 * queued weights into the Infinity Cache while x is prepared makes the round slower, not faster
 * (the products read the bytes again). Kept so generated code links; it does nothing. */
void rt_gemv_open(struct rt *R);
void rt_gemv_go(struct rt *R);

/* Y = X W^T for t tokens: X [t cols], Y [t rows], both token-major, X rows cols apart
 * (rt.c:244-249: x_stride = cols). Returns when Y is valid. */
void rt_gemm(struct rt *R, const void *w, long rows, long cols, const float *x, long t, float *y);
/* The same, queued into the round of rt_gemv_go (rt.c:260-265). */
void rt_gemm_q(struct rt *R, const void *w, long rows, long cols, const float *x, long t, float *y);

/* ---- load time (src/card/gemv.h:50-67; gemv.c:13-52; engine.c:303-316) */

/* Bytes of the repacked form: rows/16 * cols/32 * 544, which is also the GGUF size. (gemv.c:13) */
long gemv_i_bytes(long rows, long cols);

/* GGUF Q8_0 rows (rows*cols/32 blocks of 34 B, host memory) into form S at out (host memory,
 * gemv_i_bytes(rows, cols) bytes; out must not overlap q8). The host-side analogue of the
 * reference's repack into form I (gemv.c:23-40), for callers that stage weights themselves. */
void gemv_i_repack(const uint8_t *q8, long rows, long cols, void *out);

/* GGUF Q8_0 rows in host memory to HBM, repacked there into form S by the GPU: the handle for
 * `w`. Call once per distinct tensor (tied tensors share a handle, engine.c:307-310). The
 * host buffer may be freed on return. NULL when HBM is full. */
const void *rt_q8_upload(struct rt *R, const uint8_t *q8, long rows, long cols);
/* Addition (no reference counterpart; the GGUF loader's path): the same for GGUF Q8_0 rows read
 * from an open file at byte `offset`, straight into pinned staging in chunks of whole 16-row
 * groups (64 MiB, or Q8_UPLOAD_CHUNK bytes, or rt_set_upload_chunk's), each repacked on the device while the next is read.
 * NULL when HBM is full or a read fails (errno set). */
const void *rt_q8_upload_fd(struct rt *R, int fd, uint64_t offset, long rows, long cols);
/* The same for a matrix already in form S in host memory (gemv_i_repack's output). */
const void *rt_q8_upload_packed(struct rt *R, const void *packed, long rows, long cols);
/* Frees an uploaded matrix. */
void rt_q8_free(struct rt *R, const void *w);

/* Row `row` of an uploaded matrix, dequantised: z[k] = q * d, exact (src/card/rt.h:85; rt.c:484-501,
 * the embedding read). z host memory, cols floats; returns when z is valid. Like the reference's it
 * takes no struct rt: it uses the runtime rt_init set up last. */
void rt_q8_row(const void *w, long cols, long row, float *z);

/* ---- activations already in HBM (additions: no copies, stream-ordered, no wait)
 *
 * x, y are device addresses (from rt_dev_alloc, or any HIP allocation on the device). The
 * products are enqueued on the runtime's stream in call order, so a product that reads
 * another's y sees it; rt_dev_sync waits for all of them. These are what a caller that keeps
 * its activations in HBM uses, and what the throughput figures time. */
void rt_gemv_dev(struct rt *R, const void *w, long rows, long cols, const float *x, float *y);
/* Y = X W^T, t tokens (1..64), X rows x_stride floats apart (x_stride >= cols, % 4 == 0). */
void rt_gemm_dev(struct rt *R, const void *w, long rows, long cols, const float *x, long x_stride, long t, float *y);
/* rt_gemm_dev that allocates nothing, for callers that cannot call hipMalloc (code under HIP graph
 * capture, tight serving loops, harnesses that forbid allocation). No counterpart in the reference.
 * The same kernels and the same results, bit for bit; the matrix-core product's K-split partials
 * (t >= 5) live in a static device array of the library, 32 MiB (8 Mi floats) on every GPU it runs
 * on, held until the process ends. A product whose partials would exceed it is refused with the
 * reason. Every call on a GPU shares that GPU's array: calls that overlap on one GPU (two streams,
 * two runtimes) race. */
void rt_gemm_dev_noalloc(struct rt *R, const void *w, long rows, long cols, const float *x, long x_stride, long t, float *y);
/* A round of n (1..RT_BATCH) products sharing x, none reading another's y: y[i] = X w[i]^T,
 * w[i] [rows[i] cols]. At t <= 4 one launch where the decode kernel takes the shapes; from 5
 * tokens, 64 at a time, one matrix-core launch for the products and one launch of their partial
 * sums (each product on its own K split). Each y has
 * the bits of its own single product. The device form of rt_gemv_q x n + rt_gemv_go, which uses
 * the same launches for queued products that share x (the DeltaNet quartet QKV/GATE/BETA/ALPHA,
 * src/apl/qwen35.apl:93-96; the attention layer's Q/K/V, qwen35.apl:117-119). */
void rt_gemv_round_dev(struct rt *R, int n, const void *const *w, const long *rows, long cols, const float *x, long x_stride, long t, float *const *y);
/* The FFN's fused pair: Y[k] = SiLU(G[k]) * U[k] with G = X Wg^T and U = X Wu^T, both [rows cols],
 * x read once for both; SiLU(g) = g / (1 + exp(-g)) (src/apl/qwen35.apl:38, 125). t tokens: up to
 * 4 one decode launch; from 5, 64 tokens at a time, the two products as a matrix-core round and
 * their sums with the SwiGLU in one more launch. */
void rt_gemv_swiglu_dev(struct rt *R, const void *wg, const void *wu, long rows, long cols, const float *x, long x_stride, long t, float *y);
/* ---- the epilogues on either side of a product (additions; the reference computes them on its
 * host around the products: RMS = {⍺×⍵×(RMS_EPS+(+/⍵×⍵)÷≢⍵)*¯0.5}, src/apl/qwen35.apl:49, before a
 * layer's mixer and FFN, and the residual Z←X+… after them, qwen35.apl:131-139). Fused into the
 * decode kernel (t <= 4) for K = 2048, 4096, 6144 and 12288 and the residual into the
 * matrix-core product's for t >= 5; other shapes run the norm or the add as a kernel of its own. The
 * norm is s = 1 / sqrt(eps + sum_k x[k]^2 / cols) per token in F32, xn[k] = nw[k] * (x[k] * s); its
 * sum runs in a fixed order for a given shape, so results repeat bit for bit, and a fused and a
 * separate norm differ only by that order (an ulp or so of s). The residual is one F32 add of the
 * product, the same bits fused or apart. */
/* xn = the normed x, t tokens (x rows x_stride floats apart, xn rows cols apart; xn may be x when
 * x_stride == cols); cols % 4 == 0. */
void rt_rmsnorm_dev(struct rt *R, const float *x, long x_stride, long t, long cols, const float *nw, float eps, float *xn);
/* Y = RMS(X) W^T: the normed x is never stored. */
void rt_gemm_norm_dev(struct rt *R, const void *w, long rows, long cols, const float *x, long x_stride, long t, const float *nw, float eps, float *y);
/* The fused pair on RMS(X): Y = SiLU(RMS(X) Wg^T) * (RMS(X) Wu^T) (W_PNORM RMS then the FFN, qwen35.apl:125, 132). */
void rt_gemv_swiglu_norm_dev(struct rt *R, const void *wg, const void *wu, long rows, long cols, const float *x, long x_stride, long t, const float *nw,
                             float eps, float *y);
/* A round of products sharing RMS(X) (the DeltaNet quartet on W_ANORM RMS X): at t <= 4 one
 * launch with the norm fused; from 5 tokens the norm, then the round's launches as above. */
void rt_gemv_round_norm_dev(struct rt *R, int n, const void *const *w, const long *rows, long cols, const float *x, long x_stride, long t,
                            const float *nw, float eps, float *const *y);
/* Y = R + X W^T (after W_OUT and W_DOWN); r [t rows] may be y, the residual stream updated in place. */
void rt_gemm_residual_dev(struct rt *R, const void *w, long rows, long cols, const float *x, long x_stride, long t, const float *r, float *y);
/* z[i*cols ..] = row rows[i] of w dequantised, i < n (rows: device longs, each < the matrix's
 * rows; z device). The embedding read of a batch of tokens. An addition. The indices are device
 * data the host does not see: one outside [0, rows) reads nothing and gives a row of NaN. */
void rt_q8_rows_dev(struct rt *R, const void *w, long cols, const long *rows, long n, float *z);
/* *idx (device) = the greedy next token over a[0..n) (device): the lowest i whose bits equal the
 * fmaxf fold of a, as the host's rt_maxv then rt_index_of give it (src/card/rt.c:137-165) for
 * Next = {w index-of max/w} (src/apl/qwen35.apl:161). Deterministic. An addition. */
void rt_argmax_dev(struct rt *R, const float *a, long n, long *idx);
/* Device memory for activations, and copies to and from it on the runtime's stream. rt_dev_free
 * takes any HIP allocation of the device; every buffer that rt_q8_repack_dev registered inside it
 * stops being a weight handle. */
void *rt_dev_alloc(struct rt *R, long bytes);
void rt_dev_free(struct rt *R, void *p);
void rt_dev_upload(struct rt *R, void *dst, const void *src, long bytes);
void rt_dev_download(struct rt *R, void *dst, const void *src, long bytes);
void rt_dev_sync(struct rt *R);

/* A recorded sequence of device products, replayed with one call (a HIP graph captured from
 * the runtime's stream): rt_graph_begin, then any rt_*_dev products (no host-pointer products,
 * no copies), then rt_graph_end returns the sequence; rt_graph_launch enqueues one replay on the
 * stream, in order with every other product. The pointers recorded are used as they are. */
void rt_graph_begin(struct rt *R);
void *rt_graph_end(struct rt *R);
void rt_graph_launch(struct rt *R, void *graph);
void rt_graph_free(struct rt *R, void *graph);

/* ---- host-side tests and benchmarks (additions) */

/* Synthetic GGUF Q8_0 rows written on the GPU at dst (device, rows*cols/32*34 bytes): q uniform
 * integers in [-127, 127]; d = binary16(|N(0, sigma)| / 127) when dist == 0, or
 * binary16(lognormal(mu, sigma)) when dist == 1. A function of (seed, row, block) only. */
void rt_q8_fill_dev(struct rt *R, void *dst, long rows, long cols, uint64_t seed, int dist, float mu, float sigma);
/* Form S from GGUF rows, both in HBM (the repack rt_q8_upload runs). */
void rt_q8_repack_dev(struct rt *R, const void *q8_dev, long rows, long cols, void *out_dev);
/* F32 N(0,1) values on the GPU: a function of (seed, index) only. */
void rt_f32_fill_dev(struct rt *R, float *dst, long n, uint64_t seed);
/* dst = src on the runtime's stream by a plain kernel that reads and writes every byte once
 * (16-byte aligned, bytes % 16 == 0): the yardstick the benchmark scales the HBM byte counters by. */
void rt_dev_copy(struct rt *R, void *dst, const void *src, long bytes);

/* The floor of a product (a measurement tool, like rt_dev_copy): the loads the product kernel
 * makes for Y = X W^T at t tokens (x rows x_stride floats apart), on the product's own grid, and
 * no arithmetic but a checksum.
 * t = 1 to 4, the decode kernel: every row's weights and scales, both matrices of the fused pair
 * when w1 != NULL; workgroup b stores the wrapping sum of every 32-bit word it read (scales
 * zero-extended; each workgroup reads all of x, each scale is read by two lanes) to sink[b]. For
 * the decode token's shapes at one token and the 9B verify shapes (the fused pair 12288 x 4096,
 * down 4096 x 12288) at 2 to 4; any other shape aborts.
 * t = 5 to 16, the x-resident matrix-core kernel (one matrix, w1 NULL): its grid, K split and
 * loads, every weight word and scale added once and every x word as loaded (each workgroup reads
 * its K range of x), each workgroup adding its sum to sink[0] (zero it first). Any shape the
 * product takes.
 * sink: device, `rows` unsigned (the entries past the grid are not written). */
void rt_q8_read_dev(struct rt *R, const void *w0, const void *w1, long rows, long cols, const float *x, long x_stride, long t, unsigned *sink);

/* The product kernels' primitive conversions on the GPU, lane by lane: o8[i] = fma(x8[i],
 * (float)q[i], c8[i]) with the int8 convert of the weights (n8 % 4 == 0), of[i] = fma(xf[i],
 * (float)binary16 h[i], cf[i]) with the scale convert; all device arrays. The reference's
 * gate 2.1 s8 and f16 sets (src/gate/upconv_kernel.c:18-22, 51-55) hash these. */
void rt_prims_dev(struct rt *R, const int8_t *q, const float *x8, const float *c8, float *o8, long n8, const uint16_t *h, const float *xf,
                  const float *cf, float *of, long nf);

/* Product kernels: 0 = the fast kernels (default), 1 = the reference-order kernels, whose every
 * y is bit-identical to the reference's F32 host path (src/card/gemv.c:165-193 at one thread;
 * gemm.c:20-23 per token). Returns the previous mode. Q8_EXACT=1 in the environment sets 1.
 *
 * In the fast kernels a token's y does not depend on how many tokens it was computed with, within
 * t = 1..4 (the decode kernels) and within t >= 5 (the matrix-core product, whose K split is a
 * function of the matrix's shape alone); across the two it differs within the parity bar. The
 * reference-order kernels keep the reference's gemm(t)[k] == gemv(x[k]) (src/card/gemm.h:5-7) at
 * every t. */
int rt_set_exact(struct rt *R, int exact);

/* Measurement and test settings (additions), each returning the previous value where it has one:
 * rt_set_epi_apart(R, 1) runs every epilogue as a kernel of its own (the norm's sum then in that
 * kernel's order: an ulp or so of its scale; the residual the same bits); rt_set_upload_chunk sets
 * the upload's chunk in bytes (whole 16-row groups; the bits do not change); rt_set_x_direct(R, 0)
 * makes the host-pointer calls copy x to HBM before their decode products instead of letting the
 * kernels read it from pinned host memory (the default, 1; the same bits); rt_gemm_force makes
 * the matrix-core product use `ks` K splits (0: the planner's; other splits, other bits) and, with
 * streaming != 0, the streaming kernel for one token tile instead of the x-resident one (the same
 * sums). */
int rt_set_epi_apart(struct rt *R, int apart);
int rt_set_x_direct(struct rt *R, int direct);
long rt_set_upload_chunk(struct rt *R, long bytes);
void rt_gemm_force(struct rt *R, int streaming, int ks);

/* Event timing on the runtime's stream: rt_timer_start, then rt_timer_stop returns the
 * milliseconds between them (waits for the stream). */
void rt_timer_start(struct rt *R);
float rt_timer_stop(struct rt *R);

/* Kernel timing, for the benchmark: while on, every product records its (first) kernel's own
 * start and end (events attached to the kernel's dispatch), up to 16384 products; rt_ktime_read
 * waits for the stream and returns how many it filled: the kind (RT_K_*), the shape, the kernel's
 * duration in microseconds, its name as rocprof prints it (64 bytes each in names, NUL-padded;
 * names may be NULL) and its grid in threads (grid may be NULL); reading clears the records.
 * rt_ktime(R, 1) also clears. */
#define RT_K_GEMV 0      /* t <= 4, the decode kernels */
#define RT_K_GEMV_PAIR 1 /* the fused gate/up pair, t <= 4 */
#define RT_K_GEMM 2      /* t >= 5, the matrix-core kernel */
#define RT_K_GEMM_PAIR 3
#define RT_K_EXACT 4 /* the reference-order kernel */
#define RT_K_ROUND 5 /* a round of products sharing x, one launch (rows: their sum) */
void rt_ktime(struct rt *R, int on);
long rt_ktime_read(struct rt *R, int *kind, long *rows, long *cols, long *t, float *us, char *names, long *grid, long max);

/* The host-pointer calls' own time, for the benchmark (an addition): while on, every call that
 * waits for its y (rt_gemv, rt_gemm, rt_gemv_go, rt_q8_row's wait excepted) adds, in microseconds of
 * host time, its phases to us[]: RT_HT_STAGE x into the pinned staging, RT_HT_LAUNCH the launches
 * (x's copy, the products, the completion flag), RT_HT_WAIT until the flag is seen, RT_HT_COPY_OUT
 * y out of the pinned staging; rt_host_timing_read returns the number of calls summed.
 * rt_host_timing(R, on) also clears the sums. */
#define RT_HT_STAGE 0
#define RT_HT_LAUNCH 1
#define RT_HT_WAIT 2
#define RT_HT_COPY_OUT 3
#define RT_HT_PHASES 4
void rt_host_timing(struct rt *R, int on);
long rt_host_timing_read(struct rt *R, double *us);

/* The device's name and its count of compute units, for reports. */
void rt_device_info(struct rt *R, char *name, long name_len, int *cus);

#ifdef __cplusplus
}
#endif

#endif
