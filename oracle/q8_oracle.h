/* q8_oracle.h: the CPU oracle of the Q8_0 weight products. TEST INFRASTRUCTURE ONLY: the
 * tests, the smoke check and the benchmark's CPU-baseline leg call it as the checker; no
 * product path reads, links or runs anything here.
 *
 * A restatement, in this file's own code, of the reference's F32 host C path for
 *   gemv: y = W x             (src/card/gemv.c:165-193, 244-257 at one thread)
 *   gemm: Y = X W^T per token (src/card/gemm.c:20-23, 188-200, 241-255)
 * with the host model's rounding (src/card/knc.h:159-173, 195-201, 230-243): one fmaf per
 * step, int8 -> binary32 and binary16 -> binary32 exact. For every row r:
 *   T(r,b) = fold over i = 0..31 of  T = fmaf((float)q[r][32b+i], x[32b+i], T)   from +0
 *   y[r]   = fold over b = 0..cols/32-1 of  acc = fmaf(T(r,b), half(d[r][b]), acc)   from +0
 * plus the F64 closed form y[r] = sum over k of (double)d*q * (double)x[k] (the meaning of
 * W+.x x in the GNU APL F64 reference, src/apl/gguf_read.apl:37-46; tests/host/gguf_rows.c:45-58).
 *
 * What pins each function (the tests hold each to it):
 *   q8o_half         all 65536 binary16 patterns against numpy's float16 -> float32, and the
 *                    reference's gate 2.1 f16 hash (tests/golden/gate-2.1.txt:6)
 *   q8o_gate_a       the reference's gate A line (tests/golden/gate-a.txt:1)
 *   q8o_gate21       the reference's gate 2.1 hash lines (tests/golden/gate-2.1.txt:1-7)
 *   q8o_gemv/gemm    bit for bit against the reference's own gemv.c/gemm.c compiled from its
 *                    sources (oracle/_ref) and against fixtures made from that build
 *                    (tests/golden/ref_products.npz); against the F64 closed form within F32
 *                    error; x = e_j gives column j of d*q exactly; zero scales give +0
 *   q8o_gemv_f64     brute force on tiny shapes in exact rational arithmetic (Python
 *                    fractions) and linearity in x
 *   q8o_repack_s     the device form's definition checked byte by byte on tiny shapes
 *                    against an independent index formula in the tests
 *   q8o_row          bit for bit against the reference's rt_q8_row on form I (oracle/_ref),
 *                    and against numpy's d * q
 *   q8o_next         against the reference's rt_maxv + rt_index_of (oracle/_ref) on random,
 *                    tied, NaN-holding and ragged arrays, and numpy's nanargmax
 *   q8o_rmsnorm_f64  against the reference's own F32 norm composed from its host rt_sum,
 *                    rt_s_div, rt_s_add and rt_s_rsqrt (oracle/_ref) within F32 error; a constant
 *                    vector's closed form; scale invariance and unit RMS at eps = 0
 *   q8o_gemm_f64d    equal to q8o_gemm_f64 on F32-representable x; linearity in x
 * Nothing here is "parity unpinned". */
#ifndef Q8_ORACLE_H
#define Q8_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* IEEE binary16 -> binary32, exact for every pattern (knc.h:159-173). */
float q8o_half(uint16_t h);

/* The reference's F32 order, one row at a time; x rows x_stride floats apart. */
void q8o_gemv(const uint8_t *q8, long rows, long cols, const float *x, float *y);
void q8o_gemm(const uint8_t *q8, long rows, long cols, const float *x, long x_stride, long t, float *y);
/* The same on `threads` pthreads, each a contiguous range of 16-row groups: the same bits at
 * any thread count (gemv.h:1-5). Threads pinned to the first `threads` CPUs this process may
 * use. For the CPU baseline. */
void q8o_gemm_mt(const uint8_t *q8, long rows, long cols, const float *x, long x_stride, long t, float *y, int threads);

/* F64 closed form, Y [t rows]. */
void q8o_gemm_f64(const uint8_t *q8, long rows, long cols, const float *x, long x_stride, long t, double *y);

/* The same with F64 x (the product of a normed x, which is not an F32 vector). */
void q8o_gemm_f64d(const uint8_t *q8, long rows, long cols, const double *x, long t, double *y);

/* The RMS norm in F64 (src/apl/qwen35.apl:49, RMS←{⍺×⍵×(RMS_EPS+(+/⍵×⍵)÷≢⍵)*¯0.5}), per token:
 * xn[i][k] = nw[k] * (x[i][k] * (eps + sum_k x[i][k]^2 / cols)^-0.5); x rows x_stride apart, xn
 * rows cols apart. */
void q8o_rmsnorm_f64(const float *x, long x_stride, long t, long cols, const float *nw, double eps, double *xn);

/* SiLU(g) * u in F64 (src/apl/qwen35.apl:38; docs/model.md:29: Sig = 1 / (1 + exp(min(700, -g)))). */
void q8o_swiglu_f64(const double *g, const double *u, long n, double *y);

/* Row `row` of GGUF Q8_0 rows dequantised: z[k] = (float)q * half(d), one rounding, exact
 * (src/card/rt.c:484-501). */
void q8o_row(const uint8_t *q8, long cols, long row, float *z);
/* The greedy next token (src/card/rt.c:137-165, rt_maxv then rt_index_of; src/apl/qwen35.apl:161):
 * m = fmaxf fold of a from a[0], then the lowest i whose bits equal m's (n when none). */
long q8o_next(const float *a, long n);

/* Form S (include/q8_rt.h): per 16-row group, 16*cols int8 row by row, then 16 rows of
 * cols/32 binary16 scales. */
void q8o_repack_s(const uint8_t *q8, long rows, long cols, uint8_t *out);

/* Gate A (src/gate/gate_common.h, fma_ref.c): out[0] = FNV-1a hash of C after C = fmaf(A, B, C),
 * out[1..3] = bits of C[0], C[1], C[4095]. */
void q8o_gate_a(uint64_t out[4]);
/* Gate 2.1 (src/gate/upconv_common.h, upconv_cmp.c): the 7 hashes in file order
 * s8, u8fma, u8mul, b16, bcast, f16, hsum. */
void q8o_gate21(uint64_t out[7]);
/* Gate 2.1's inputs, for the GPU run of the same conversions: q[512], h[131072],
 * x8/c8[512], xf/cf[131072]. */
void q8o_gate21_inputs(int8_t *q, uint16_t *h, float *x8, float *c8, float *xf, float *cf);
/* Gate 2.1's s8 lanes (512) and f16 lanes (131072) themselves. */
void q8o_gate21_arrays(float *s8, float *f16);
/* FNV-1a over the 32-bit words of n floats (gate_common.h). */
uint64_t q8o_hash(const float *v, long n);

#ifdef __cplusplus
}
#endif

#endif
