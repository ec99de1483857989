/* q8_oracle.c: see q8_oracle.h. TEST INFRASTRUCTURE ONLY (the checker, never the product).
 * Built with -O2 -ffp-contract=off (the reference's host flags, scripts/lib.sh:37): every
 * rounding below is written out, one fmaf per step. */
#define _GNU_SOURCE
#include "q8_oracle.h"

#include <math.h>
#include <pthread.h>
#include <sched.h>
#include <stdlib.h>
#include <string.h>

#define BLOCK 32
#define GROUP 16
#define BLOCK_BYTES 34

/* knc.h:159-173: sign, exponent and mantissa moved into place; a subnormal binary16 is
 * m * 2^-24, exact in binary32; inf and NaN keep their payload. */
float q8o_half(uint16_t h)
{
    uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31u, m = h & 1023u, u;
    float f;
    if (e == 31) {
        u = s | 0x7f800000u | m << 13;
    } else if (e != 0) {
        u = s | (e + 112u) << 23 | m << 13;
    } else {
        f = ldexpf((float)m, -24);
        return s ? -f : f;
    }
    memcpy(&f, &u, 4);
    return f;
}

static inline float block_scale(const uint8_t *blk)
{
    return q8o_half((uint16_t)(blk[0] | blk[1] << 8));
}

/* One row in the reference's order (gemv.c:166-193 over all blocks of the row, whole groups):
 * per block T from +0 by 32 fmaf in column order, then acc = fmaf(T, d, acc). */
static float row_product(const uint8_t *row, long nb, const float *x)
{
    float acc = 0.0f;
    for (long b = 0; b < nb; b++) {
        const uint8_t *blk = row + b * BLOCK_BYTES;
        const int8_t *q = (const int8_t *)(blk + 2);
        const float *xb = x + b * BLOCK;
        float t = 0.0f;
        for (int i = 0; i < BLOCK; i++)
            t = fmaf((float)q[i], xb[i], t);
        acc = fmaf(t, block_scale(blk), acc);
    }
    return acc;
}

void q8o_gemv(const uint8_t *q8, long rows, long cols, const float *x, float *y)
{
    q8o_gemm(q8, rows, cols, x, cols, 1, y);
}

/* gemm.c gives every token the same operations in the same order as gemv's (gemm.h:6-7), so
 * token k's row is row_product of x[k]; Y is token-major, Y[k*rows + r] (gemm.c:209). */
static void gemm_rows(const uint8_t *q8, long r0, long r1, long rows, long cols, const float *x, long x_stride, long t, float *y)
{
    const long nb = cols / BLOCK, row_bytes = nb * BLOCK_BYTES;
    for (long k = 0; k < t; k++)
        for (long r = r0; r < r1; r++)
            y[k * rows + r] = row_product(q8 + r * row_bytes, nb, x + k * x_stride);
}

void q8o_gemm(const uint8_t *q8, long rows, long cols, const float *x, long x_stride, long t, float *y)
{
    gemm_rows(q8, 0, rows, rows, cols, x, x_stride, t, y);
}

struct mt_job {
    const uint8_t *q8;
    long rows, cols, x_stride, t;
    const float *x;
    float *y;
    int tid, n, cpu;
};

static void *mt_main(void *arg)
{
    const struct mt_job *j = arg;
    if (j->cpu >= 0) {
        cpu_set_t s;
        CPU_ZERO(&s);
        CPU_SET((size_t)j->cpu, &s);
        sched_setaffinity(0, sizeof s, &s);
    }
    const long ng = j->rows / GROUP;
    gemm_rows(j->q8, ng * j->tid / j->n * GROUP, ng * (j->tid + 1) / j->n * GROUP, j->rows, j->cols, j->x, j->x_stride, j->t, j->y);
    return NULL;
}

void q8o_gemm_mt(const uint8_t *q8, long rows, long cols, const float *x, long x_stride, long t, float *y, int threads)
{
    if (threads < 1)
        threads = 1;
    /* the CPUs this process may run on, in order: worker i on the i-th of them */
    cpu_set_t allowed;
    int cpus[1024], ncpu = 0;
    CPU_ZERO(&allowed);
    if (sched_getaffinity(0, sizeof allowed, &allowed) == 0)
        for (int c = 0; c < CPU_SETSIZE && ncpu < 1024; c++)
            if (CPU_ISSET((size_t)c, &allowed))
                cpus[ncpu++] = c;
    struct mt_job *jobs = calloc((size_t)threads, sizeof *jobs);
    pthread_t *th = calloc((size_t)threads, sizeof *th);
    if (!jobs || !th)
        abort();
    for (int i = 0; i < threads; i++) {
        jobs[i] = (struct mt_job){.q8 = q8, .rows = rows, .cols = cols, .x_stride = x_stride, .t = t, .x = x, .y = y, .tid = i, .n = threads,
                                  .cpu = i < ncpu ? cpus[i] : -1};
        if (i > 0 && pthread_create(&th[i], NULL, mt_main, &jobs[i]) != 0)
            abort();
    }
    /* the caller is worker 0 and keeps its own affinity */
    jobs[0].cpu = -1;
    mt_main(&jobs[0]);
    for (int i = 1; i < threads; i++)
        pthread_join(th[i], NULL);
    free(jobs);
    free(th);
}

void q8o_gemm_f64(const uint8_t *q8, long rows, long cols, const float *x, long x_stride, long t, double *y)
{
    const long nb = cols / BLOCK, row_bytes = nb * BLOCK_BYTES;
    for (long k = 0; k < t; k++) {
        const float *xk = x + k * x_stride;
        for (long r = 0; r < rows; r++) {
            const uint8_t *row = q8 + r * row_bytes;
            double s = 0.0;
            for (long b = 0; b < nb; b++) {
                const double d = (double)block_scale(row + b * BLOCK_BYTES);
                const int8_t *q = (const int8_t *)(row + b * BLOCK_BYTES + 2);
                for (int i = 0; i < BLOCK; i++)
                    s += d * (double)q[i] * (double)xk[b * BLOCK + i];
            }
            y[k * rows + r] = s;
        }
    }
}

void q8o_gemm_f64d(const uint8_t *q8, long rows, long cols, const double *x, long t, double *y)
{
    const long nb = cols / BLOCK, row_bytes = nb * BLOCK_BYTES;
    for (long k = 0; k < t; k++) {
        const double *xk = x + k * cols;
        for (long r = 0; r < rows; r++) {
            const uint8_t *row = q8 + r * row_bytes;
            double s = 0.0;
            for (long b = 0; b < nb; b++) {
                const double d = (double)block_scale(row + b * BLOCK_BYTES);
                const int8_t *q = (const int8_t *)(row + b * BLOCK_BYTES + 2);
                for (int i = 0; i < BLOCK; i++)
                    s += d * (double)q[i] * xk[b * BLOCK + i];
            }
            y[k * rows + r] = s;
        }
    }
}

void q8o_rmsnorm_f64(const float *x, long x_stride, long t, long cols, const float *nw, double eps, double *xn)
{
    for (long i = 0; i < t; i++) {
        const float *xi = x + i * x_stride;
        double ss = 0.0;
        for (long k = 0; k < cols; k++)
            ss += (double)xi[k] * (double)xi[k];
        const double s = 1.0 / sqrt(eps + ss / (double)cols);
        for (long k = 0; k < cols; k++)
            xn[i * cols + k] = (double)nw[k] * ((double)xi[k] * s);
    }
}

void q8o_swiglu_f64(const double *g, const double *u, long n, double *y)
{
    for (long i = 0; i < n; i++) {
        const double e = -g[i] < 700.0 ? -g[i] : 700.0;
        y[i] = g[i] / (1.0 + exp(e)) * u[i];
    }
}

void q8o_repack_s(const uint8_t *q8, long rows, long cols, uint8_t *out)
{
    const long nb = cols / BLOCK, row_bytes = nb * BLOCK_BYTES, group_bytes = GROUP * cols + GROUP * nb * 2;
    for (long r = 0; r < rows; r++) {
        uint8_t *grp = out + (r / GROUP) * group_bytes;
        uint8_t *qdst = grp + (r % GROUP) * cols;
        uint8_t *ddst = grp + GROUP * cols + (r % GROUP) * nb * 2;
        for (long b = 0; b < nb; b++) {
            const uint8_t *blk = q8 + r * row_bytes + b * BLOCK_BYTES;
            memcpy(qdst + b * BLOCK, blk + 2, BLOCK);
            memcpy(ddst + b * 2, blk, 2);
        }
    }
}

/* ---- the reference's primitive gates: inputs from xorshift32, the top 24 bits as a signed
 * integer scaled by 2^-23 (src/gate/gate_common.h:14-37), results hashed by FNV-1a over their
 * 32-bit words (gate_common.h:46-55). The input order is the reference's, so the hashes are
 * comparable with its golden files. */

static uint32_t xs32(uint32_t *s)
{
    uint32_t v = *s;
    v ^= v << 13;
    v ^= v >> 17;
    v ^= v << 5;
    return *s = v;
}

static float unit24(uint32_t *s)
{
    const int32_t v = (int32_t)(xs32(s) >> 8) - 8388608;
    return (float)v * (1.0f / 8388608.0f);
}

static uint32_t bits(float f)
{
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

uint64_t q8o_hash(const float *v, long n)
{
    uint64_t h = 0xcbf29ce484222325ull;
    for (long i = 0; i < n; i++) {
        h ^= bits(v[i]);
        h *= 0x100000001b3ull;
    }
    return h;
}

#define GATE_N 4096
void q8o_gate_a(uint64_t out[4])
{
    static float a[GATE_N], b[GATE_N], c[GATE_N];
    uint32_t s = 0x9E3779B9u;
    for (int i = 0; i < GATE_N; i++) {
        a[i] = unit24(&s);
        b[i] = unit24(&s);
        c[i] = unit24(&s);
    }
    for (int i = 0; i < GATE_N; i++)
        c[i] = fmaf(a[i], b[i], c[i]);
    out[0] = q8o_hash(c, GATE_N);
    out[1] = bits(c[0]);
    out[2] = bits(c[1]);
    out[3] = bits(c[GATE_N - 1]);
}

#define N8 512
#define NB 4096
#define NF 131072
#define NH 4096

struct g21 {
    int8_t q[N8];
    uint8_t u[N8];
    uint16_t h[NF];
    float x8[N8], c8[N8], xb[NB], cb[NB], s[NB / 16], xf[NF], cf[NF], xh[NH];
};

/* src/gate/upconv_common.h:62-89, in its order of draws */
static void g21_fill(struct g21 *in)
{
    uint32_t s = 0x2545F491u;
    memset(in, 0, sizeof *in);
    for (int i = 0; i < N8; i++) {
        const int half = i >= 256;
        in->q[i] = (int8_t)(uint8_t)i;
        in->u[i] = (uint8_t)i;
        in->x8[i] = half ? unit24(&s) : 1.0f;
        in->c8[i] = half ? unit24(&s) : 0.0f;
    }
    for (int i = 0; i < NF; i++) {
        const int half = i >= 65536;
        in->h[i] = (uint16_t)i;
        in->xf[i] = half ? unit24(&s) : 1.0f;
        in->cf[i] = half ? unit24(&s) : 0.0f;
    }
    for (int i = 0; i < NB; i++) {
        in->xb[i] = unit24(&s);
        in->cb[i] = unit24(&s);
    }
    for (int i = 0; i < NB / 16; i++)
        in->s[i] = unit24(&s);
    for (int i = 0; i < NH; i++) {
        const float m = unit24(&s);
        const uint32_t p2 = (uint32_t)(127 + (int)(xs32(&s) % 41u) - 20) << 23;
        float f;
        memcpy(&f, &p2, 4);
        in->xh[i] = m * f;
    }
}

void q8o_gate21_inputs(int8_t *q, uint16_t *h, float *x8, float *c8, float *xf, float *cf)
{
    struct g21 *in = malloc(sizeof *in);
    if (!in)
        abort();
    g21_fill(in);
    memcpy(q, in->q, sizeof in->q);
    memcpy(h, in->h, sizeof in->h);
    memcpy(x8, in->x8, sizeof in->x8);
    memcpy(c8, in->c8, sizeof in->c8);
    memcpy(xf, in->xf, sizeof in->xf);
    memcpy(cf, in->cf, sizeof in->cf);
    free(in);
}

/* the pairing i^1, i^2, i^4, i^8 of the 16-lane sum (knc.h:244-253) */
static float tree16(const float *x)
{
    float v[16], t[16];
    memcpy(v, x, sizeof v);
    for (int k = 1; k < 16; k <<= 1) {
        for (int i = 0; i < 16; i++)
            t[i] = v[i] + v[i ^ k];
        memcpy(v, t, sizeof v);
    }
    return v[0];
}

void q8o_gate21_arrays(float *s8, float *f16)
{
    struct g21 *in = malloc(sizeof *in);
    if (!in)
        abort();
    g21_fill(in);
    for (int i = 0; i < N8; i++)
        s8[i] = fmaf(in->x8[i], (float)in->q[i], in->c8[i]);
    for (int i = 0; i < NF; i++)
        f16[i] = fmaf(in->xf[i], q8o_half(in->h[i]), in->cf[i]);
    free(in);
}

void q8o_gate21(uint64_t out[7])
{
    struct g21 *in = malloc(sizeof *in);
    float *s8 = malloc(sizeof(float) * N8), *u8fma = malloc(sizeof(float) * N8), *u8mul = malloc(sizeof(float) * N8);
    float *b16 = malloc(sizeof(float) * NB), *f16 = malloc(sizeof(float) * NF), *hs = malloc(sizeof(float) * NH / 16);
    if (!in || !s8 || !u8fma || !u8mul || !b16 || !f16 || !hs)
        abort();
    g21_fill(in);
    for (int i = 0; i < N8; i++) {
        s8[i] = fmaf(in->x8[i], (float)in->q[i], in->c8[i]);
        u8fma[i] = fmaf(in->x8[i], (float)in->u[i], in->c8[i]);
        volatile float p = in->x8[i] * (float)in->u[i];
        u8mul[i] = p + in->c8[i];
    }
    for (int i = 0; i < NB; i++)
        b16[i] = fmaf(in->xb[i], in->s[i / 16], in->cb[i]);
    for (int i = 0; i < NF; i++)
        f16[i] = fmaf(in->xf[i], q8o_half(in->h[i]), in->cf[i]);
    for (int b = 0; b < NH / 16; b++)
        hs[b] = tree16(in->xh + 16 * b);
    out[0] = q8o_hash(s8, N8);
    out[1] = q8o_hash(u8fma, N8);
    out[2] = q8o_hash(u8mul, N8);
    out[3] = q8o_hash(b16, NB);
    out[4] = out[3]; /* bcast: the same products by another instruction (upconv_cmp.c:56) */
    out[5] = q8o_hash(f16, NF);
    out[6] = q8o_hash(hs, NH / 16);
    free(in);
    free(s8);
    free(u8fma);
    free(u8mul);
    free(b16);
    free(f16);
    free(hs);
}

/* rt.c:484-501: the block's q converted to F32 and multiplied by the block scale (fma(1, d, +0)
 * = d exactly), one rounding per weight, which is exact. */
void q8o_row(const uint8_t *q8, long cols, long row, float *z)
{
    const long nb = cols / BLOCK;
    const uint8_t *r = q8 + row * nb * BLOCK_BYTES;
    for (long b = 0; b < nb; b++) {
        const float d = block_scale(r + b * BLOCK_BYTES);
        const int8_t *q = (const int8_t *)(r + b * BLOCK_BYTES + 2);
        for (int i = 0; i < BLOCK; i++)
            z[b * BLOCK + i] = (float)q[i] * d;
    }
}

/* rt.c:137-150 (rt_maxv: fmaxf from a[0]) then rt.c:153-165 (rt_index_of: bit-identical match,
 * the lowest index). */
long q8o_next(const float *a, long n)
{
    float m = a[0];
    for (long i = 0; i < n; i++)
        m = fmaxf(m, a[i]);
    uint32_t want;
    memcpy(&want, &m, 4);
    for (long i = 0; i < n; i++) {
        uint32_t got;
        memcpy(&got, a + i, 4);
        if (got == want)
            return i;
    }
    return n;
}
