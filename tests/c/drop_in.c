/* drop_in.c: a C caller of the Q8_0 products written against include/q8_rt.h alone, the way the
 * reference's generated code calls its runtime (src/apl/compiler/em.apl:601-617, 1044-1045):
 * rt_init, weights uploaded once, then rt_gemv; rt_gemv_q x4 sharing x with open/go (the DeltaNet
 * quartet, src/apl/qwen35.apl:93-96); rt_gemm for t tokens. Checks, on synthetic weights:
 *   - exact mode: every y bit-identical to the reference's fold order, computed here in plain C;
 *   - gemm(t)[k] == gemv(x[k]) bit for bit in exact mode (scripts/check.sh:132-149);
 *   - fast mode: within NRMSE 1e-5 of an F64 sum.
 * Prints PASS/FAIL lines; exit 0 only if all pass. Needs the GPU. */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "q8_rt.h"

static unsigned s = 12345u;
static unsigned xs(void)
{
    s ^= s << 13;
    s ^= s >> 17;
    s ^= s << 5;
    return s;
}

static float half_to_float(uint16_t h)
{
    unsigned sign = (unsigned)(h >> 15) << 31, e = (h >> 10) & 31u, m = h & 1023u, u;
    float f;
    if (e == 31)
        u = sign | 0x7f800000u | m << 13;
    else if (e)
        u = sign | (e + 112u) << 23 | m << 13;
    else {
        f = ldexpf((float)m, -24);
        return sign ? -f : f;
    }
    memcpy(&f, &u, 4);
    return f;
}

/* binary16 of a small positive value, by truncation (the test needs only valid scales) */
static uint16_t to_half(float v)
{
    unsigned u;
    memcpy(&u, &v, 4);
    int e = (int)((u >> 23) & 255) - 127 + 15;
    if (e <= 0)
        return (uint16_t)((u & 0x7fffff) | 0x800000) >> (14 - e);
    return (uint16_t)(e << 10 | ((u >> 13) & 1023));
}

static void make(uint8_t *q8, long rows, long cols)
{
    for (long b = 0; b < rows * cols / 32; b++) {
        uint16_t d = to_half((float)(xs() % 1000 + 1) * 2e-7f);
        memcpy(q8 + 34 * b, &d, 2);
        for (int i = 0; i < 32; i++)
            q8[34 * b + 2 + i] = (uint8_t)(int8_t)((int)(xs() % 255) - 127);
    }
}

static void ref_fold(const uint8_t *q8, long rows, long cols, const float *x, float *y)
{
    for (long r = 0; r < rows; r++) {
        float acc = 0.0f;
        for (long b = 0; b < cols / 32; b++) {
            const uint8_t *blk = q8 + (r * (cols / 32) + b) * 34;
            float t = 0.0f;
            for (int i = 0; i < 32; i++)
                t = fmaf((float)(int8_t)blk[2 + i], x[32 * b + i], t);
            acc = fmaf(t, half_to_float((uint16_t)(blk[0] | blk[1] << 8)), acc);
        }
        y[r] = acc;
    }
}

static double nrmse64(const uint8_t *q8, long rows, long cols, const float *x, const float *y)
{
    double num = 0, den = 0;
    for (long r = 0; r < rows; r++) {
        double acc = 0;
        for (long b = 0; b < cols / 32; b++) {
            const uint8_t *blk = q8 + (r * (cols / 32) + b) * 34;
            for (int i = 0; i < 32; i++)
                acc += (double)half_to_float((uint16_t)(blk[0] | blk[1] << 8)) * (int8_t)blk[2 + i] * x[32 * b + i];
        }
        num += (y[r] - acc) * (y[r] - acc);
        den += acc * acc;
    }
    return sqrt(num / den);
}

static int fails;
static void check(int ok, const char *what)
{
    printf("%s  %s\n", ok ? "PASS" : "FAIL", what);
    fails += !ok;
}

int main(void)
{
    struct rt R;
    memset(&R, 0, sizeof R);
    if (rt_init(&R, 1) != 0) {
        printf("FAIL  rt_init: no GPU\n");
        return 1;
    }
    const long rows = 256, cols = 1024, T = 6;
    uint8_t *q8[4];
    const void *w[4];
    for (int k = 0; k < 4; k++) {
        q8[k] = malloc((size_t)gemv_i_bytes(rows, cols));
        make(q8[k], rows, cols);
        w[k] = rt_q8_upload(&R, q8[k], rows, cols);
    }
    float *x = malloc(sizeof(float) * (size_t)(cols * T)), *y = malloc(sizeof(float) * (size_t)(rows * T));
    float *want = malloc(sizeof(float) * (size_t)(rows * T)), *yq[4];
    for (long i = 0; i < cols * T; i++)
        x[i] = (float)((int)(xs() % 20001) - 10000) * 1e-4f;
    for (int k = 0; k < 4; k++)
        yq[k] = malloc(sizeof(float) * (size_t)rows);

    rt_set_exact(&R, 1);
    ref_fold(q8[0], rows, cols, x, want);
    rt_gemv(&R, w[0], rows, cols, x, y);
    check(memcmp(y, want, sizeof(float) * (size_t)rows) == 0, "exact rt_gemv == the reference fold, bit for bit");
    rt_gemm(&R, w[0], rows, cols, x, T, y);
    int same = 1;
    for (long k = 0; k < T; k++) {
        float one[256];
        rt_gemv(&R, w[0], rows, cols, x + k * cols, one);
        same &= memcmp(one, y + k * rows, sizeof one) == 0;
    }
    check(same, "exact rt_gemm(t=6)[k] == rt_gemv(x[k]), bit for bit");
    rt_gemv_open(&R);
    for (int k = 0; k < 4; k++)
        rt_gemv_q(&R, w[k], rows, cols, x, yq[k]);
    rt_gemv_go(&R);
    same = 1;
    for (int k = 0; k < 4; k++) {
        ref_fold(q8[k], rows, cols, x, want);
        same &= memcmp(yq[k], want, sizeof(float) * (size_t)rows) == 0;
    }
    check(same, "exact queued round of 4 sharing x == the reference fold");

    rt_set_exact(&R, 0);
    rt_gemv(&R, w[1], rows, cols, x, y);
    check(nrmse64(q8[1], rows, cols, x, y) <= 1e-5, "fast rt_gemv within NRMSE 1e-5 of F64");
    rt_gemm(&R, w[2], rows, cols, x, T, y);
    int ok = 1;
    for (long k = 0; k < T; k++)
        ok &= nrmse64(q8[2], rows, cols, x + k * cols, y + k * rows) <= 1e-5;
    check(ok, "fast rt_gemm(t=6) within NRMSE 1e-5 of F64 per token");
    rt_fini(&R);
    printf("%s\n", fails ? "FAILED" : "ALL PASS");
    return fails != 0;
}
