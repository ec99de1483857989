/* drop_in.c: a C caller of the Q8_0 products written against include/q8_rt.h alone, the way the
 * reference's generated code calls its runtime (src/apl/compiler/em.apl:601-617, 1044-1045):
 * rt_init, weights uploaded once, then rt_gemv; rt_gemv_q x4 sharing x with open/go (the DeltaNet
 * quartet, src/apl/qwen35.apl:93-96); rt_gemm for t tokens. Checks, on synthetic weights:
 *   - exact mode: every y bit-identical to the reference's fold order, computed here in plain C;
 *   - gemm(t)[k] == gemv(x[k]) bit for bit in exact mode (scripts/check.sh:132-149);
 *   - fast mode: within NRMSE 1e-5 of an F64 sum;
 *   - include/q8_gguf.h: a GGUF v3 file written here (two Q8_0 tensors and a third tied to the
 *     first by offset) read and uploaded; the tie shares one handle, and the uploaded matrices give
 *     the reference fold of the rows written.
 * Prints PASS/FAIL lines; exit 0 only if all pass. Needs the GPU. */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <unistd.h>

#include "q8_gguf.h"
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

/* GGUF v3 pieces: little-endian integers, u64-length strings */
static void put_u32(FILE *f, uint32_t v) { fwrite(&v, 4, 1, f); }
static void put_u64(FILE *f, uint64_t v) { fwrite(&v, 8, 1, f); }
static void put_str(FILE *f, const char *s)
{
    put_u64(f, strlen(s));
    fwrite(s, 1, strlen(s), f);
}

/* A file with one key and tensors "a" (data a), "b" (data b) and "a.tied" (a's offset), all
 * rows x cols Q8_0; the data start at a multiple of 32. */
static int write_gguf(const char *path, const uint8_t *a, const uint8_t *b, long rows, long cols)
{
    FILE *f = fopen(path, "wb");
    if (!f)
        return -1;
    const uint64_t bytes = (uint64_t)gemv_i_bytes(rows, cols), off_b = (bytes + 31) / 32 * 32;
    fwrite("GGUF", 1, 4, f);
    put_u32(f, 3);
    put_u64(f, 3); /* tensors */
    put_u64(f, 1); /* keys */
    put_str(f, "general.architecture");
    put_u32(f, 8); /* string */
    put_str(f, "qwen35");
    const char *names[3] = {"a", "b", "a.tied"};
    const uint64_t offs[3] = {0, off_b, 0};
    for (int i = 0; i < 3; i++) {
        put_str(f, names[i]);
        put_u32(f, 2);
        put_u64(f, (uint64_t)cols);
        put_u64(f, (uint64_t)rows);
        put_u32(f, 8); /* Q8_0 */
        put_u64(f, offs[i]);
    }
    for (long pos = ftell(f); pos % 32; pos++)
        fputc(0, f);
    fwrite(a, 1, bytes, f);
    for (uint64_t k = bytes; k < off_b; k++)
        fputc(0, f);
    fwrite(b, 1, bytes, f);
    return fclose(f);
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

    char path[] = "/tmp/q8_drop_in_XXXXXX";
    const int fd = mkstemp(path);
    struct rt_gguf g;
    char err[512] = "";
    ok = fd >= 0 && write_gguf(path, q8[0], q8[3], rows, cols) == 0 && rt_gguf_read(&g, path, err, sizeof err) == 0;
    check(ok, "a GGUF file written here reads (rt_gguf_read)");
    if (ok) {
        check(rt_gguf_upload(&R, &g, path, err, sizeof err) == 0 && g.q8_count == 2, "rt_gguf_upload: two distinct matrices");
        const struct rt_gguf_tensor *ta = rt_gguf_tensor(&g, "a"), *tb = rt_gguf_tensor(&g, "b"), *tt = rt_gguf_tensor(&g, "a.tied");
        check(ta && tb && tt && ta->w && tt->w == ta->w && tb->w != ta->w && rt_gguf_tensor_at(&g, tb->offset) == tb,
              "the tie by offset shares one handle; lookups by name and by offset agree");
        rt_set_exact(&R, 1);
        same = ta && tb && ta->w && tb->w;
        for (int k = 0; same && k < 2; k++) {
            rt_gemv(&R, k ? tb->w : ta->w, rows, cols, x, y);
            ref_fold(q8[k ? 3 : 0], rows, cols, x, want);
            same &= memcmp(y, want, sizeof(float) * (size_t)rows) == 0;
        }
        check(same, "exact products on the file's matrices == the reference fold of the rows written");
        rt_set_exact(&R, 0);
        rt_gguf_release(&R, &g);
        rt_gguf_free(&g);
    } else {
        printf("      %s\n", err);
    }
    if (fd >= 0) {
        close(fd);
        unlink(path);
    }
    rt_fini(&R);
    printf("%s\n", fails ? "FAILED" : "ALL PASS");
    return fails != 0;
}
