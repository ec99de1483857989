/* q8_hostbench.c: the host-pointer entry points timed from C, as the reference's generated code
 * calls them (src/card/rt.h:61-72), with nothing between the calls but the caller's own loop.
 * Prints one JSON object:
 *   rt_gemv_4096x4096   rt_gemv on 4096x4096 over rotated copies (>= 512 MB, so the 256 MB
 *                       Infinity Cache cannot serve them): microseconds a call, and the call's
 *                       phases (rt_host_timing: x staged, launches, wait, y copied out);
 *   quartet_round_9b    rt_gemv_q x 4 + rt_gemv_go on the 9B DeltaNet quartet (8192, 4096, 32, 32
 *                       rows x 4096, sharing x; src/apl/qwen35.apl:93-96), rotated;
 *   token_9b            the 9B decode token: per layer rt_gemv (QKV 6144x4096), rt_gemv (out
 *                       4096x4096), rt_gemv_q x 2 + rt_gemv_go (gate and up 12288x4096, sharing
 *                       x), rt_gemv (down 4096x12288), 32 distinct layers, then rt_gemv (head
 *                       151936x4096): milliseconds a token and the phases of its calls.
 * Weights are synthetic (rt_q8_fill_dev, repacked on the device). Needs the GPU. Usage:
 * q8_hostbench [passes [x_direct]]: 10 passes by default; x_direct 0 or 1 sets rt_set_x_direct
 * (default: the library's). */
#define _POSIX_C_SOURCE 199309L
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "q8_rt.h"

static double now_us(void)
{
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec * 1e6 + ts.tv_nsec * 1e-3;
}

static struct rt R;
static void *staging;
static unsigned long seed = 500;

/* a synthetic Q8_0 matrix, repacked into a device buffer that becomes its handle */
static const void *matrix(long rows, long cols)
{
    void *w = rt_dev_alloc(&R, rows * cols / 32 * 34);
    if (!w) {
        fprintf(stderr, "q8_hostbench: out of device memory\n");
        exit(1);
    }
    rt_q8_fill_dev(&R, staging, rows, cols, ++seed, 0, 0.0f, 0.02f);
    rt_q8_repack_dev(&R, staging, rows, cols, w);
    return w;
}

static float *vec(long n)
{
    float *v = malloc(sizeof(float) * (size_t)n);
    for (long i = 0; i < n; i++)
        v[i] = (float)((i * 2654435761u) % 2001u) / 1000.0f - 1.0f;
    return v;
}

static void phases(const char *key, double calls_per_unit)
{
    double us[RT_HT_PHASES];
    const long n = rt_host_timing_read(&R, us);
    printf("\"%s\": {\"calls\": %ld, \"stage_x_us\": %.3f, \"launch_us\": %.3f, \"wait_us\": %.3f, \"copy_out_us\": %.3f}", key, n,
           us[RT_HT_STAGE] / n * calls_per_unit, us[RT_HT_LAUNCH] / n * calls_per_unit, us[RT_HT_WAIT] / n * calls_per_unit,
           us[RT_HT_COPY_OUT] / n * calls_per_unit);
}

int main(int argc, char **argv)
{
    const int passes = argc > 1 ? atoi(argv[1]) : 10;
    if (rt_init(&R, 1) != 0) {
        fprintf(stderr, "q8_hostbench: rt_init failed\n");
        return 1;
    }
    /* the library's default unless the second argument sets it */
    int direct = rt_set_x_direct(&R, 1);
    if (argc > 2)
        direct = atoi(argv[2]) != 0;
    rt_set_x_direct(&R, direct);
    staging = rt_dev_alloc(&R, 151936L * 4096 / 32 * 34);
    const long H = 4096, F = 12288, Q = 6144, V = 151936;
    printf("{\"x_direct\": %d, ", direct);

    /* rt_gemv 4096x4096, 31 copies (527 MB) */
    {
        enum { N = 31 };
        const void *w[N];
        for (int i = 0; i < N; i++)
            w[i] = matrix(H, H);
        float *x = vec(H), *y = vec(H);
        for (int i = 0; i < N; i++)
            rt_gemv(&R, w[i], H, H, x, y);
        rt_host_timing(&R, 1);
        const double t0 = now_us();
        for (int p = 0; p < passes; p++)
            for (int i = 0; i < N; i++)
                rt_gemv(&R, w[i], H, H, x, y);
        const double us = (now_us() - t0) / (passes * N);
        const double bytes = (double)H * H / 32 * 34 + 8.0 * H;
        printf("\"rt_gemv_4096x4096\": {\"us_per_call\": %.3f, \"GB/s\": %.1f, \"copies\": %d, ", us, bytes / us / 1e3, N);
        phases("phases_per_call", 1.0);
        printf("}, ");
        rt_host_timing(&R, 0);
        for (int i = 0; i < N; i++)
            rt_dev_free(&R, (void *)w[i]);
        free(x);
        free(y);
    }

    /* the DeltaNet quartet, 12 rotated sets (1.7 GB) */
    {
        enum { N = 12 };
        const long rows[4] = {8192, 4096, 32, 32};
        const void *w[N][4];
        for (int i = 0; i < N; i++)
            for (int k = 0; k < 4; k++)
                w[i][k] = matrix(rows[k], H);
        float *x = vec(H), *y[4];
        for (int k = 0; k < 4; k++)
            y[k] = vec(rows[k]);
        for (int p = -1; p < passes; p++) {
            if (p == 0) {
                rt_host_timing(&R, 1);
            }
            const double t0 = now_us();
            for (int i = 0; i < N; i++) {
                rt_gemv_open(&R);
                for (int k = 0; k < 4; k++)
                    rt_gemv_q(&R, w[i][k], rows[k], H, x, y[k]);
                rt_gemv_go(&R);
            }
            if (p == passes - 1) {
                double bytes = 4.0 * H;
                for (int k = 0; k < 4; k++)
                    bytes += (double)rows[k] * H / 32 * 34 + 4.0 * rows[k];
                const double us = (now_us() - t0) / N;
                printf("\"quartet_round_9b\": {\"us_per_round\": %.3f, \"GB/s\": %.1f, ", us, bytes / us / 1e3);
                phases("phases_per_round", 1.0);
                printf("}, ");
            }
        }
        rt_host_timing(&R, 0);
        for (int i = 0; i < N; i++)
            for (int k = 0; k < 4; k++)
                rt_dev_free(&R, (void *)w[i][k]);
        free(x);
        for (int k = 0; k < 4; k++)
            free(y[k]);
    }

    /* the 9B token through the host-pointer entry points */
    {
        enum { L = 32 };
        const void *qkv[L], *out[L], *gate[L], *up[L], *down[L], *head;
        for (int l = 0; l < L; l++) {
            qkv[l] = matrix(Q, H);
            out[l] = matrix(H, H);
            gate[l] = matrix(F, H);
            up[l] = matrix(F, H);
            down[l] = matrix(H, F);
        }
        head = matrix(V, H);
        float *x0 = vec(H), *yq = vec(Q), *yo = vec(H), *g = vec(F), *u = vec(F), *yd = vec(H), *logits = vec(V);
        const int tokens = passes < 5 ? passes : 5;
        double ms = 0.0;
        for (int tk = -1; tk < tokens; tk++) {
            if (tk == 0)
                rt_host_timing(&R, 1);
            const double t0 = now_us();
            const float *x = x0;
            for (int l = 0; l < L; l++) {
                rt_gemv(&R, qkv[l], Q, H, x, yq);
                rt_gemv(&R, out[l], H, H, yq, yo);
                rt_gemv_open(&R);
                rt_gemv_q(&R, gate[l], F, H, yo, g);
                rt_gemv_q(&R, up[l], F, H, yo, u);
                rt_gemv_go(&R);
                rt_gemv(&R, down[l], H, F, g, yd);
                x = yd;
            }
            rt_gemv(&R, head, V, H, x, logits);
            if (tk >= 0)
                ms += (now_us() - t0) / 1e3;
        }
        ms /= tokens;
        double bytes = (double)V * H / 32 * 34 + 4.0 * (H + V);
        bytes += L * ((double)Q * H / 32 * 34 + 4.0 * (H + Q) + (double)H * H / 32 * 34 + 8.0 * H + 2.0 * F * H / 32 * 34 + 4.0 * (H + 2 * F) +
                      (double)H * F / 32 * 34 + 4.0 * (F + H));
        printf("\"token_9b\": {\"ms_per_token\": %.4f, \"GB/s\": %.1f, \"pct_hbm\": %.1f, \"calls_per_token\": %d, \"bytes_per_token\": %.0f, "
               "\"tokens_timed\": %d, ",
               ms, bytes / ms / 1e6, 100.0 * bytes / ms / 1e6 / 8000.0, 4 * L + 1, bytes, tokens);
        phases("phases_per_token", 4.0 * L + 1);
        printf("}");
        rt_host_timing(&R, 0);
    }
    printf("}\n");
    rt_fini(&R);
    return 0;
}
