/* q8_kernels.hip: the Q8_0 product kernels for gfx950 and their launchers.
 *
 *   gemv_s      decode, t = 1..4 tokens: HBM-bound (1.88 flop/B). Each wave owns RW rows
 *               of one 16-row group and the whole of K; each lane takes 16-column units
 *               (one 16-byte load of one row) 64 units apart, so a wave reads 1 KiB of a row
 *               per load. Per unit: 16 exact int8->f32 converts, shared by the t tokens, a
 *               16-step fma chain per token, then acc = fma(s, d, acc) with the unit's
 *               binary16 block scale. One fixed-order sum over the wave's lanes at the end.
 *               With a second matrix the pair shares every load of x and ends in
 *               SiLU(g) * u (the FFN's gate and up, src/apl/qwen35.apl:125).
 *   exact_s     the reference's order (src/card/gemv.c:166-193; gemm.c:20-23 per token): one
 *               lane per (token, row), T from +0 by 32 fma in column order, then
 *               acc = fma(T, d, acc). Bit-identical to the reference's F32 host path.
 *   repack_s    GGUF rows to form S.
 *   fill_*      synthetic weights and activations, a function of (seed, index) only.
 *   prims       the conversions above, lane by lane, for the known-answer gates. */
#include <hip/hip_runtime.h>

#include <limits.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>

#include "q8_device.h"

/* ---------------------------------------------------------------- decode GEMV */

void *q8_next_start = nullptr, *q8_next_stop = nullptr;
long *q8_next_grid = nullptr;
static char *q8_next_name = nullptr;

void q8_time_next(void *start_event, void *stop_event, char *name, long *grid)
{
    q8_next_start = start_event;
    q8_next_stop = stop_event;
    q8_next_name = name;
    q8_next_grid = grid;
}

void q8_time_name(const char *base, int n, ...)
{
    va_list ap;
    va_start(ap, n);
    int k = snprintf(q8_next_name, 64, "%s", base);
    for (int i = 0; i < n && k < 63; i++)
        k += snprintf(q8_next_name + k, (size_t)(64 - k), "%s%d", i ? ", " : "<", va_arg(ap, int));
    if (n && k < 63)
        snprintf(q8_next_name + k, (size_t)(64 - k), ">");
    va_end(ap);
}

#define GEMV_WAVES 4 /* waves per workgroup */

template <int MT, int RW, int PAIR>
__global__ __launch_bounds__(64 * GEMV_WAVES) void gemv_s(const uint8_t *__restrict__ w0, const uint8_t *__restrict__ w1, long rows, long cols,
                                                          const float *__restrict__ x, long x_stride, float *__restrict__ y)
{
    const int lane = threadIdx.x & 63;
    const long r0 = ((long)blockIdx.x * GEMV_WAVES + (threadIdx.x >> 6)) * RW;
    if (r0 >= rows)
        return;
    const long units = cols / 16; /* even: cols % 32 == 0 */
    const uint8_t *wq[PAIR + 1][RW];
    const uint16_t *wd[PAIR + 1][RW];
#pragma unroll
    for (int p = 0; p <= PAIR; p++) {
        const uint8_t *w = p ? w1 : w0;
#pragma unroll
        for (int r = 0; r < RW; r++) {
            wq[p][r] = w + q8s_row_q(r0 + r, cols);
            wd[p][r] = (const uint16_t *)(w + q8s_row_d(r0 + r, cols));
        }
    }
    float acc[PAIR + 1][RW][MT];
#pragma unroll
    for (int p = 0; p <= PAIR; p++)
#pragma unroll
        for (int r = 0; r < RW; r++)
#pragma unroll
            for (int m = 0; m < MT; m++)
                acc[p][r][m] = 0.0f;

    for (long u = lane; u < units; u += 64) {
        /* every load of the step first: RW (x2) rows of weights, their scales, x */
        uint4 q[PAIR + 1][RW];
        uint16_t dh[PAIR + 1][RW];
#pragma unroll
        for (int p = 0; p <= PAIR; p++)
#pragma unroll
            for (int r = 0; r < RW; r++) {
                q[p][r] = *(const uint4 *)(wq[p][r] + 16 * u);
                dh[p][r] = wd[p][r][u >> 1];
            }
        float4 xv[MT][4];
#pragma unroll
        for (int m = 0; m < MT; m++)
#pragma unroll
            for (int c = 0; c < 4; c++)
                xv[m][c] = *(const float4 *)(x + m * x_stride + 16 * u + 4 * c);
#pragma unroll
        for (int p = 0; p <= PAIR; p++)
#pragma unroll
            for (int r = 0; r < RW; r++) {
                const uint32_t qw[4] = {q[p][r].x, q[p][r].y, q[p][r].z, q[p][r].w};
                float wf[16];
#pragma unroll
                for (int j = 0; j < 16; j++)
                    wf[j] = q8_s8(qw[j >> 2], j & 3);
                const float d = q8_half(dh[p][r]);
#pragma unroll
                for (int m = 0; m < MT; m++) {
                    const float xs[16] = {xv[m][0].x, xv[m][0].y, xv[m][0].z, xv[m][0].w, xv[m][1].x, xv[m][1].y, xv[m][1].z, xv[m][1].w,
                                          xv[m][2].x, xv[m][2].y, xv[m][2].z, xv[m][2].w, xv[m][3].x, xv[m][3].y, xv[m][3].z, xv[m][3].w};
                    float s = 0.0f;
#pragma unroll
                    for (int j = 0; j < 16; j++)
                        s = __builtin_fmaf(wf[j], xs[j], s);
                    acc[p][r][m] = __builtin_fmaf(s, d, acc[p][r][m]);
                }
            }
    }
#pragma unroll
    for (int p = 0; p <= PAIR; p++)
#pragma unroll
        for (int r = 0; r < RW; r++)
#pragma unroll
            for (int m = 0; m < MT; m++)
                acc[p][r][m] = q8_wave_sum(acc[p][r][m]);
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < RW; r++)
#pragma unroll
            for (int m = 0; m < MT; m++)
                y[m * rows + r0 + r] = PAIR ? q8_swiglu(acc[0][r][m], acc[PAIR][r][m]) : acc[0][r][m];
    }
}

/* The decode kernel for cols % 1024 == 0: a workgroup of NW waves owns RW rows and all of K;
 * wave w takes the K-slice [w*1024*S, (w+1)*1024*S), S steps of 64 16-column units (lane l:
 * units l + 64 s). Every load of a lane is issued before any arithmetic, x first and then the
 * weights row by row (loads retire in order, so row r's arithmetic waits for rows 0..r only), so
 * the whole matrix is in flight in the first round trip: the layer matrices are latency-bound
 * otherwise. Per unit: 16 exact int8->f32 converts shared by the MT tokens, a 16-step fma chain
 * per token, then acc = fma(s, d, acc) with the unit's block scale. The lanes' partials are summed
 * by q8_wave_sum_dpp, the NW waves' in LDS in wave order: the same order every run. */
/* EPI: 0 none; 1 the RMS norm of x first (e.nw, e.eps); 2 y = e.res + the product (q8_epi). y and
 * e.res may be the same array: each element is read and then written by the one thread that owns it. */
template <int MT, int RW, int S, int NW, int PAIR, int EPI>
__device__ __forceinline__ void gemv_body(const uint8_t *__restrict__ w0, const uint8_t *__restrict__ w1, long rows, long cols, const float *__restrict__ x,
                                          long x_stride, float *y, long r0, q8_epi e)
{
    constexpr int P = PAIR + 1;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const long u0 = (long)wave * 64 * S + lane;

    float4 xv[MT][S][4];
#pragma unroll
    for (int m = 0; m < MT; m++)
#pragma unroll
        for (int s = 0; s < S; s++)
#pragma unroll
            for (int c = 0; c < 4; c++)
                xv[m][s][c] = *(const float4 *)(x + m * x_stride + 16 * (u0 + 64 * s) + 4 * c);
    /* the residual of the output this thread stores (thread k < RW*MT stores row k / MT, token
     * k % MT; the others load one of those too, so the load is unconditional), issued with x so
     * that it is not a memory latency at the kernel's end */
    float rv = 0.0f;
    if constexpr (EPI == 2) {
        static_assert(NW > 1, "the residual epilogue stores from threads < RW * MT");
        const int k = (int)threadIdx.x % (RW * MT);
        rv = e.res[(long)(k % MT) * rows + r0 + k / MT];
    }
    /* the norm's weights, the lane's columns, issued with x before the matrix */
    float4 nv[S][4];
    if constexpr (EPI == 1) {
#pragma unroll
        for (int s = 0; s < S; s++)
#pragma unroll
            for (int c = 0; c < 4; c++)
                nv[s][c] = *(const float4 *)(e.nw + 16 * (u0 + 64 * s) + 4 * c);
        /* keep them there: left to itself the scheduler issues them after the matrix, and the
         * products of x and the norm weights, which every fma needs, then wait for all of it */
        __builtin_amdgcn_sched_barrier(0);
    }
    uint4 q[RW][P][S];
    uint16_t dh[RW][P][S];
#pragma unroll
    for (int r = 0; r < RW; r++)
#pragma unroll
        for (int p = 0; p < P; p++) {
            const uint8_t *w = p ? w1 : w0;
            const uint8_t *wq = w + q8s_row_q(r0 + r, cols);
            const uint16_t *wd = (const uint16_t *)(w + q8s_row_d(r0 + r, cols));
#pragma unroll
            for (int s = 0; s < S; s++) {
                q[r][p][s] = *(const uint4 *)(wq + 16 * (u0 + 64 * s));
                dh[r][p][s] = wd[(u0 + 64 * s) >> 1];
            }
        }
    /* every load issued before any arithmetic: left to itself the scheduler sinks the last rows'
     * loads past the first rows' arithmetic, and past the wait for x, so they start a memory round
     * trip late (4096x12288 at one token 10.85 against 11.0 us, at three 13.3 against 13.5). Not
     * for 16 rows at two tokens, where the scheduler's own order measured faster (4096x12288: 11.4
     * against 11.6 us) */
    if constexpr (!(MT == 2 && RW == 16))
        __builtin_amdgcn_sched_barrier(0);

    /* the norm: x <- nw * x at once, and per token the sum of x^2 (the lane's, then the wave's,
     * left in LDS for the final reduction, whose barrier covers it); s = 1 / sqrt(eps + sum / cols)
     * multiplies the outputs at the end, W (nw * x) s = W (nw * (x s)): no barrier before the
     * arithmetic starts, and x and nw are dead once multiplied */
    float ss[MT];
    if constexpr (EPI == 1) {
#pragma unroll
        for (int m = 0; m < MT; m++) {
            float a = 0.0f;
#pragma unroll
            for (int s = 0; s < S; s++)
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    const float4 v = xv[m][s][c], g = nv[s][c];
                    a = __builtin_fmaf(v.x, v.x, a);
                    a = __builtin_fmaf(v.y, v.y, a);
                    a = __builtin_fmaf(v.z, v.z, a);
                    a = __builtin_fmaf(v.w, v.w, a);
                    xv[m][s][c] = make_float4(g.x * v.x, g.y * v.y, g.z * v.z, g.w * v.w);
                }
            ss[m] = q8_wave_sum_dpp(a);
        }
    }
    /* the wave's RW*P*MT sums over its lanes (q8_wave_sums, padded to a power of two), each
     * written to LDS once; then the NW waves' in wave order. CH: in chunks of up to 8 rows, each
     * chunk's sums run while later rows' loads still arrive. The two forms give the same bits; the
     * compiler allocates their registers differently, and each was measured where it is used:
     * chunks for the pair at 2 tokens (20.0 against 21.2 us on 12288x4096) and for 16 rows at 3
     * tokens (119 registers, where one block of sums spills: 13.7 against 14.4 us at 8 rows on
     * 4096x12288); one block everywhere else (the pair at 1 token 18.0 against 18.5 us, 16 rows at
     * 2 and 4 tokens 11.7 / 14.5 against 12.5 / 15.6). */
    constexpr bool CH = (PAIR && MT == 2) || (MT == 3 && RW == 16);
    constexpr int RC = CH && RW > 8 ? 8 : RW, VC = RC * P * MT, VP = q8_pow2ceil(VC);
    __shared__ float red[NW][RW * P * MT];
    __shared__ float nsum[EPI == 1 ? NW : 1][MT];
    if constexpr (EPI == 1) {
        if (lane == 0)
#pragma unroll
            for (int m = 0; m < MT; m++)
                nsum[wave][m] = ss[m];
    }
    /* row r's sum of token m of matrix p over the lane's columns */
    auto row_sum = [&](int r, int p, int m) {
        float acc = 0.0f;
#pragma unroll
        for (int s = 0; s < S; s++) {
            const uint32_t qw[4] = {q[r][p][s].x, q[r][p][s].y, q[r][p][s].z, q[r][p][s].w};
            const float xs[16] = {xv[m][s][0].x, xv[m][s][0].y, xv[m][s][0].z, xv[m][s][0].w, xv[m][s][1].x, xv[m][s][1].y,
                                  xv[m][s][1].z, xv[m][s][1].w, xv[m][s][2].x, xv[m][s][2].y, xv[m][s][2].z, xv[m][s][2].w,
                                  xv[m][s][3].x, xv[m][s][3].y, xv[m][s][3].z, xv[m][s][3].w};
            float sum = 0.0f;
#pragma unroll
            for (int j = 0; j < 16; j++)
                sum = __builtin_fmaf(q8_s8(qw[j >> 2], j & 3), xs[j], sum);
            acc = __builtin_fmaf(sum, q8_half(dh[r][p][s]), acc);
        }
        return acc;
    };
    /* a block of VC sums (rows [ch*RC, +RC)) over the lanes, into LDS */
    auto lane_sums = [&](float (&vals)[VP], int ch) {
#pragma unroll
        for (int i = VC; i < VP; i++)
            vals[i] = 0.0f;
        q8_wave_sums<VP>(vals, lane);
        if (q8_wave_sums_owner<VP>(lane)) {
#pragma unroll
            for (int k = 0; k < (VP >> q8_wave_sums_steps<VP>()); k++) {
                const int g = q8_wave_sums_index<VP>(lane, k);
                if (g < VC)
                    red[wave][ch * VC + g] = vals[k];
            }
        }
    };
    if constexpr (CH) {
#pragma unroll
        for (int ch = 0; ch < RW / RC; ch++) {
            float vals[VP];
#pragma unroll
            for (int rr = 0; rr < RC; rr++)
#pragma unroll
                for (int p = 0; p < P; p++)
#pragma unroll
                    for (int m = 0; m < MT; m++)
                        vals[(rr * P + p) * MT + m] = row_sum(ch * RC + rr, p, m);
            lane_sums(vals, ch);
        }
    } else {
        float acc[RW][P][MT];
#pragma unroll
        for (int r = 0; r < RW; r++)
#pragma unroll
            for (int p = 0; p < P; p++)
#pragma unroll
                for (int m = 0; m < MT; m++)
                    acc[r][p][m] = row_sum(r, p, m);
        float vals[VP];
#pragma unroll
        for (int r = 0; r < RW; r++)
#pragma unroll
            for (int p = 0; p < P; p++)
#pragma unroll
                for (int m = 0; m < MT; m++)
                    vals[(r * P + p) * MT + m] = acc[r][p][m];
        lane_sums(vals, 0);
    }
    __syncthreads();
    if (threadIdx.x < RW * MT) {
        const int r = threadIdx.x / MT, m = threadIdx.x % MT;
        float v[P];
#pragma unroll
        for (int p = 0; p < P; p++) {
            v[p] = red[0][(r * P + p) * MT + m];
#pragma unroll
            for (int k = 1; k < NW; k++)
                v[p] += red[k][(r * P + p) * MT + m];
        }
        if constexpr (EPI == 1) {
            /* the token's sum of x^2 over the waves, in wave order */
            float tot = nsum[0][m];
#pragma unroll
            for (int k = 1; k < NW; k++)
                tot += nsum[k][m];
            const float sc = 1.0f / sqrtf(e.eps + tot / (float)cols);
#pragma unroll
            for (int p = 0; p < P; p++)
                v[p] *= sc;
        }
        const long i = m * rows + r0 + r;
        const float o = PAIR ? q8_swiglu(v[0], v[P - 1]) : v[0];
        y[i] = EPI == 2 ? rv + o : o;
    }
}

template <int MT, int RW, int S, int NW, int PAIR>
__global__ __launch_bounds__(64 * NW) void gemv_k(const uint8_t *__restrict__ w0, const uint8_t *__restrict__ w1, long rows, long cols,
                                                  const float *__restrict__ x, long x_stride, float *__restrict__ y)
{
    gemv_body<MT, RW, S, NW, PAIR, 0>(w0, w1, rows, cols, x, x_stride, y, (long)blockIdx.x * RW, q8_epi{});
}

/* the same with an epilogue fused (EPI 1: the norm of x first; 2: the residual added to y) */
template <int MT, int RW, int S, int NW, int PAIR, int EPI>
__global__ __launch_bounds__(64 * NW) void gemv_ke(const uint8_t *__restrict__ w0, const uint8_t *__restrict__ w1, long rows, long cols,
                                                   const float *__restrict__ x, long x_stride, float *y, q8_epi e)
{
    gemv_body<MT, RW, S, NW, PAIR, EPI>(w0, w1, rows, cols, x, x_stride, y, (long)blockIdx.x * RW, e);
}

/* A round of up to Q8_ROUND_MAX products that share x (the reference's queued products, none
 * reading another's result, src/card/rt.c:216-242), as one launch: workgroup b belongs to the
 * product p with start[p] <= b < start[p+1] and takes its rows [(b - start[p]) * RW, +RW). */
template <int MT, int RW, int S, int NW>
__global__ __launch_bounds__(64 * NW) void gemv_round(q8_round r, long cols, const float *__restrict__ x, long x_stride)
{
    int p = 0;
#pragma unroll
    for (int k = 1; k < Q8_ROUND_MAX; k++)
        if (k < r.n && (long)blockIdx.x >= r.start[k])
            p = k;
    gemv_body<MT, RW, S, NW, 0, 0>((const uint8_t *)r.w[p], nullptr, r.rows[p], cols, x, x_stride, r.y[p], ((long)blockIdx.x - r.start[p]) * RW, q8_epi{});
}

/* a round with the RMS norm of x fused: every workgroup normalises the x it reads */
template <int MT, int RW, int S, int NW>
__global__ __launch_bounds__(64 * NW) void gemv_round_norm(q8_round r, long cols, const float *__restrict__ x, long x_stride, q8_epi e)
{
    int p = 0;
#pragma unroll
    for (int k = 1; k < Q8_ROUND_MAX; k++)
        if (k < r.n && (long)blockIdx.x >= r.start[k])
            p = k;
    gemv_body<MT, RW, S, NW, 0, 1>((const uint8_t *)r.w[p], nullptr, r.rows[p], cols, x, x_stride, r.y[p], ((long)blockIdx.x - r.start[p]) * RW, e);
}

template <int MT, int RW, int S, int NW, int PAIR>
static void gemv_launch(hipStream_t s, const uint8_t *a, const uint8_t *b, long rows, long cols, const float *x, long xs, float *y)
{
    Q8_LAUNCH(q8_time_name("gemv_k", 5, MT, RW, S, NW, PAIR), (gemv_k<MT, RW, S, NW, PAIR>), dim3((unsigned)(rows / RW)), dim3(64 * NW), s, a, b, rows,
              cols, x, xs, y);
}

/* K = 1024 * S * NW; RW rows a workgroup (rows % RW == 0) */
template <int MT, int RW, int PAIR>
static bool gemv_go_rw(hipStream_t s, int nw, long kb, const uint8_t *a, const uint8_t *b, long rows, long cols, const float *x, long xs, float *y)
{
#define K1(S, N)                                                                                                       \
    if (nw == N && kb == (long)S * N) {                                                                                \
        gemv_launch<MT, RW, S, N, PAIR>(s, a, b, rows, cols, x, xs, y);                                                \
        return true;                                                                                                   \
    }
    K1(1, 1) K1(1, 2) K1(1, 4) K1(1, 6) K1(1, 8) K1(1, 12) K1(1, 16) K1(2, 4) K1(3, 4) K1(4, 4) K1(2, 2) K1(3, 2) K1(2, 1) K1(2, 8)
#undef K1
    return false;
}

/* The decode kernel's rows a workgroup (rw) and waves (nw) for a shape; kb = cols / 1024 */
static void gemv_choose(int pair, int mt, long rows, long kb, int *rw_out, int *nw_out)
{
    /* measured on the 9B shapes: 8 rows a workgroup (for the pair 4 at 1 token, the same 8 rows of
     * loads a lane, and 8 at 2 to 4: 12288x4096 at 3 tokens 22.5 against 24.6 us), one 1024-column
     * step a wave, so K = 4096 takes 4 waves and K = 12288 takes 12 */
    int rw = pair ? (mt == 1 ? 4 : 8) : 8, nw = (int)kb;
    if (kb > 16 || kb == 3 || kb == 5 || kb == 7 || (kb > 8 && kb != 12 && kb != 16))
        nw = kb % 4 == 0 ? 4 : kb % 2 == 0 ? 2 : 1;
    /* 2 to 4 tokens at K = 12288: 16 rows, one 12-wave workgroup a CU and the grid in one round
     * (4096 x 12288: 11.4 against 12.3 us at 2 tokens, 13.7 against 14.4 at 3, 14.5 against 16.2
     * at 4) */
    if (!pair && mt >= 2 && nw == 12 && rows / 16 >= 256)
        rw = 16;
    /* small matrices (the 2B layer's): fewer rows a workgroup, so that at least 1024 waves (4096
     * for the pair) stream. At one token 3072x2048 3.5 against 3.6 us at 4 rows (1536 waves) and 2,
     * the pair 6144x2048 6.7 against 7.0 at 2 rows and 4, 2048x6144 4.8 against 4.9 at 8 and 4 */
    while (rw > 2 && rows / rw * nw < (pair ? 4096 : 1024))
        rw /= 2;
    *rw_out = rw, *nw_out = nw;
}

template <int MT, int PAIR>
static void gemv_go(hipStream_t s, const void *w0, const void *w1, long rows, long cols, const float *x, long xs, float *y)
{
    const uint8_t *a = (const uint8_t *)w0, *b = (const uint8_t *)w1;
    const long kb = cols % 1024 ? 0 : cols / 1024;
    int rw, nw;
    gemv_choose(PAIR, MT, rows, kb, &rw, &nw);
    if (kb && rows % rw == 0) {
        bool done = false;
        switch (rw) {
        case 1: done = gemv_go_rw<MT, 1, PAIR>(s, nw, kb, a, b, rows, cols, x, xs, y); break;
        case 2: done = gemv_go_rw<MT, 2, PAIR>(s, nw, kb, a, b, rows, cols, x, xs, y); break;
        case 8: done = gemv_go_rw<MT, 8, PAIR>(s, nw, kb, a, b, rows, cols, x, xs, y); break;
        case 16: done = gemv_go_rw<MT, 16, PAIR>(s, nw, kb, a, b, rows, cols, x, xs, y); break;
        default: done = rw == 4 && gemv_go_rw<MT, 4, PAIR>(s, nw, kb, a, b, rows, cols, x, xs, y); break;
        }
        if (done)
            return;
    }
    /* any other cols (a multiple of 32): the loop over K */
    const long waves = rows / 4;
    Q8_LAUNCH(q8_time_name("gemv_s", 3, MT, 4, PAIR), (gemv_s<MT, 4, PAIR>), dim3((unsigned)((waves + GEMV_WAVES - 1) / GEMV_WAVES)), dim3(64 * GEMV_WAVES), s,
              a, b, rows, cols, x, xs, y);
}

template <int PAIR>
static void gemv_t(hipStream_t s, const void *w0, const void *w1, long rows, long cols, const float *x, long xs, long t, float *y)
{
    switch (t) {
    case 1: gemv_go<1, PAIR>(s, w0, w1, rows, cols, x, xs, y); break;
    case 2: gemv_go<2, PAIR>(s, w0, w1, rows, cols, x, xs, y); break;
    case 3: gemv_go<3, PAIR>(s, w0, w1, rows, cols, x, xs, y); break;
    default: gemv_go<4, PAIR>(s, w0, w1, rows, cols, x, xs, y); break;
    }
}

void q8_launch_gemv(q8_stream_t stream, const void *w0, const void *w1, long rows, long cols, const float *x, long x_stride, long t, float *y)
{
    hipStream_t s = (hipStream_t)stream;
    /* at most 4 tokens a launch; more go token slice by token slice */
    for (long k = 0; k < t; k += 4) {
        const long n = t - k < 4 ? t - k : 4;
        if (w1)
            gemv_t<1>(s, w0, w1, rows, cols, x + k * x_stride, x_stride, n, y + k * rows);
        else
            gemv_t<0>(s, w0, w1, rows, cols, x + k * x_stride, x_stride, n, y + k * rows);
    }
}

/* ---- the epilogue kernels: the layer shapes' K (S = 1 and NW = 2, 4, 6, 12: K = 2048, 4096,
 * 6144, 12288) at 2, 4 or 8 rows a workgroup; any other shape runs its epilogue apart */
template <int MT, int RW, int PAIR, int EPI>
static bool gemv_epi_rw(hipStream_t s, int nw, long kb, const uint8_t *a, const uint8_t *b, long rows, long cols, const float *x, long xs, float *y,
                        const q8_epi &e)
{
#define K1(S, N)                                                                                                       \
    if (nw == N && kb == (long)S * N) {                                                                                \
        Q8_LAUNCH(q8_time_name("gemv_ke", 6, MT, RW, S, N, PAIR, EPI), (gemv_ke<MT, RW, S, N, PAIR, EPI>), dim3((unsigned)(rows / RW)), dim3(64 * N), s, \
                  a, b, rows, cols, x, xs, y, e);                                                                      \
        return true;                                                                                                   \
    }
    K1(1, 2) K1(1, 4) K1(1, 6)
    /* K = 12288 (the down matrix): not the pair (no layer has one there), nor 4 tokens at 8 rows
     * with the norm (both would spill registers) */
    if constexpr (!PAIR && !(MT == 4 && RW == 8 && EPI == 1)) {
        K1(1, 12)
    }
#undef K1
    return false;
}

template <int MT, int PAIR, int EPI>
static bool gemv_epi_go(hipStream_t s, const void *w0, const void *w1, long rows, long cols, const float *x, long xs, float *y, const q8_epi &e)
{
    const uint8_t *a = (const uint8_t *)w0, *b = (const uint8_t *)w1;
    const long kb = cols % 1024 ? 0 : cols / 1024;
    int rw, nw;
    gemv_choose(PAIR, 1, rows, kb, &rw, &nw); /* the fused-epilogue instances: as measured at one token */
    /* the pair with the norm: its norm weights take more registers, and 8 rows a workgroup (one
     * round of fewer, longer workgroups) is the faster shape then (12288x4096: 20.5 against 21.3 us) */
    if (PAIR && EPI == 1 && rw == 4 && rows % 8 == 0 && rows / 8 * nw >= 2048)
        rw = 8;
    if (!kb || rows % rw)
        return false;
    switch (rw) {
    case 2: return gemv_epi_rw<MT, 2, PAIR, EPI>(s, nw, kb, a, b, rows, cols, x, xs, y, e);
    case 4: return gemv_epi_rw<MT, 4, PAIR, EPI>(s, nw, kb, a, b, rows, cols, x, xs, y, e);
    case 8: return gemv_epi_rw<MT, 8, PAIR, EPI>(s, nw, kb, a, b, rows, cols, x, xs, y, e);
    default: return false;
    }
}

template <int MT>
static bool gemv_epi_t(hipStream_t s, const void *w0, const void *w1, long rows, long cols, const float *x, long xs, float *y, const q8_epi &e)
{
    if (w1)
        return gemv_epi_go<MT, 1, 1>(s, w0, w1, rows, cols, x, xs, y, e);
    return e.nw ? gemv_epi_go<MT, 0, 1>(s, w0, w1, rows, cols, x, xs, y, e) : gemv_epi_go<MT, 0, 2>(s, w0, w1, rows, cols, x, xs, y, e);
}

int q8_launch_gemv_epi(q8_stream_t stream, const void *w0, const void *w1, long rows, long cols, const float *x, long x_stride, long t, float *y,
                       q8_epi e)
{
    if (t < 1 || t > 4 || (e.nw != nullptr) == (e.res != nullptr) || (w1 && e.res))
        return -1;
    hipStream_t s = (hipStream_t)stream;
    bool done;
    switch (t) {
    case 1: done = gemv_epi_t<1>(s, w0, w1, rows, cols, x, x_stride, y, e); break;
    case 2: done = gemv_epi_t<2>(s, w0, w1, rows, cols, x, x_stride, y, e); break;
    case 3: done = gemv_epi_t<3>(s, w0, w1, rows, cols, x, x_stride, y, e); break;
    default: done = gemv_epi_t<4>(s, w0, w1, rows, cols, x, x_stride, y, e); break;
    }
    return done ? 0 : -1;
}

/* The RMS norm apart: one workgroup of 256 a token; x^2 summed by each thread over its columns,
 * then by the wave and across the 4 waves in a fixed order; xn may be x (xs == cols). */
__global__ __launch_bounds__(256) void rmsnorm_k(const float *x, long xs, long cols, const float *__restrict__ nw, float eps, float *xn)
{
    const float *xr = x + (long)blockIdx.x * xs;
    float *o = xn + (long)blockIdx.x * cols;
    float a = 0.0f;
    for (long k = 4 * (long)threadIdx.x; k < cols; k += 1024) {
        const float4 v = *(const float4 *)(xr + k);
        a = __builtin_fmaf(v.x, v.x, a);
        a = __builtin_fmaf(v.y, v.y, a);
        a = __builtin_fmaf(v.z, v.z, a);
        a = __builtin_fmaf(v.w, v.w, a);
    }
    a = q8_wave_sum_dpp(a);
    __shared__ float part[4];
    if ((threadIdx.x & 63) == 0)
        part[threadIdx.x >> 6] = a;
    __syncthreads();
    const float sc = 1.0f / sqrtf(eps + ((part[0] + part[1]) + (part[2] + part[3])) / (float)cols);
    for (long k = 4 * (long)threadIdx.x; k < cols; k += 1024) {
        const float4 v = *(const float4 *)(xr + k), g = *(const float4 *)(nw + k);
        *(float4 *)(o + k) = make_float4(g.x * (v.x * sc), g.y * (v.y * sc), g.z * (v.z * sc), g.w * (v.w * sc));
    }
}

void q8_launch_rmsnorm(q8_stream_t stream, const float *x, long x_stride, long t, long cols, const float *nw, float eps, float *xn)
{
    rmsnorm_k<<<dim3((unsigned)t), dim3(256), 0, (hipStream_t)stream>>>(x, x_stride, cols, nw, eps, xn);
}

__global__ __launch_bounds__(256) void add_k(const float *a, const float *b, long n, float *y)
{
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i < n)
        y[i] = a[i] + b[i];
}

void q8_launch_add(q8_stream_t stream, const float *a, const float *b, long n, float *y)
{
    add_k<<<dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream>>>(a, b, n, y);
}

template <int MT, int RW>
static bool round_go(hipStream_t s, int nw, long kb, const q8_round &r, long cols, const float *x, long xs)
{
#define K1(S, N)                                                                                                       \
    if (nw == N && kb == (long)S * N) {                                                                                \
        Q8_LAUNCH(q8_time_name("gemv_round", 4, MT, RW, S, N), (gemv_round<MT, RW, S, N>), dim3((unsigned)r.start[r.n]), dim3(64 * N), s, r, cols, x,  \
                  xs);                                                                                                 \
        return true;                                                                                                   \
    }
    K1(1, 1) K1(1, 2) K1(1, 4) K1(1, 6) K1(1, 8) K1(1, 12) K1(1, 16) K1(2, 4) K1(3, 4) K1(4, 4)
#undef K1
    return false;
}

constexpr int ROUND_RW = 8;

/* the round's table and waves; false when the kernel does not take the shape */
static bool round_plan(int n, const void *const *w, const long *rows, long cols, long t, float *const *y, q8_round &r, int &nw, long &kb)
{
    kb = cols % 1024 ? 0 : cols / 1024;
    if (n < 1 || n > Q8_ROUND_MAX || t < 1 || t > 4 || !kb)
        return false;
    nw = (int)kb;
    if (kb > 16 || kb == 3 || kb == 5 || kb == 7 || (kb > 8 && kb != 12 && kb != 16))
        nw = kb % 4 == 0 ? 4 : kb % 2 == 0 ? 2 : 1;
    r = q8_round{};
    r.n = n;
    for (int i = 0; i < n; i++) {
        if (rows[i] % ROUND_RW)
            return false;
        r.w[i] = w[i];
        r.y[i] = y[i];
        r.rows[i] = rows[i];
        r.start[i + 1] = r.start[i] + rows[i] / ROUND_RW;
    }
    return true;
}

template <int MT, int RW>
static bool round_norm_go(hipStream_t s, int nw, long kb, const q8_round &r, long cols, const float *x, long xs, const q8_epi &e)
{
#define K1(S, N)                                                                                                       \
    if (nw == N && kb == (long)S * N) {                                                                                \
        Q8_LAUNCH(q8_time_name("gemv_round_norm", 4, MT, RW, S, N), (gemv_round_norm<MT, RW, S, N>), dim3((unsigned)r.start[r.n]), dim3(64 * N), s, r, \
                  cols, x, xs, e);                                                                                     \
        return true;                                                                                                   \
    }
    K1(1, 2) K1(1, 4) K1(1, 6)
    if constexpr (MT < 4) { /* 4 tokens at K = 12288 would spill registers */
        K1(1, 12)
    }
#undef K1
    return false;
}

int q8_launch_gemv_round_epi(q8_stream_t stream, int n, const void *const *w, const long *rows, long cols, const float *x, long x_stride, long t,
                             float *const *y, q8_epi e)
{
    q8_round r;
    int nw;
    long kb;
    if (!e.nw || e.res || !round_plan(n, w, rows, cols, t, y, r, nw, kb))
        return -1;
    hipStream_t s = (hipStream_t)stream;
    constexpr int RW = ROUND_RW;
    bool done = false;
    switch (t) {
    case 1: done = round_norm_go<1, RW>(s, nw, kb, r, cols, x, x_stride, e); break;
    case 2: done = round_norm_go<2, RW>(s, nw, kb, r, cols, x, x_stride, e); break;
    case 3: done = round_norm_go<3, RW>(s, nw, kb, r, cols, x, x_stride, e); break;
    default: done = round_norm_go<4, RW>(s, nw, kb, r, cols, x, x_stride, e); break;
    }
    return done ? 0 : -1;
}

int q8_launch_gemv_round(q8_stream_t stream, int n, const void *const *w, const long *rows, long cols, const float *x, long x_stride, long t, float *const *y)
{
    q8_round r;
    int nw;
    long kb;
    if (!round_plan(n, w, rows, cols, t, y, r, nw, kb))
        return -1;
    constexpr int RW = ROUND_RW;
    hipStream_t s = (hipStream_t)stream;
    bool done = false;
    switch (t) {
    case 1: done = round_go<1, RW>(s, nw, kb, r, cols, x, x_stride); break;
    case 2: done = round_go<2, RW>(s, nw, kb, r, cols, x, x_stride); break;
    case 3: done = round_go<3, RW>(s, nw, kb, r, cols, x, x_stride); break;
    default: done = round_go<4, RW>(s, nw, kb, r, cols, x, x_stride); break;
    }
    return done ? 0 : -1;
}

/* ---------------------------------------------------------------- the reference's order */

__global__ __launch_bounds__(256) void exact_s(const uint8_t *__restrict__ w, long rows, long cols, const float *__restrict__ x, long x_stride, long t,
                                               float *__restrict__ y)
{
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * t)
        return;
    const long r = i % rows, m = i / rows;
    const uint8_t *q = w + q8s_row_q(r, cols);
    const uint16_t *d = (const uint16_t *)(w + q8s_row_d(r, cols));
    const float *xm = x + m * x_stride;
    float acc = 0.0f;
    for (long b = 0; b < cols / Q8_BLOCK; b++) {
        float tb = 0.0f;
        for (int h = 0; h < 2; h++) {
            const uint4 v = *(const uint4 *)(q + 32 * b + 16 * h);
            const uint32_t qw[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int j = 0; j < 16; j++)
                tb = __builtin_fmaf(q8_s8(qw[j >> 2], j & 3), xm[32 * b + 16 * h + j], tb);
        }
        acc = __builtin_fmaf(tb, q8_half(d[b]), acc);
    }
    y[m * rows + r] = acc;
}

void q8_launch_exact(q8_stream_t stream, const void *w, long rows, long cols, const float *x, long x_stride, long t, float *y)
{
    const long n = rows * t;
    Q8_LAUNCH(q8_time_name("exact_s", 0), exact_s, dim3((unsigned)((n + 255) / 256)), dim3(256), (hipStream_t)stream, (const uint8_t *)w, rows, cols, x, x_stride, t, y);
}

__global__ __launch_bounds__(256) void swiglu_ew(const float *__restrict__ g, const float *__restrict__ u, long n, float *__restrict__ y)
{
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n)
        y[i] = q8_swiglu(g[i], u[i]);
}

void q8_launch_swiglu_ew(q8_stream_t stream, const float *g, const float *u, long n, float *y)
{
    swiglu_ew<<<dim3((unsigned)((n + 255) / 256)), 256, 0, (hipStream_t)stream>>>(g, u, n, y);
}

/* ---------------------------------------------------------------- GGUF -> form S */

/* One thread per block of 32 weights: the 34 GGUF bytes (2-byte aligned: 34 = 2 * 17) in, 32
 * int8 to the row's q (32-byte aligned: two 16-byte stores) and the scale to the row's d. */
__global__ __launch_bounds__(256) void repack_s(const uint8_t *__restrict__ q8, long rows, long cols, uint8_t *__restrict__ out)
{
    const long nb = cols / Q8_BLOCK;
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * nb)
        return;
    const long r = i / nb, b = i % nb;
    const uint16_t *src = (const uint16_t *)(q8 + i * Q8_BLOCK_BYTES);
    uint16_t h[17];
#pragma unroll
    for (int k = 0; k < 17; k++)
        h[k] = src[k];
    uint32_t v[8];
#pragma unroll
    for (int k = 0; k < 8; k++)
        v[k] = (uint32_t)h[1 + 2 * k] | (uint32_t)h[2 + 2 * k] << 16;
    uint4 *dq = (uint4 *)(out + q8s_row_q(r, cols) + Q8_BLOCK * b);
    dq[0] = make_uint4(v[0], v[1], v[2], v[3]);
    dq[1] = make_uint4(v[4], v[5], v[6], v[7]);
    ((uint16_t *)(out + q8s_row_d(r, cols)))[b] = h[0];
}

void q8_launch_repack(q8_stream_t stream, const void *q8, long rows, long cols, void *out)
{
    const long n = rows * (cols / Q8_BLOCK);
    repack_s<<<dim3((unsigned)((n + 255) / 256)), 256, 0, (hipStream_t)stream>>>((const uint8_t *)q8, rows, cols, (uint8_t *)out);
}

/* ---------------------------------------------------------------- rows and the greedy next token */

/* z[i][k] = q * d of row rows[i] (src/card/rt.c:484-501: q converted, times the block scale, one
 * rounding; exact, since d*q has at most 19 significant bits). One thread per 4 columns. An index
 * outside [0, nrows) reads nothing and gives a row of NaN: the indices are device data, which the
 * host cannot check before the launch. */
__global__ __launch_bounds__(256) void q8_rows_k(const uint8_t *__restrict__ w, long cols, long nrows, const long *__restrict__ rows, long n,
                                                 float *__restrict__ z)
{
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const long per = cols / 4;
    if (i >= n * per)
        return;
    const long k = i / per, c4 = 4 * (i % per);
    const long r = rows[k];
    if (r < 0 || r >= nrows) {
        const float nan = __builtin_nanf("");
        *(float4 *)(z + k * cols + c4) = make_float4(nan, nan, nan, nan);
        return;
    }
    const uint32_t q = *(const uint32_t *)(w + q8s_row_q(r, cols) + c4);
    const float d = q8_half(((const uint16_t *)(w + q8s_row_d(r, cols)))[c4 / Q8_BLOCK]);
    *(float4 *)(z + k * cols + c4) = make_float4(q8_s8(q, 0) * d, q8_s8(q, 1) * d, q8_s8(q, 2) * d, q8_s8(q, 3) * d);
}

void q8_launch_rows(q8_stream_t stream, const void *w, long cols, long nrows, const long *rows, long n, float *z)
{
    const long m = n * (cols / 4);
    q8_rows_k<<<dim3((unsigned)((m + 255) / 256)), 256, 0, (hipStream_t)stream>>>((const uint8_t *)w, cols, nrows, rows, n, z);
}

/* The greedy next token of the reference's Next = {w index-of max/w} (src/apl/qwen35.apl:161; the
 * host's rt_maxv then rt_index_of, src/card/rt.c:137-165): m = the fmaxf fold of a, then the lowest
 * i whose bits equal m's. Pass 1: each workgroup's 4096 elements give (its m, its lowest such i);
 * pass 2, one workgroup: m over the candidates, then the lowest candidate i with m's bits. The
 * workgroup holding the first index of the global maximum has that maximum as its own. */
#define ARG_CHUNK 4096
__device__ __forceinline__ void argmax_block(float m, long idx, float *sm, long *si, float *out_m, long *out_i)
{
    /* m: fmaxf over the block, in a fixed tree */
    sm[threadIdx.x] = m;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if ((int)threadIdx.x < o)
            sm[threadIdx.x] = fmaxf(sm[threadIdx.x], sm[threadIdx.x + o]);
        __syncthreads();
    }
    const float bm = sm[0];
    __syncthreads();
    /* the lowest index whose value has bm's bits */
    si[threadIdx.x] = __builtin_bit_cast(uint32_t, m) == __builtin_bit_cast(uint32_t, bm) ? idx : LONG_MAX;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if ((int)threadIdx.x < o)
            si[threadIdx.x] = si[threadIdx.x] < si[threadIdx.x + o] ? si[threadIdx.x] : si[threadIdx.x + o];
        __syncthreads();
    }
    if (threadIdx.x == 0)
        *out_m = bm, *out_i = si[0];
}

__global__ __launch_bounds__(256) void argmax1(const float *__restrict__ a, long n, float *__restrict__ cm, long *__restrict__ ci)
{
    __shared__ float sm[256];
    __shared__ long si[256];
    const long b0 = (long)blockIdx.x * ARG_CHUNK;
    const long b1 = b0 + ARG_CHUNK < n ? b0 + ARG_CHUNK : n;
    /* each thread: fmaxf of its elements, then the lowest of its indices with that value's bits */
    float m = a[b0];
    for (long i = b0 + threadIdx.x; i < b1; i += 256)
        m = fmaxf(m, a[i]);
    long idx = LONG_MAX;
    for (long i = b0 + threadIdx.x; i < b1; i += 256)
        if (__builtin_bit_cast(uint32_t, a[i]) == __builtin_bit_cast(uint32_t, m)) {
            idx = i;
            break;
        }
    /* a thread whose range does not hold its own m (the a[b0] start) offers no index */
    argmax_block(idx == LONG_MAX ? a[b0] : m, idx, sm, si, cm + blockIdx.x, ci + blockIdx.x);
}

__global__ __launch_bounds__(256) void argmax2(const float *__restrict__ cm, const long *__restrict__ ci, long nc, long *__restrict__ out)
{
    __shared__ float sm[256];
    __shared__ long si[256];
    float m = cm[0];
    for (long i = threadIdx.x; i < nc; i += 256)
        m = fmaxf(m, cm[i]);
    long idx = LONG_MAX;
    for (long i = threadIdx.x; i < nc; i += 256)
        if (__builtin_bit_cast(uint32_t, cm[i]) == __builtin_bit_cast(uint32_t, m)) {
            idx = ci[i];
            break;
        }
    float om;
    argmax_block(idx == LONG_MAX ? cm[0] : m, idx, sm, si, &om, out);
}

long q8_argmax_chunks(long n) { return (n + ARG_CHUNK - 1) / ARG_CHUNK; }

void q8_launch_argmax(q8_stream_t stream, const float *a, long n, float *cm, long *ci, long *out)
{
    const long nc = q8_argmax_chunks(n);
    argmax1<<<dim3((unsigned)nc), 256, 0, (hipStream_t)stream>>>(a, n, cm, ci);
    argmax2<<<1, 256, 0, (hipStream_t)stream>>>(cm, ci, nc, out);
}

/* ---------------------------------------------------------------- synthetic inputs */

/* splitmix64's finaliser: a bijection of 64-bit words with full avalanche */
__device__ __forceinline__ uint64_t mix64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

__device__ __forceinline__ uint64_t hash3(uint64_t seed, uint64_t a, uint64_t b)
{
    return mix64(mix64(seed ^ mix64(a + 0x9e3779b97f4a7c15ull)) + b);
}

/* uniform in (0, 1]: 24 random bits */
__device__ __forceinline__ float unit_open(uint32_t v) { return ((float)(v >> 8) + 1.0f) * (1.0f / 16777216.0f); }

/* N(0,1) by Box-Muller from one 64-bit word */
__device__ __forceinline__ float normal01(uint64_t h)
{
    const float u1 = unit_open((uint32_t)h), u2 = unit_open((uint32_t)(h >> 32));
    return sqrtf(-2.0f * logf(u1)) * cosf(6.2831853071795864f * u2);
}

/* One thread per block: scale from hash(seed, row, block), then 32 q uniform in [-127, 127]
 * from 16 more words (the high 32 bits times 255, shifted: bias below 2^-24). */
__global__ __launch_bounds__(256) void fill_q8(uint8_t *__restrict__ dst, long rows, long cols, uint64_t seed, int dist, float mu, float sigma)
{
    const long nb = cols / Q8_BLOCK;
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * nb)
        return;
    const long r = i / nb, b = i % nb;
    const float z = normal01(hash3(seed, (uint64_t)r, (uint64_t)b * 64u));
    const float dv = dist == 0 ? fabsf(z) * sigma / 127.0f : expf(mu + sigma * z);
    const _Float16 d16 = (_Float16)dv;
    uint16_t out[17];
    out[0] = __builtin_bit_cast(uint16_t, d16);
    for (int k = 0; k < 16; k++) {
        const uint64_t h = hash3(seed, (uint64_t)r, (uint64_t)b * 64u + 1u + (uint64_t)k);
        const int q0 = (int)(((h >> 32) * 255u) >> 32) - 127;
        const int q1 = (int)(((h & 0xffffffffu) * 255u) >> 32) - 127;
        out[1 + k] = (uint16_t)((uint8_t)(int8_t)q0 | (uint16_t)(uint8_t)(int8_t)q1 << 8);
    }
    uint16_t *p = (uint16_t *)(dst + i * Q8_BLOCK_BYTES);
    for (int k = 0; k < 17; k++)
        p[k] = out[k];
}

void q8_launch_fill(q8_stream_t stream, void *dst, long rows, long cols, uint64_t seed, int dist, float mu, float sigma)
{
    const long n = rows * (cols / Q8_BLOCK);
    fill_q8<<<dim3((unsigned)((n + 255) / 256)), 256, 0, (hipStream_t)stream>>>((uint8_t *)dst, rows, cols, seed, dist, mu, sigma);
}

__global__ __launch_bounds__(256) void fill_f32(float *__restrict__ dst, long n, uint64_t seed)
{
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n)
        dst[i] = normal01(hash3(seed, 0x5eedull, (uint64_t)i));
}

void q8_launch_fill_f32(q8_stream_t stream, float *dst, long n, uint64_t seed)
{
    fill_f32<<<dim3((unsigned)((n + 255) / 256)), 256, 0, (hipStream_t)stream>>>(dst, n, seed);
}

/* dst = src, n16 16-byte words, one per thread: every byte read once and written once, which
 * makes it the yardstick for the HBM byte counters. */
__global__ __launch_bounds__(256) void copy16(uint4 *__restrict__ dst, const uint4 *__restrict__ src, long n16)
{
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n16)
        dst[i] = src[i];
}

void q8_launch_copy(q8_stream_t stream, void *dst, const void *src, long n16)
{
    copy16<<<dim3((unsigned)((n16 + 255) / 256)), 256, 0, (hipStream_t)stream>>>((uint4 *)dst, (const uint4 *)src, n16);
}

/* The decode product's loads at one token and nothing else: the floor a product of that shape
 * and grid cannot go below. Workgroup b of NW waves reads what gemv_k<1, RW, 1, NW, PAIR> reads for
 * its rows [b*RW, +RW): x (the lane's 16 columns, four 16-byte loads), then each row's 16 bytes of
 * weights and its binary16 scale (both matrices with PAIR), every load issued at once; the lane adds
 * every 32-bit word it loaded (the scale zero-extended) into a wrapping sum, the wave's lanes are
 * added, the NW waves' through LDS, and one thread stores the workgroup's sum to sink[blockIdx.x]:
 * the product's own end (a sum over lanes and waves, one barrier, a store) without its arithmetic.
 * The sums make the loads live and give a checksum the tests recompute. */
template <int RW, int NW, int PAIR, int MT>
__global__ __launch_bounds__(64 * NW) void read_k(const uint8_t *__restrict__ w0, const uint8_t *__restrict__ w1, long cols, const float *__restrict__ x,
                                                  long x_stride, unsigned *sink)
{
    constexpr int P = PAIR + 1;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const long u0 = (long)wave * 64 + lane, r0 = (long)blockIdx.x * RW;
    uint4 xv[MT][4];
#pragma unroll
    for (int m = 0; m < MT; m++)
#pragma unroll
        for (int c = 0; c < 4; c++)
            xv[m][c] = *(const uint4 *)(x + m * x_stride + 16 * u0 + 4 * c);
    uint4 q[RW][P];
    uint16_t dh[RW][P];
#pragma unroll
    for (int r = 0; r < RW; r++)
#pragma unroll
        for (int p = 0; p < P; p++) {
            const uint8_t *w = p ? w1 : w0;
            q[r][p] = *(const uint4 *)(w + q8s_row_q(r0 + r, cols) + 16 * u0);
            dh[r][p] = ((const uint16_t *)(w + q8s_row_d(r0 + r, cols)))[u0 >> 1];
        }
    __builtin_amdgcn_sched_barrier(0);
    unsigned acc = 0;
#pragma unroll
    for (int m = 0; m < MT; m++)
#pragma unroll
        for (int c = 0; c < 4; c++)
            acc += xv[m][c].x + xv[m][c].y + xv[m][c].z + xv[m][c].w;
#pragma unroll
    for (int r = 0; r < RW; r++)
#pragma unroll
        for (int p = 0; p < P; p++)
            acc += q[r][p].x + q[r][p].y + q[r][p].z + q[r][p].w + (unsigned)dh[r][p];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1)
        acc += (unsigned)__shfl_xor((int)acc, off, 64);
    __shared__ unsigned red[NW];
    if (lane == 0)
        red[wave] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned v = red[0];
#pragma unroll
        for (int k = 1; k < NW; k++)
            v += red[k];
        sink[blockIdx.x] = v;
    }
}

/* the decode kernel's grid for a product at t tokens (gemv_choose), or false when no instance
 * takes it: at one token the shapes of the decode tokens' products (cols a multiple of 1024), at 2
 * to 4 the 9B verify shapes (the fused pair 12288 x 4096 and down 4096 x 12288) */
int q8_launch_read(q8_stream_t stream, const void *w0, const void *w1, long rows, long cols, const float *x, long x_stride, long t, unsigned *sink)
{
    const long kb = cols % 1024 ? 0 : cols / 1024;
    if (t < 1 || t > 4)
        return -1;
    int rw, nw;
    gemv_choose(w1 != nullptr, (int)t, rows, kb, &rw, &nw);
    if (!kb || rows % rw || kb != nw)
        return -1;
    hipStream_t s = (hipStream_t)stream;
    const uint8_t *a = (const uint8_t *)w0, *b = (const uint8_t *)w1;
#define RD(RW_, NW_, P_, MT_)                                                                                          \
    if (t == MT_ && rw == RW_ && nw == NW_ && (b != nullptr) == (P_ == 1)) {                                           \
        Q8_LAUNCH(q8_time_name("read_k", 4, RW_, NW_, P_, MT_), (read_k<RW_, NW_, P_, MT_>), dim3((unsigned)(rows / RW_)), dim3(64 * NW_), s, a, b,   \
                  cols, x, x_stride, sink);                                                                            \
        return 0;                                                                                                      \
    }
    RD(8, 4, 0, 1) RD(8, 12, 0, 1) RD(4, 4, 1, 1) RD(8, 2, 0, 1) RD(4, 2, 0, 1) RD(2, 2, 0, 1) RD(4, 6, 0, 1) RD(2, 6, 0, 1) RD(2, 2, 1, 1)
    RD(4, 2, 1, 1) RD(8, 6, 0, 1)
    RD(8, 4, 1, 2) RD(8, 4, 1, 3) RD(8, 4, 1, 4) RD(16, 12, 0, 2) RD(16, 12, 0, 3) RD(16, 12, 0, 4)
#undef RD
    return -1;
}

/* *flag = seq, stored by lane 0 with release order at system scope: the host sees it after every
 * store of the kernels before this one on the stream (each kernel's end writes back its stores). */
__global__ void set_flag(unsigned *flag, unsigned seq)
{
    if (threadIdx.x == 0)
        __hip_atomic_store(flag + threadIdx.x, seq + threadIdx.x, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

void q8_launch_flag(q8_stream_t stream, unsigned *flag, unsigned seq)
{
    set_flag<<<1, 64, 0, (hipStream_t)stream>>>(flag, seq);
}

/* ---------------------------------------------------------------- primitive gates */

/* o8[i] = fma(x8[i], s8(q[i]), c8[i]) through the product kernels' byte convert (four bytes
 * a word, as they load them); of[i] = fma(xf[i], half(h[i]), cf[i]). n8 % 4 == 0. */
__global__ __launch_bounds__(256) void prims(const int8_t *__restrict__ q, const float *__restrict__ x8, const float *__restrict__ c8, float *__restrict__ o8,
                                             long n8, const uint16_t *__restrict__ h, const float *__restrict__ xf, const float *__restrict__ cf,
                                             float *__restrict__ of, long nf)
{
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (4 * i < n8) {
        const uint32_t w = ((const uint32_t *)q)[i];
#pragma unroll
        for (int k = 0; k < 4; k++)
            o8[4 * i + k] = __builtin_fmaf(x8[4 * i + k], q8_s8(w, k), c8[4 * i + k]);
    }
    if (i < nf)
        of[i] = __builtin_fmaf(xf[i], q8_half(h[i]), cf[i]);
}

void q8_launch_prims(q8_stream_t stream, const int8_t *q, const float *x8, const float *c8, float *o8, long n8, const uint16_t *h, const float *xf,
                     const float *cf, float *of, long nf)
{
    const long n = nf > n8 / 4 ? nf : n8 / 4;
    prims<<<dim3((unsigned)((n + 255) / 256)), 256, 0, (hipStream_t)stream>>>(q, x8, c8, o8, n8, h, xf, cf, of, nf);
}
