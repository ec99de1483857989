/* q8_mx.hip: the decode product for 3 and 4 tokens on the matrix cores (gemv_mx), and its launcher. */
#include <hip/hip_runtime.h>

#include <stdio.h>
#include <stdlib.h>

#include "q8_device.h"

typedef float q8_f32x4 __attribute__((ext_vector_type(4)));

/* The decode product for 3 and 4 tokens with the token products on the matrix cores
 * (v_mfma_f32_4x4x1_16b_f32): one instruction is 16 independent 4x4 outer products, block b of
 * lanes 4b..4b+3 adding A[i] B[j] to D[i][j], A[i] from lane 4b+i, B[j] from lane 4b+j, D[i][j]
 * in item i of lane 4b+j. Lane 4b+j holds token j's x and row j's weights (of a 4-row group) at
 * the same 64 columns, so each instruction takes the 4 tokens times 4 rows of one column per
 * block: 64 weights times 4 tokens, F32 products and sums as the decode kernel's fma chain, and
 * a weight is converted once (v_cvt_f32_i32) whatever the number of tokens. Tokens past MT are
 * not loaded and their outputs are dropped.
 *
 * Workgroup: NW waves, RGW groups of 4 rows, all of K = 1024*NW; wave w takes columns
 * [1024 w, +1024), lane 4b+j the 64 columns [1024 w + 64 b, +64). x is loaded once and kept in
 * registers; the weights then stream in steps of one matrix's 4 rows (the pair's gate and up of a
 * row group are two steps) through NB register buffers: the loads of step s+NB are issued as soon
 * as step s is computed, so each wave keeps NB steps in flight and computes every step while later
 * ones are still arriving (with all of a wave's loads issued at once, every wave's last load
 * lands near the end and the arithmetic runs after the memory instead of under it).
 *
 * The loads do not follow the lane layout: a quad holding four rows (or tokens) at one column
 * would touch four cache lines per quad and load, so each load reads 16 contiguous bytes a lane
 * of ONE row (token), 64 a quad, and a 4x4 transpose inside each quad (DPP) then gives every
 * lane its own row's (token's) bytes. A weight load is 1 KiB of one row, contiguous; an x load
 * 64 bytes a quad of one token. Each lane's scales (two blocks of its row) come from one
 * coalesced dword load of the 4 rows' scales and a ds_bpermute. Per 16 columns the 16
 * instructions accumulate from zero and the block scale is applied after them,
 * acc = fma(D, d, acc), per token as the reference applies it after its 32-column chain
 * (src/card/gemm.c:20-23). The lanes' partials are summed over b by DPP within each row of 16
 * lanes, then over the four lane rows and the NW waves in LDS, in a fixed order: the same every
 * run. */
template <int MT, int NW, int PAIR, int RGW, int NB, int EPI>
__global__ __launch_bounds__(64 * NW) void gemv_mx(const uint8_t *__restrict__ w0, const uint8_t *__restrict__ w1, long rows, long cols,
                                                   const float *__restrict__ x, long x_stride, float *y, const float *res)
{
    constexpr int P = PAIR + 1, OUT = P * 4 * MT;
    static_assert(RGW * 4 * MT <= 64 * NW, "one output a thread");
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int b = lane >> 2, j = lane & 3;
    const long r0 = (long)blockIdx.x * 4 * RGW;
    const long c0 = (long)wave * 1024; /* the wave's columns */
    /* thread k < 4*RGW*MT stores row r0 + k / MT, token k % MT; with the residual (EPI 2) it reads
     * that element of res here, with x, so that the read is no latency at the end (y may be res:
     * each element is read and then written by the one thread that owns it) */
    const int ko = (int)threadIdx.x % (4 * RGW * MT);
    const long yo = (long)(ko % MT) * rows + r0 + ko / MT;
    float rv = 0.0f;
    if constexpr (EPI == 2)
        rv = res[yo];

    /* x: load (h, c) is token h, floats [64 b + 16 c + 4 j, +4) of the wave's columns */
    uint4 xr[4][4]; /* [c][h] */
#pragma unroll
    for (int c = 0; c < 4; c++)
#pragma unroll
        for (int h = 0; h < 4; h++)
            xr[c][h] = h < MT ? *(const uint4 *)(x + h * x_stride + c0 + 64 * b + 16 * c + 4 * j) : make_uint4(0u, 0u, 0u, 0u);
    /* the weights stream in steps: step s is matrix s % P of row group s / P (the pair's gate and
     * up of a group are two steps), through NB register buffers, the loads of step s + NB issued as
     * soon as step s is computed. Load r of a step is row 4n + r, bytes [64 b + 16 j, +16) of the
     * wave's columns; lane L: the dword L & 15 (blocks 2(L & 15), +1) of row 4n + (L >> 4)'s 32
     * scales here */
    constexpr int ST = RGW * P;
    uint4 q[NB][4];
    uint32_t dl[NB];
#define Q8_MX_LOAD(s, k)                                                                                               \
    {                                                                                                                  \
        const int n_ = (s) / P;                                                                                        \
        const uint8_t *w = (s) % P ? w1 : w0;                                                                          \
        _Pragma("unroll") for (int r = 0; r < 4; r++) q[k][r] =                                                        \
            *(const uint4 *)(w + q8s_row_q(r0 + 4 * n_ + r, cols) + c0 + 64 * b + 16 * j);                              \
        dl[k] = *(const uint32_t *)(w + q8s_row_d(r0 + 4 * n_ + (lane >> 4), cols) + 2 * (c0 / 32) + 4 * (lane & 15));  \
    }
#pragma unroll
    for (int s = 0; s < NB && s < ST; s++) {
        Q8_MX_LOAD(s, s)
    }
    /* keep the loads where they are: left to itself the scheduler sinks them between the MFMAs to
     * save registers, and each wait then costs a memory round trip */
    __builtin_amdgcn_sched_barrier(0);

    /* lane 4b+j: xr[c][h] = token j, floats [64 b + 16 c + 4 h, +4) */
#pragma unroll
    for (int c = 0; c < 4; c++)
        q8_quad_transpose4(xr[c]);

    __shared__ float red[RGW][NW][4][OUT];
    q8_f32x4 acc[P];
#pragma unroll
    for (int s = 0; s < ST; s++) {
        const int k = s % NB, n = s / P, p = s % P;
        /* lane 4b+j: q[k][r] = row 4n + j, bytes [64 b + 16 r, +16); ds = the scales of blocks
         * 2b, 2b+1 of row 4n + j (from lane 16 j + b) */
        q8_quad_transpose4(q[k]);
        const uint32_t ds = (uint32_t)__builtin_amdgcn_ds_bpermute(4 * (16 * j + b), (int)dl[k]);
        acc[p] = q8_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const uint32_t qw[4] = {q[k][r].x, q[k][r].y, q[k][r].z, q[k][r].w};
            const uint32_t xw[16] = {xr[r][0].x, xr[r][0].y, xr[r][0].z, xr[r][0].w, xr[r][1].x, xr[r][1].y, xr[r][1].z, xr[r][1].w,
                                     xr[r][2].x, xr[r][2].y, xr[r][2].z, xr[r][2].w, xr[r][3].x, xr[r][3].y, xr[r][3].z, xr[r][3].w};
            q8_f32x4 dv = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int e = 0; e < 16; e++)
                dv = __builtin_amdgcn_mfma_f32_4x4x1f32(__builtin_bit_cast(float, xw[e]), q8_s8(qw[e >> 2], e & 3), dv, 0, 0, 0);
            const float d = q8_half((uint16_t)(ds >> (16 * (r >> 1))));
#pragma unroll
            for (int i = 0; i < 4; i++)
                acc[p][i] = __builtin_fmaf(dv[i], d, acc[p][i]);
        }
        if (p == P - 1) {
            /* over b within each row of 16 lanes: (v + ror 8) + ror 4 of that, every lane the sum
             * of the four lanes of its j; lanes 16R + j (R = 0..3) keep it for the LDS sum */
#pragma unroll
            for (int pp = 0; pp < P; pp++)
#pragma unroll
                for (int i = 0; i < MT; i++) {
                    float v = acc[pp][i];
                    v += Q8_DPP(v, 0x128); /* row_ror:8 */
                    v += Q8_DPP(v, 0x124); /* row_ror:4 */
                    if ((lane & 12) == 0)
                        red[n][wave][lane >> 4][(pp * 4 + j) * MT + i] = v;
                }
        }
        if (s + NB < ST) {
            __builtin_amdgcn_sched_barrier(0);
            Q8_MX_LOAD(s + NB, k)
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#undef Q8_MX_LOAD
    __syncthreads();
    if (threadIdx.x < 4 * RGW * MT) {
        const int n = ko / (4 * MT), jr = (ko / MT) % 4, i = ko % MT;
        float v[P];
#pragma unroll
        for (int p = 0; p < P; p++) {
            const int o = (p * 4 + jr) * MT + i;
            float a = 0.0f;
#pragma unroll
            for (int w = 0; w < NW; w++)
                a += (red[n][w][0][o] + red[n][w][1][o]) + (red[n][w][2][o] + red[n][w][3][o]);
            v[p] = a;
        }
        const float o = PAIR ? q8_swiglu(v[0], v[P - 1]) : v[0];
        y[yo] = EPI == 2 ? rv + o : o;
    }
}

/* The matrix-core decode kernel's row groups (of 4 rows) a workgroup, or 0 when it does not take
 * the shape: K a multiple of 1024 with 2, 4, 6, 8, 12 or 16 waves, rows a multiple of 4. The
 * largest of 4, 2, 1 that divides the row groups and leaves at least 3072 waves (3 a SIMD), else
 * 1. Measured on the 9B shapes: 4 for the gate+up pair (768 workgroups of 4 waves) and for down
 * (256 of 12). Q8_GEMV_MX = "1", "2" or "4" sends 3 and 4 tokens here with that many row
 * groups (for measuring it against the VALU kernel); unset or "0", they stay on the VALU kernel. */
static int mx_choose(long rows, long cols)
{
    const char *v = getenv("Q8_GEMV_MX"); /* read at every call: tests switch it */
    const int cached = v ? atoi(v) : -1;
    const long kb = cols % 1024 ? 0 : cols / 1024;
    if (cached == 0 || !(kb == 2 || kb == 4 || kb == 6 || kb == 8 || kb == 12 || kb == 16) || rows % 4)
        return 0;
    const long groups = rows / 4;
    if (cached == 1 || cached == 2 || cached == 4)
        return groups % cached == 0 ? cached : 0;
    for (int c = 4; c > 1; c /= 2)
        if (groups % c == 0 && groups / c * kb >= 3072)
            return c;
    return 1;
}

/* Whether the kernel takes t tokens of a product: a shape it runs (mx_choose), and only when
 * Q8_GEMV_MX sets the row groups. The VALU decode kernel, its lanes summed by q8_wave_sums, is
 * as fast or faster at every 9B shape measured at 3 and 4 tokens (4096x12288: 13.4 / 14.5 against
 * 16.2 / 16.8 us; the pair 12288x4096: 24.4 / 25.3 against 27.2 / 28.5; 6144x4096: 8.6 / 9.0
 * against 12.0 / 11.6; 151936x4096: 141 / 163 against 141 / 169), and keeps each token's bits
 * those of its one-token product. */
bool q8_gemv_mx_takes(long rows, long cols, long t, bool pair)
{
    (void)pair;
    if ((t != 3 && t != 4) || mx_choose(rows, cols) == 0)
        return false;
    const char *v = getenv("Q8_GEMV_MX");
    return v && atoi(v) > 0;
}

/* steps in flight a wave: 2 (the pair's gate and up of a row group, or two row groups) */
template <int MT, int PAIR, int RGW, int EPI>
static bool mx_go_nw(hipStream_t s, long kb, const uint8_t *a, const uint8_t *b, long rows, long cols, const float *x, long xs, float *y, const float *res)
{
    constexpr int NB = 2;
#define K1(N)                                                                                                          \
    if (kb == N) {                                                                                                     \
        Q8_LAUNCH(q8_time_name("gemv_mx", 6, MT, N, PAIR, RGW, NB, EPI), (gemv_mx<MT, N, PAIR, RGW, NB, EPI>), dim3((unsigned)(rows / (4 * RGW))),      \
                  dim3(64 * N), s, a, b, rows, cols, x, xs, y, res);                                                   \
        return true;                                                                                                   \
    }
    K1(2) K1(4) K1(6) K1(8) K1(12) K1(16)
#undef K1
    return false;
}

template <int MT, int PAIR, int EPI>
static bool mx_go(hipStream_t s, const uint8_t *a, const uint8_t *b, long rows, long cols, const float *x, long xs, float *y, const float *res)
{
    const long kb = cols / 1024;
    switch (mx_choose(rows, cols)) {
    case 1: return mx_go_nw<MT, PAIR, 1, EPI>(s, kb, a, b, rows, cols, x, xs, y, res);
    case 2: return mx_go_nw<MT, PAIR, 2, EPI>(s, kb, a, b, rows, cols, x, xs, y, res);
    case 4: return mx_go_nw<MT, PAIR, 4, EPI>(s, kb, a, b, rows, cols, x, xs, y, res);
    default: return false;
    }
}

bool q8_launch_gemv_mx(q8_stream_t stream, const void *w0, const void *w1, long rows, long cols, const float *x, long x_stride, long t, float *y,
                       const float *res)
{
    hipStream_t s = (hipStream_t)stream;
    const uint8_t *a = (const uint8_t *)w0, *b = (const uint8_t *)w1;
    if (!q8_gemv_mx_takes(rows, cols, t, w1 != nullptr) || (w1 && res))
        return false;
    if (w1)
        return t == 3 ? mx_go<3, 1, 0>(s, a, b, rows, cols, x, x_stride, y, nullptr) : mx_go<4, 1, 0>(s, a, b, rows, cols, x, x_stride, y, nullptr);
    if (res)
        return t == 3 ? mx_go<3, 0, 2>(s, a, b, rows, cols, x, x_stride, y, res) : mx_go<4, 0, 2>(s, a, b, rows, cols, x, x_stride, y, res);
    return t == 3 ? mx_go<3, 0, 0>(s, a, b, rows, cols, x, x_stride, y, nullptr) : mx_go<4, 0, 0>(s, a, b, rows, cols, x, x_stride, y, nullptr);
}
