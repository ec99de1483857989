/* q8_gemm.hip: Y = X W^T for t >= 5 tokens on the matrix cores (v_mfma_f32_16x16x32_bf16).
 *
 * One Q8_0 block is 32 columns: exactly the K of one 16x16x32 MFMA, so a block's partial sum
 * S[token][row] = sum_k x[token][k] q[row][k] comes out of the matrix core whole and the block
 * scale is applied after it, acc = fma(S, d, acc), as the reference applies it after its
 * 32-column chain (src/card/gemm.c:20-23).
 *
 * Operands. q (|q| <= 128) is exact in bf16. x is not: each F32 x is split into three bf16
 * limbs x = hi + mid + lo by truncation (hi = x's top 16 bits, r = x - hi exactly, mid = r's top
 * 16 bits, lo = r - mid exactly, and lo has at most 8 significant bits), so the three MFMAs
 * hi*q + mid*q + lo*q see every bit of x; each product is exact and the matrix core adds them
 * in F32. Accuracy is that of an F32 sum, far inside NRMSE 1e-5.
 *
 * Layouts (lane l of a wave): A = x limbs, A[m][k] at lane m + 16*(k/8), item k%8 (m = token);
 * B = weights, B[k][n] at lane n + 16*(k/8), item k%8 (n = row of W: 8 bytes of row n of form
 * S, one global_load_dwordx2); D[m][n] at lane n + 16*(m/4), item m%4. So each lane needs the
 * scale of one row per block, and x_split's A tiles are 1 KiB each, read whole by a wave.
 *
 *   xsplit      x F32 [t cols] -> the limbs in A layout, tokens padded to 16 with zeros:
 *               xs[((tt*nb + b)*3 + limb)*64 + lane] = 8 bf16 (one uint4)
 *   gemm_mfma   a workgroup of 4 waves owns 4*RT row tiles of 16 rows (waves split rows, so the
 *               four read the same x tiles: one L2 read, three L1 hits) and a range of blocks;
 *               with the blocks split over KS workgroups, each writes its partial Y to a
 *               workspace with device-scope stores, and the last of the KS to finish (a
 *               counter per row tile, atomically incremented once the workgroup's stores are
 *               acknowledged) reads the KS partials with device-scope loads, adds them in
 *               split order and writes Y. The same order every run: deterministic. The last
 *               one also resets the counter, so the counters stay zero between products. */
#include <hip/hip_runtime.h>

#include <stdio.h>
#include <stdlib.h>

#include "q8_device.h"

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

/* bf16 bits (the top half) of two F32 values that are exact in bf16, packed a | b << 16 */
__device__ __forceinline__ uint32_t pack_hi(float a, float b)
{
    return __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, b), __builtin_bit_cast(uint32_t, a), 0x07060302u);
}

/* Column order inside a block. A lane loads 16 bytes of one row: columns [64c + 16kq, +16),
 * half of block 2c for kq < 2 (lanes 0-31), half of block 2c+1 for kq >= 2 (lanes 32-63). Two
 * v_permlane32_swap (lanes l and l + 32 trade a dword) leave every lane 8 bytes of each block:
 * for both, lane group kq holds the block's columns KCOL(kq) .. KCOL(kq) + 7 with
 * KCOL = {0, 16, 8, 24}. The x limbs are written in the same order, so each MFMA still sums
 * over the block's 32 columns exactly once. */
__host__ __device__ constexpr int kcol(int kq) { return 8 * ((kq & 1) * 2 + (kq >> 1)); }

/* ---------------------------------------------------------------- x -> bf16 limbs */

/* xs[((tt*nbp + b)*3 + limb)*64 + lane], nbp = nb rounded up to even (the odd block's partner is
 * zeros), tokens padded to 16 with zeros */
__global__ __launch_bounds__(256) void xsplit(const float *__restrict__ x, long x_stride, long t, long cols, long mt, uint4 *__restrict__ xs)
{
    const long nb = cols / Q8_BLOCK, nbp = (nb + 1) & ~1L;
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= mt * nbp * 64)
        return;
    const int lane = (int)(i & 63);
    const long b = (i >> 6) % nbp, tt = (i >> 6) / nbp;
    const long tok = tt * 16 + (lane & 15);
    const long k0 = b * Q8_BLOCK + kcol(lane >> 4);
    float v[8];
    if (tok < t && b < nb) {
        const float4 a = *(const float4 *)(x + tok * x_stride + k0), c = *(const float4 *)(x + tok * x_stride + k0 + 4);
        v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = c.x, v[5] = c.y, v[6] = c.z, v[7] = c.w;
    } else {
#pragma unroll
        for (int j = 0; j < 8; j++)
            v[j] = 0.0f;
    }
    uint32_t h[4], m[4], o[4];
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
        float hi[2], mid[2], lo[2];
#pragma unroll
        for (int e = 0; e < 2; e++) {
            hi[e] = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, v[j + e]) & 0xffff0000u);
            const float r = v[j + e] - hi[e];
            mid[e] = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, r) & 0xffff0000u);
            lo[e] = r - mid[e];
        }
        h[j / 2] = pack_hi(hi[0], hi[1]);
        m[j / 2] = pack_hi(mid[0], mid[1]);
        o[j / 2] = pack_hi(lo[0], lo[1]);
    }
    uint4 *dst = xs + ((tt * nbp + b) * 3) * 64 + lane;
    dst[0] = make_uint4(h[0], h[1], h[2], h[3]);
    dst[64] = make_uint4(m[0], m[1], m[2], m[3]);
    dst[128] = make_uint4(o[0], o[1], o[2], o[3]);
}

/* ---------------------------------------------------------------- the product */

/* 8 int8 (two dwords) to 8 bf16 */
__device__ __forceinline__ bf16x8 q8_bf16(uint32_t a, uint32_t b)
{
    return __builtin_bit_cast(bf16x8, make_uint4(pack_hi((float)(int8_t)a, (float)(int8_t)(a >> 8)), pack_hi((float)(int8_t)(a >> 16), (float)(int8_t)(a >> 24)),
                                                 pack_hi((float)(int8_t)b, (float)(int8_t)(b >> 8)), pack_hi((float)(int8_t)(b >> 16), (float)(int8_t)(b >> 24))));
}

/* The MFMAs of one block for a wave's RT row tiles and MT token tiles: wb[r] the row tiles'
 * weights, d[r] their scales (0 for a block past the end), xa the block's x limbs. */
template <int MT, int RT>
__device__ __forceinline__ void mfma_block(const bf16x8 (&wb)[RT], const float (&d)[RT], const uint4 (&xa)[MT][3], f32x4 (&acc)[RT][MT])
{
#pragma unroll
    for (int r = 0; r < RT; r++)
#pragma unroll
        for (int m = 0; m < MT; m++) {
            f32x4 p = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, xa[m][0]), wb[r], f32x4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
            p = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, xa[m][1]), wb[r], p, 0, 0, 0);
            p = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, xa[m][2]), wb[r], p, 0, 0, 0);
#pragma unroll
            for (int j = 0; j < 4; j++)
                acc[r][m][j] = __builtin_fmaf(p[j], d[r], acc[r][m][j]);
        }
}

/* x limbs of block b for the MT token tiles */
template <int MT>
__device__ __forceinline__ void load_x(uint4 (&xa)[MT][3], const uint4 *xs, long nbp, long b, int lane)
{
#pragma unroll
    for (int m = 0; m < MT; m++)
#pragma unroll
        for (int l = 0; l < 3; l++)
            xa[m][l] = xs[((m * nbp + b) * 3 + l) * 64 + lane];
}

/* Y (ks == 1) or this split's partial (ks > 1) from the accumulators of the waves that write, for
 * token tiles [tt0/16.., +MT); with ks > 1 the last workgroup of a row range (counter cnt) sums the
 * splits. rows_wg: the workgroup's rows, from row tile*rows_wg. Partials: part[split][token][row]
 * over all the product's padded tokens, so token groups of one row range share nothing. */
template <int MT, int RT>
__device__ __forceinline__ void gemm_out(const f32x4 (&acc)[RT][MT], bool writer, long rt0, long rows, long t, long tt0, int ks, int split, long cnt,
                                         long tile, long rows_wg, float *__restrict__ part, uint32_t *__restrict__ counters, float *__restrict__ y)
{
    const int lane = threadIdx.x & 63, n = lane & 15, kq = lane >> 4;
    /* lane holds D[token 16m + 4*kq + j][row 16*(rt0+r) + n] */
    if (ks == 1) {
        if (!writer)
            return;
#pragma unroll
        for (int r = 0; r < RT; r++)
#pragma unroll
            for (int m = 0; m < MT; m++)
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const long tok = 16 * (tt0 + m) + 4 * kq + j;
                    if (tok < t)
                        y[tok * rows + (rt0 + r) * 16 + n] = acc[r][m][j];
                }
        return;
    }
    /* split K: part[split][token (16*MT)][rows]. The partials go out as device-scope stores (sc1:
     * through this XCD's L2 to where every XCD reads), every lane waits for its own to be
     * acknowledged, and only then does the workgroup count itself in; the last one in reads
     * them as device-scope loads. No whole-L2 write-back or invalidate (an agent-scope fence)
     * is needed, and none is made: hundreds of workgroups serialise on those. */
    const long tp = (t + 15) / 16 * 16;
#pragma unroll
    for (int r = 0; r < (writer ? RT : 0); r++)
#pragma unroll
        for (int m = 0; m < MT; m++)
#pragma unroll
            for (int j = 0; j < 4; j++)
                if (16 * (tt0 + m) < tp) /* a group's tile past the last holds no tokens */
                    __hip_atomic_store(&part[((long)split * tp + 16 * (tt0 + m) + 4 * kq + j) * rows + (rt0 + r) * 16 + n], acc[r][m][j], __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
    __shared__ uint32_t last;
    __builtin_amdgcn_s_waitcnt(0); /* this lane's stores acknowledged */
    __syncthreads();
    if (threadIdx.x == 0)
        last = __hip_atomic_fetch_add(&counters[cnt], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (uint32_t)(ks - 1);
    __syncthreads();
    if (!last)
        return;
    /* the last workgroup: its rows x its tokens, summed in split order */
    const long r0 = tile * rows_wg;
    const long nr = rows - r0 < rows_wg ? rows - r0 : rows_wg;
    const long tok0 = 16 * tt0, nt = t - tok0 < 16 * MT ? t - tok0 : 16 * MT;
    const long n_out = nt * nr;
    /* four outputs a thread at a time, every split's load of them issued before the sums */
    for (long i0 = threadIdx.x; i0 < n_out; i0 += 4 * (long)blockDim.x) {
        float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int s0 = 0; s0 < ks; s0 += 8) {
            float ld[8][4];
#pragma unroll
            for (int s = 0; s < 8; s++)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const long i = i0 + e * (long)blockDim.x;
                    const long tok = tok0 + i / nr, row = r0 + i % nr;
                    ld[s][e] = s0 + s < ks && i < n_out
                                   ? __hip_atomic_load(&part[((long)(s0 + s) * tp + tok) * rows + row], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                   : 0.0f;
                }
#pragma unroll
            for (int s = 0; s < 8; s++)
#pragma unroll
                for (int e = 0; e < 4; e++)
                    v[e] = s0 + s == 0 ? ld[s][e] : s0 + s < ks ? v[e] + ld[s][e] : v[e];
        }
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const long i = i0 + e * (long)blockDim.x;
            if (i < n_out)
                y[(tok0 + i / nr) * rows + r0 + i % nr] = v[e];
        }
    }
    if (threadIdx.x == 0)
        __hip_atomic_store(&counters[cnt], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/* A workgroup of NW waves owns NW*RT row tiles of 16 rows (wave w: tiles [w*RT, +RT)), KP pairs
 * of blocks (split s: pairs [s*KP, +KP)) and MT token tiles (from token tile tt0 = blockIdx.y*MT).
 * Like the decode kernel, everything is issued at once: the x limbs of the range, then every
 * weight of the wave (KP pairs x RT row tiles, 16 B a lane); a memory-bound kernel is as fast as
 * the bytes it keeps in flight. The x limbs go to LDS once for the workgroup (x is issued first:
 * loads retire in order, so the LDS write waits for x only) and the NW waves read them there.
 * The ks workgroups of a row range are summed by the last to finish (gemm_out). */
template <int MT, int RT, int KP, int NW>
__global__ __launch_bounds__(64 * NW) void gemm_mfma(const uint8_t *__restrict__ w, long rows, long cols, const uint4 *__restrict__ xs, long t, int ks,
                                                     int cps, float *__restrict__ part, uint32_t *__restrict__ counters, float *__restrict__ y)
{
    constexpr int XN = MT * 2 * KP * 192;              /* uint4 of x limbs in the range */
    constexpr int XR = (XN + 64 * NW - 1) / (64 * NW); /* of them a thread */
    constexpr int DN = NW * RT * 16 * 2 * KP;          /* scales of the workgroup's rows in the range */
    constexpr int DR = (DN + 64 * NW - 1) / (64 * NW);
    __shared__ uint4 xl[XN];                           /* [tt][block in range][limb][lane] */
    __shared__ uint16_t dl[DN];                        /* [row of the workgroup][block in range] */
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const long nb = cols / Q8_BLOCK, nbp = (nb + 1) & ~1L, np = nbp / 2;
    const long tile = blockIdx.x / ks;
    const int split = (int)(blockIdx.x % ks);
    const long tt0 = (long)blockIdx.y * MT;
    const long rt0 = (tile * NW + wave) * RT;
    /* a wave past the last row tile reads row tile 0 and contributes nothing */
    const bool live = rt0 < rows / 16;
    const int n = lane & 15, kq = lane >> 4;

    f32x4 acc[RT][MT];
#pragma unroll
    for (int r = 0; r < RT; r++)
#pragma unroll
        for (int m = 0; m < MT; m++)
            acc[r][m] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    /* cps ranges of KP pairs a workgroup (one unless the K split would not fit its workspace) */
    for (int ch = 0; ch < cps; ch++) {
        const long c0 = ((long)split * cps + ch) * KP;
        /* x limbs of blocks [2*c0, 2*c0 + 2*KP) for token tiles [tt0, tt0 + MT), clamped to the matrix */
        uint4 xr[XR];
#pragma unroll
        for (int k = 0; k < XR; k++) {
            const int i = (int)threadIdx.x + 64 * NW * k;
            if (XN % (64 * NW) == 0 || i < XN) {
                const int tt = i / (2 * KP * 192), rem = i % (2 * KP * 192);
                long b = 2 * c0 + rem / 192;
                b = b < nbp ? b : nbp - 1;
                xr[k] = xs[((tt0 + tt) * nbp + b) * 192 + rem % 192];
            }
        }
        /* the scales of the workgroup's rows for the range: 2*KP consecutive threads read one row's
         * 2*KP consecutive binary16 (clamped to the matrix: a block past the end is zeroed below) */
        uint16_t dr[DR];
#pragma unroll
        for (int k = 0; k < DR; k++) {
            const int i = (int)threadIdx.x + 64 * NW * k;
            if (DN % (64 * NW) == 0 || i < DN) {
                long row = tile * NW * RT * 16 + i / (2 * KP);
                row = row < rows ? row : rows - 1;
                long b = 2 * c0 + i % (2 * KP);
                b = b < nb ? b : nb - 1;
                dr[k] = ((const uint16_t *)(w + q8s_row_d(row, cols)))[b];
            }
        }
        uint4 q[KP][RT];
#pragma unroll
        for (int p = 0; p < KP; p++) {
            const long c = c0 + p < np ? c0 + p : np - 1; /* clamped: a pair past the end is zeroed below */
#pragma unroll
            for (int r = 0; r < RT; r++) {
                const long row = live ? (rt0 + r) * 16 + n : n;
                q[p][r] = *(const uint4 *)(w + q8s_row_q(row, cols) + 16 * kq + 64 * c);
            }
        }
#pragma unroll
        for (int k = 0; k < XR; k++) {
            const int i = (int)threadIdx.x + 64 * NW * k;
            if (XN % (64 * NW) == 0 || i < XN)
                xl[i] = xr[k];
        }
#pragma unroll
        for (int k = 0; k < DR; k++) {
            const int i = (int)threadIdx.x + 64 * NW * k;
            if (DN % (64 * NW) == 0 || i < DN)
                dl[i] = dr[k];
        }
        __syncthreads();

#pragma unroll
        for (int p = 0; p < KP; p++) {
            const long c = c0 + p;
            const bool ok0 = live && c < np, ok1 = live && 2 * c + 1 < nb; /* block 2c, block 2c+1 */
            const bool keep = lane < 32 ? ok0 : ok1;
            bf16x8 wb[2][RT];
            float d[2][RT];
#pragma unroll
            for (int r = 0; r < RT; r++) {
                /* lanes 0-31 hold block 2c, 32-63 block 2c+1: trade dwords 0<->2 and 1<->3 across the halves */
                const uint32_t a0 = keep ? q[p][r].x : 0u, a1 = keep ? q[p][r].y : 0u, a2 = keep ? q[p][r].z : 0u, a3 = keep ? q[p][r].w : 0u;
                const auto s02 = __builtin_amdgcn_permlane32_swap(a0, a2, false, false);
                const auto s13 = __builtin_amdgcn_permlane32_swap(a1, a3, false, false);
                wb[0][r] = q8_bf16(s02[0], s13[0]);
                wb[1][r] = q8_bf16(s02[1], s13[1]);
                const int lr = (wave * RT + r) * 16 + n; /* the lane's row in the workgroup */
                d[0][r] = ok0 ? q8_half(dl[lr * 2 * KP + 2 * p]) : 0.0f;
                d[1][r] = ok1 ? q8_half(dl[lr * 2 * KP + 2 * p + 1]) : 0.0f;
            }
#pragma unroll
            for (int h = 0; h < 2; h++) {
                uint4 xa[MT][3];
#pragma unroll
                for (int m = 0; m < MT; m++)
#pragma unroll
                    for (int l = 0; l < 3; l++)
                        xa[m][l] = xl[((m * 2 * KP + 2 * p + h) * 3 + l) * 64 + lane];
                mfma_block<MT, RT>(wb[h], d[h], xa, acc);
            }
        }
        __syncthreads(); /* every wave done with xl before the next range overwrites it */
    }
    gemm_out<MT, RT>(acc, live, rt0, rows, t, tt0, ks, split, tile + (long)blockIdx.y * gridDim.x / ks, tile, 16L * NW * RT, part, counters, y);
}

/* ---------------------------------------------------------------- launchers */

long q8_gemm_xs_bytes(long cols, long t)
{
    const long nb = cols / Q8_BLOCK;
    return ((t + 15) / 16 + 1) * ((nb + 1) & ~1L) * 3 * 1024; /* one spare token tile: groups of 2 */
}

/* The instantiated configurations: MG token tiles a workgroup (the product's MT token tiles in
 * groups of MG, over blockIdx.y), RT row tiles a wave, KP pairs a workgroup, NW waves a workgroup.
 * x in LDS is MG * KP * 6 KiB. */
struct gemm_cfg {
    int mg, rt, kp, nw;
};
static const gemm_cfg CFGS[] = {{1, 1, 8, 8}, {1, 2, 8, 4}, {1, 1, 8, 4}, {1, 2, 4, 8}, {1, 1, 4, 8}, {1, 1, 16, 8}, {2, 1, 4, 8}, {2, 1, 8, 4}, {2, 2, 4, 4}};
#define NCFG ((int)(sizeof(CFGS) / sizeof(CFGS[0])))

/* Q8_GEMM_CFG = "MG,RT,KP,NW" picks an instantiated configuration, for tuning sweeps. */
static bool env_cfg(gemm_cfg *c)
{
    const char *v = getenv("Q8_GEMM_CFG");
    int a = 0, b = 0, d = 0, e = 0;
    if (!v || sscanf(v, "%d,%d,%d,%d", &a, &b, &d, &e) != 4)
        return false;
    for (int i = 0; i < NCFG; i++)
        if (CFGS[i].mg == a && CFGS[i].rt == b && CFGS[i].kp == d && CFGS[i].nw == e) {
            *c = CFGS[i];
            return true;
        }
    return false;
}

void q8_gemm_plan(long rows, long cols, long t, int *mg, int *rt, int *kp, int *nw, int *ks, int *cps)
{
    const long mt = (t + 15) / 16, rt16 = rows / 16;
    /* measured on the 9B FFN matrices: 16-pair ranges for one token tile, 4-pair ranges beyond */
    gemm_cfg c = mt == 1 ? CFGS[5] : CFGS[4];
    gemm_cfg e;
    if (env_cfg(&e) && e.mg <= mt)
        c = e;
    if (rt16 % c.rt)
        c = CFGS[0];
    const long tiles = (rows + 16L * c.nw * c.rt - 1) / (16L * c.nw * c.rt);
    const long np = ((cols / Q8_BLOCK) + 1) / 2;
    const long groups = (mt + c.mg - 1) / c.mg;
    const long ranges = (np + c.kp - 1) / c.kp;
    /* ranges a workgroup: one, unless the partials or the counters would not fit */
    long per = 1;
    while (per < ranges && ((ranges + per - 1) / per * mt * 16 * rows > Q8_GEMM_PART_MAX || tiles * groups > Q8_GEMM_COUNTERS))
        per++;
    *mg = c.mg, *rt = c.rt, *kp = c.kp, *nw = c.nw, *cps = (int)per;
    *ks = (int)((ranges + per - 1) / per);
}

long q8_gemm_part_floats(long rows, long cols, long t)
{
    int mg, rt, kp, nw, ks, cps;
    q8_gemm_plan(rows, cols, t, &mg, &rt, &kp, &nw, &ks, &cps);
    return ks > 1 ? (long)ks * ((t + 15) / 16) * 16 * rows : 0;
}

template <int MG, int RT, int KP, int NW>
static void gemm_go(hipStream_t s, const void *w, long rows, long cols, long t, float *y, void *xs, float *part, uint32_t *counters, int ks, int cps)
{
    const long tiles = (rows + 16L * NW * RT - 1) / (16L * NW * RT);
    const long groups = ((t + 15) / 16 + MG - 1) / MG;
    Q8_LAUNCH(q8_time_name("gemm_mfma", 4, MG, RT, KP, NW), (gemm_mfma<MG, RT, KP, NW>), dim3((unsigned)(tiles * ks), (unsigned)groups),
              dim3(64 * NW), s, (const uint8_t *)w, rows, cols, (const uint4 *)xs, t, ks, cps, part, counters, y);
}

void q8_launch_gemm_mfma(q8_stream_t stream, const void *w, long rows, long cols, const float *x, long x_stride, long t, float *y, void *xs, float *part,
                         uint32_t *counters)
{
    hipStream_t s = (hipStream_t)stream;
    int mg, rt, kp, nw, ks, cps;
    q8_gemm_plan(rows, cols, t, &mg, &rt, &kp, &nw, &ks, &cps);
    const long mt = (t + 15) / 16;
    /* token tiles past t hold zeros; a group's last tile may lie past mt (groups of MG): the
     * limbs are laid out for whole groups */
    const long mtp = (mt + mg - 1) / mg * mg;
    const long n = mtp * (((cols / Q8_BLOCK) + 1) & ~1L) * 64;
    xsplit<<<dim3((unsigned)((n + 255) / 256)), 256, 0, s>>>(x, x_stride, t, cols, mtp, (uint4 *)xs);
#define GO(G, R, P, N)                                                                                                 \
    if (mg == G && rt == R && kp == P && nw == N) {                                                                    \
        gemm_go<G, R, P, N>(s, w, rows, cols, t, y, xs, part, counters, ks, cps);                                      \
        return;                                                                                                        \
    }
    GO(1, 1, 8, 8) GO(1, 2, 8, 4) GO(1, 1, 8, 4) GO(1, 2, 4, 8) GO(1, 1, 4, 8) GO(1, 1, 16, 8) GO(2, 1, 4, 8) GO(2, 1, 8, 4) GO(2, 2, 4, 4)
#undef GO
    fprintf(stderr, "q8_gemm: no kernel for MG %d RT %d KP %d NW %d\n", mg, rt, kp, nw);
    abort();
}
