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
 * Layouts (lane l of a wave): A = x limbs, A[m][k] at lane m + 16*(k/8) (m = token); B = weights,
 * B[k][n] at lane n + 16*(k/8) (n = row of W); D[m][n] at lane n + 16*(m/4), item m%4. So each
 * lane needs the scale of one row per block. Within a block the lane groups hold the columns
 * KCOL(kq) .. +7 (below), in both operands.
 *
 *   gemm_mfma   a workgroup of NW waves owns NW row tiles of 16 rows, its token tiles and a K
 *               slice of cps ranges of KP block pairs, which it streams: for each range it loads x
 *               (split into limbs on the way into LDS), its rows' scales (into LDS) and every weight
 *               of every wave, with the next range's loads in flight during this one's wait and
 *               MFMAs. With K split over ks workgroups, each writes a partial;
 *   gemm_xres   the same for one token tile (t <= 16), with the split's x limbs and scales put in
 *               LDS once, so the weights stream with no per-range wait or barrier;
 *   gemm_sum    adds the ks partials in split order: the same order every run, deterministic;
 *   gemm_xres_round, gemm_mfma_round
 *               a round of products sharing x in one launch, each product on its own K split;
 *   gemm_xres_pair
 *               two products of one shape at t <= 16 (the FFN's gate and up): a workgroup stages
 *               x once and streams both products' rows of its tile and split;
 *   gemm_sum_round, gemm_swiglu_round
 *               every product's partials of a round in split order (the fused pair's with its
 *               SwiGLU). */
#include <hip/hip_runtime.h>

#include <stdio.h>
#include <stdlib.h>

#include "q8_device.h"

#include "q8_bf16.h"

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

/* ranges a workgroup streams without draining its loads (one unrolled pipeline) */
#define GEMM_CHUNK 8

/* The loads of one range of KP pairs, held in registers from issue to commit. */
template <int MT, int RT, int KP, int NW, int NP = 1>
struct gemm_stage {
    static constexpr int XS = MT * 2 * KP * 64;               /* x lane slots: 8 values of one token each */
    static constexpr int XR = (XS + 64 * NW - 1) / (64 * NW); /* of them a thread */
    static constexpr int DN = NW * RT * 16 * 2 * KP;          /* scales of the workgroup's rows */
    static constexpr int DR = (DN + 64 * NW - 1) / (64 * NW);
    float4 xr[XR][2];
    bool xin[XR];
    uint16_t dr[NP][DR]; /* every product's scales */
    uint4 q[NP][KP][RT];  /* every product's weights */
};

/* A workgroup of NW waves owns NW*RT row tiles of 16 rows (wave w: tiles [w*RT, +RT)), MT token
 * tiles (from token tile tt0 = blockIdx.y*MT) and cps consecutive ranges of KP pairs of blocks
 * (split s: ranges [s*cps, +cps)). For each range it loads x (split into limbs on its way into
 * LDS, shared by the NW waves), its rows' scales (into LDS) and every weight of every wave, all
 * issued at once: a memory-bound kernel is as fast as the bytes it keeps in flight. The ranges
 * are software-pipelined: the loads of range ch+1 are issued into a second register set before
 * the MFMAs of range ch, so a workgroup streams its K slice with one range always in flight.
 * The ks workgroups of a row tile write partials that gemm_sum adds in split order. blk: the
 * workgroup's index in the product's grid along x (tile blk / ks, split blk % ks). */
template <int MT, int RT, int KP, int NW, int NP = 1>
__device__ __forceinline__ void mfma_body(const uint8_t *const (&w)[NP], long rows, long cols, const float *x, long x_stride, long t, int ks,
                                          int cps, float *const (&part)[NP], float *const (&y)[NP], const float *res, unsigned blk)
{
    typedef gemm_stage<MT, RT, KP, NW, NP> stage;
    constexpr int XS = stage::XS, XR = stage::XR, DN = stage::DN, DR = stage::DR;
    constexpr int XN = MT * 2 * KP * 192; /* uint4 of x limbs in a range */
    __shared__ uint4 xls[2][XN];          /* two ranges: [tt][block in range][limb][lane] */
    __shared__ uint16_t dls[2][NP * DN];  /* two ranges: [product][row of the workgroup][block in range] */
    const int lane = threadIdx.x & 63;
    /* the wave's index, uniform (see gemm_xres) */
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    /* block, pair and range indices in 32 bits (see gemm_xres) */
    const int nb = (int)(cols / Q8_BLOCK), np = (nb + 1) / 2;
    const long tile = blk / ks;
    const int split = (int)(blk % ks);
    const long tt0 = (long)blockIdx.y * MT;
    const long rt0 = (tile * NW + wave) * RT;
    /* a row tile past the last one (of a wave's RT, any but the first may be) reads row tile 0
     * and contributes nothing */
    const bool live = rt0 < rows / 16;
    auto live_r = [&](int r) { return rt0 + r < rows / 16; };
    const int n = lane & 15, kq = lane >> 4;

    /* issue every load of the range starting at pair c0. All are unconditional, from indices
     * clamped to the matrix; what lies past t, past the last block or past the last pair is zeroed
     * after the loads (a load under a branch would make the wave wait for it before the next). */
    auto issue = [&](stage &S, int c0) {
        /* x of blocks [2*c0, 2*c0 + 2*KP) for token tiles [tt0, tt0 + MT) */
#pragma unroll
        for (int k = 0; k < XR; k++) {
            const int i = (int)threadIdx.x + 64 * NW * k;
            const int L = i & 63, bb = (i >> 6) % (2 * KP), tt = (i >> 6) / (2 * KP);
            const long tok = 16 * (tt0 + tt) + (L & 15);
            const int b = 2 * c0 + bb;
            S.xin[k] = (XS % (64 * NW) == 0 || i < XS) && tok < t && b < nb;
            const float *px = x + (tok < t ? tok : t - 1) * x_stride + (long)(b < nb ? b : nb - 1) * Q8_BLOCK + kcol(L >> 4);
            S.xr[k][0] = *(const float4 *)px;
            S.xr[k][1] = *(const float4 *)(px + 4);
        }
        /* the scales: 2*KP consecutive threads read one row's 2*KP consecutive binary16 */
#pragma unroll
        for (int k = 0; k < DR; k++) {
            const int i = (int)threadIdx.x + 64 * NW * k;
            if (DN % (64 * NW) == 0 || i < DN) {
                long row = tile * NW * RT * 16 + i / (2 * KP);
                row = row < rows ? row : rows - 1;
                int b = 2 * c0 + i % (2 * KP);
                b = b < nb ? b : nb - 1;
#pragma unroll
                for (int pp = 0; pp < NP; pp++)
                    S.dr[pp][k] = ((const uint16_t *)(w[pp] + q8s_row_d(row, cols)))[b];
            }
        }
#pragma unroll
        for (int pp = 0; pp < NP; pp++)
#pragma unroll
            for (int p = 0; p < KP; p++) {
                const int c = c0 + p < np ? c0 + p : np - 1;
#pragma unroll
                for (int r = 0; r < RT; r++) {
                    /* the row tile at a uniform base, the lane's row and 16 bytes at a 32-bit offset */
                    const uint8_t *wt = w[pp] + q8s_row_q(live_r(r) ? (rt0 + r) * 16 : 0, cols) + 64L * c;
                    S.q[pp][p][r] = *(const uint4 *)(wt + (unsigned)(n * cols + 16 * kq));
                }
            }
    };
    /* the range's x limbs and scales into LDS buffer bf */
    auto commit = [&](const stage &S, int bf) {
        uint4 *xl = xls[bf];
        uint16_t *dl = dls[bf];
#pragma unroll
        for (int k = 0; k < XR; k++) {
            const int i = (int)threadIdx.x + 64 * NW * k;
            if (XS % (64 * NW) == 0 || i < XS) {
                const int L = i & 63, blk = i >> 6; /* blk = tt * 2KP + bb */
                const float4 z = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                uint4 h, m, o;
                xsplit8(S.xin[k] ? S.xr[k][0] : z, S.xin[k] ? S.xr[k][1] : z, h, m, o);
                xl[(blk * 3 + 0) * 64 + L] = h;
                xl[(blk * 3 + 1) * 64 + L] = m;
                xl[(blk * 3 + 2) * 64 + L] = o;
            }
        }
#pragma unroll
        for (int pp = 0; pp < NP; pp++)
#pragma unroll
            for (int k = 0; k < DR; k++) {
                const int i = (int)threadIdx.x + 64 * NW * k;
                if (DN % (64 * NW) == 0 || i < DN)
                    dl[pp * DN + i] = S.dr[pp][k];
            }
    };
    f32x4 acc[NP][RT][MT];
#pragma unroll
    for (int pp = 0; pp < NP; pp++)
#pragma unroll
        for (int r = 0; r < RT; r++)
#pragma unroll
            for (int m = 0; m < MT; m++)
                acc[pp][r][m] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    /* the MFMAs of the range starting at pair c0, from LDS buffer bf and the stage's weights */
    auto compute = [&](const stage &S, int bf, int c0) {
        const uint4 *xl = xls[bf];
        const uint16_t *dl = dls[bf];
#pragma unroll
        for (int p = 0; p < KP; p++) {
            const int c = c0 + p;
            const bool ok0 = c < np, ok1 = 2 * c + 1 < nb; /* block 2c, block 2c+1 */
            bf16x8 wb[NP][2][RT];
            float d[NP][2][RT];
#pragma unroll
            for (int pp = 0; pp < NP; pp++)
#pragma unroll
                for (int r = 0; r < RT; r++) {
                    /* a block past the matrix needs no masking: its x limbs in LDS are zero and a bf16 weight is
                     * finite, so its MFMAs give exactly 0 (its scale is zeroed below). Lanes 0-31 hold block 2c,
                     * 32-63 block 2c+1: trade dwords 0<->2 and 1<->3 across the halves */
                    const auto s02 = __builtin_amdgcn_permlane32_swap(S.q[pp][p][r].x, S.q[pp][p][r].z, false, false);
                    const auto s13 = __builtin_amdgcn_permlane32_swap(S.q[pp][p][r].y, S.q[pp][p][r].w, false, false);
                    wb[pp][0][r] = q8_bf16(s02[0], s13[0]);
                    wb[pp][1][r] = q8_bf16(s02[1], s13[1]);
                    const int lr = (wave * RT + r) * 16 + n; /* the lane's row in the workgroup */
                    const float d0 = q8_half(dl[pp * DN + lr * 2 * KP + 2 * p]), d1 = q8_half(dl[pp * DN + lr * 2 * KP + 2 * p + 1]);
                    d[pp][0][r] = ok0 && live_r(r) ? d0 : 0.0f;
                    d[pp][1][r] = ok1 && live_r(r) ? d1 : 0.0f;
                }
#pragma unroll
            for (int h = 0; h < 2; h++) {
                if constexpr (NP == 1) {
                    uint4 xa[MT][3];
#pragma unroll
                    for (int m = 0; m < MT; m++)
#pragma unroll
                        for (int l = 0; l < 3; l++)
                            xa[m][l] = xl[((m * 2 * KP + 2 * p + h) * 3 + l) * 64 + lane];
                    mfma_block<MT, RT>(wb[0][h], d[0][h], xa, acc[0]);
                } else {
                    /* a pair: one token tile's limbs at a time (12 registers, not 12 per tile), read once
                     * for both products' MFMAs, in the order of mfma_block for each product */
#pragma unroll
                    for (int m = 0; m < MT; m++) {
                        uint4 xa[1][3];
#pragma unroll
                        for (int l = 0; l < 3; l++)
                            xa[0][l] = xl[((m * 2 * KP + 2 * p + h) * 3 + l) * 64 + lane];
#pragma unroll
                        for (int pp = 0; pp < NP; pp++) {
                            f32x4 a1[RT][1];
#pragma unroll
                            for (int r = 0; r < RT; r++)
                                a1[r][0] = acc[pp][r][m];
                            mfma_block<1, RT>(wb[pp][h], d[pp][h], xa, a1);
#pragma unroll
                            for (int r = 0; r < RT; r++)
                                acc[pp][r][m] = a1[r][0];
                        }
                    }
                }
            }
        }
    };
    /* the pipeline over the split's cps ranges, in chunks of up to GEMM_CHUNK ranges: two
     * register sets and two LDS buffers taking turns. Issue range ch+1, then commit range ch
     * (waiting for its x and scales only) and compute it, so two ranges are in flight while the
     * wave waits. One barrier a range, after the commit: the commit of range ch+1 writes the
     * other LDS buffer, last read by range ch-1, which every wave finished before it passed the
     * barrier of range ch. A chunk is unrolled whole (no loop back edge inside it, where the
     * compiler's wait counting would drain the loads in flight), and a barrier closes it (the
     * next chunk starts on buffer 0 again). The issue is unconditional (past the chunk's last
     * range it loads that range again, from L2): under a branch, the wait before the commit
     * would also wait for the loads just issued. The scheduling barriers keep the compiler from
     * moving the loads off their place. */
    const int r0 = split * cps, nr = (np + KP - 1) / KP;
    const int mine = nr - r0 < cps ? nr - r0 : cps; /* the last split may hold fewer ranges */
    for (int base = 0; base < mine; base += GEMM_CHUNK) {
        const int nc = mine - base < GEMM_CHUNK ? mine - base : GEMM_CHUNK;
        const int rb = r0 + base;
        stage A, B;
        __builtin_amdgcn_sched_barrier(0);
        issue(A, rb * KP);
#pragma unroll
        for (int ch = 0; ch < GEMM_CHUNK; ch += 2) {
            __builtin_amdgcn_sched_barrier(0);
            issue(B, (rb + (ch + 1 < nc ? ch + 1 : nc - 1)) * KP);
            __builtin_amdgcn_sched_barrier(0);
            commit(A, 0);
            __syncthreads();
            compute(A, 0, (rb + ch) * KP);
            if (ch + 1 >= nc)
                break;
            __builtin_amdgcn_sched_barrier(0);
            issue(A, (rb + (ch + 2 < nc ? ch + 2 : nc - 1)) * KP);
            __builtin_amdgcn_sched_barrier(0);
            commit(B, 1);
            __syncthreads();
            compute(B, 1, (rb + ch + 1) * KP);
            if (ch + 2 >= nc)
                break;
        }
        __syncthreads(); /* every wave done with both buffers before the next chunk */
    }
    /* lane holds D[token 16(tt0+m) + 4*kq + j][row 16*(rt0+r) + n]: to Y (plus the residual when
     * res is given), or to this split's partial, part[split][token][row] over the product's padded
     * tokens (summed by gemm_sum) */
    if (!live)
        return;
    const long tp = (t + 15) / 16 * 16;
#pragma unroll
    for (int pp = 0; pp < NP; pp++)
#pragma unroll
        for (int r = 0; r < RT; r++) {
            if (!live_r(r))
                continue;
#pragma unroll
            for (int m = 0; m < MT; m++)
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const long tok = 16 * (tt0 + m) + 4 * kq + j;
                    if (ks == 1) {
                        const long i = tok * rows + (rt0 + r) * 16 + n;
                        if (tok < t)
                            y[pp][i] = res ? res[i] + acc[pp][r][m][j] : acc[pp][r][m][j];
                    } else if (tok < tp) {
                        part[pp][((long)split * tp + tok) * rows + (rt0 + r) * 16 + n] = acc[pp][r][m][j];
                    }
                }
        }
}

template <int MT, int RT, int KP, int NW>
__global__ __launch_bounds__(64 * NW) void gemm_mfma(const uint8_t *w, long rows, long cols, const float *x, long x_stride, long t, int ks, int cps,
                                                     float *part, float *y, const float *res)
{
    const uint8_t *const wv[1] = {w};
    float *const pv[1] = {part}, *const yv[1] = {y};
    mfma_body<MT, RT, KP, NW>(wv, rows, cols, x, x_stride, t, ks, cps, pv, yv, res, blockIdx.x);
}

/* A round of products sharing x (17 <= t <= 64) as one launch: workgroup (b, g) runs position
 * (b - start[p], g) of product p's grid at this launch's NW, on the product's own K split */
template <int MT, int RT, int KP, int NW>
__global__ __launch_bounds__(64 * NW) void gemm_mfma_round(q8_gemm_round r, long cols, const float *x, long x_stride, long t)
{
    int p = 0;
#pragma unroll
    for (int k = 1; k < Q8_ROUND_MAX; k++)
        if (k < r.n && (long)blockIdx.x >= r.start[k])
            p = k;
    const uint8_t *const wv[1] = {(const uint8_t *)r.w[p]};
    float *const ov[1] = {r.out[p]};
    mfma_body<MT, RT, KP, NW>(wv, r.rows[p], cols, x, x_stride, t, r.ks[p], r.cps[p], ov, ov, nullptr, (unsigned)(blockIdx.x - r.start[p]));
}

/* The two products of a round of one shape (the FFN's gate and up) at 17 <= t <= 64: each range's
 * x goes to LDS once for both, and each wave reads a block's x limbs once for both products'
 * MFMAs. Each product's sums are those of its own launch, in the same order. */
template <int MT, int RT, int KP, int NW>
__global__ __launch_bounds__(64 * NW) void gemm_mfma_pair(q8_gemm_round r, long cols, const float *x, long x_stride, long t)
{
    const uint8_t *const wv[2] = {(const uint8_t *)r.w[0], (const uint8_t *)r.w[1]};
    float *const ov[2] = {r.out[0], r.out[1]};
    mfma_body<MT, RT, KP, NW, 2>(wv, r.rows[0], cols, x, x_stride, t, r.ks[0], r.cps[0], ov, ov, nullptr, blockIdx.x);
}

/* One token tile (t <= 16) with x resident in LDS. A workgroup of NW waves owns NW row tiles
 * (wave w: row tile tile*NW + w) and the split's cps ranges of KP pairs, taken in segments of up
 * to SC ranges. For a segment, the workgroup first puts x of the segment's blocks (split into
 * limbs, only the lanes that hold a token's values load them) and its rows' scales into LDS, one
 * barrier; then each wave streams its weights through two register sets (range ch+1's loads in
 * flight during range ch's MFMAs) with no further synchronisation. gemm_mfma instead loads x and
 * the scales for every range, and waits for them and for a barrier before each range's MFMAs.
 * The sums are gemm_mfma's in the same order, so on the same split the two give the same bits.
 * blk: the workgroup's index in the product's grid (tile blk / ks, split blk % ks). */
template <int KP, int NW, int SC, int NP = 1>
__device__ __forceinline__ void xres_body(const uint8_t *const (&w)[NP], long rows, long cols, const float *x, long x_stride, long t, int ks,
                                          int cps, float *const (&part)[NP], float *const (&y)[NP], const float *res, unsigned blk)
{
    constexpr int BS = 2 * KP * SC;                     /* blocks of a segment */
    constexpr int XS = 64 * BS;                         /* x lane slots of a segment: 8 values of one token */
    constexpr int XR = (XS + 64 * NW - 1) / (64 * NW);  /* of them a thread */
    constexpr int DN = NW * 16 * BS;                    /* scales of a segment */
    constexpr int DR = (DN + 64 * NW - 1) / (64 * NW);
    constexpr int DP = BS + 2;                          /* scale row pitch in LDS (halves): an odd dword count, no bank conflicts */
    __shared__ uint4 xls[BS * 3 * 64];                  /* [block][limb][lane] */
    constexpr int DL = NW * 16 * DP;                    /* a product's scales in LDS (halves) */
    __shared__ uint16_t dls[NP * DL];                   /* [product][row of the workgroup][block] */
    const int lane = threadIdx.x & 63;
    /* the wave's index, uniform: everything derived from it (the row tile, whether the wave is
     * live, the range tests) stays in scalar registers */
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    /* block, pair and range indices in 32 bits: gfx9 compares 64-bit values only in vector registers */
    const int nb = (int)(cols / Q8_BLOCK), np = (nb + 1) / 2;
    const long tile = blk / ks;
    const int split = (int)(blk % ks);
    const long rt0 = tile * NW + wave;
    /* a wave past the last row tile reads row tile 0 and contributes nothing */
    const bool live = rt0 < rows / 16;
    const int n = lane & 15, kq = lane >> 4;
    /* the row tile's weights at a uniform base; the lane's row and 16 bytes at a 32-bit offset */
    const uint8_t *wt[NP];
#pragma unroll
    for (int pp = 0; pp < NP; pp++)
        wt[pp] = w[pp] + q8s_row_q(live ? rt0 * 16 : 0, cols);
    const unsigned woff = (unsigned)(n * cols + 16 * kq);

    /* acc: the sums of the product being streamed (product 0 at a segment's start); oth: the other
     * product's of a pair */
    f32x4 acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f}, oth = acc;
    const int r0 = split * cps, nr = (np + KP - 1) / KP;
    const int mine = nr - r0 < cps ? nr - r0 : cps; /* the last split may hold fewer ranges */
    for (int sb = 0; sb < mine; sb += SC) {
        const int nc = mine - sb < SC ? mine - sb : SC;
        const int c00 = (r0 + sb) * KP, b0 = 2 * c00; /* the segment's first pair and block */
        /* step e of the segment's stream: the range of product pe it reads (a pair streams product
         * 0's nc ranges, then product 1's); past the last step, the last range again */
        auto step = [&](int e, int &pe) {
            pe = NP == 2 && e >= nc ? 1 : 0;
            const int rr = e - pe * nc;
            return rr < nc ? rr : nc - 1;
        };
        uint4 q[2][KP];
        float4 xr[XR][2];
        uint16_t dr[NP][DR];
        /* every load of the segment's x and scales, then ranges 0 and 1's weights, all unconditional
         * from clamped indices (what lies past t or past the last block is zeroed after the loads):
         * two ranges in flight while the x limbs are made, as during the stream */
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int k = 0; k < XR; k++) {
            const int s = (int)threadIdx.x + 64 * NW * k;
            const int L = s & 63, bs = s >> 6, tok = L & 15;
            int b = b0 + (bs < BS ? bs : BS - 1);
            b = b < nb ? b : nb - 1;
            const float *px = x + (tok < t ? tok : t - 1) * x_stride + (long)b * Q8_BLOCK + kcol(L >> 4);
            xr[k][0] = *(const float4 *)px;
            xr[k][1] = *(const float4 *)(px + 4);
        }
#pragma unroll
        for (int pp = 0; pp < NP; pp++)
#pragma unroll
            for (int k = 0; k < DR; k++) {
                const int s = (int)threadIdx.x + 64 * NW * k;
                long row = tile * NW * 16 + s / BS;
                row = row < rows ? row : rows - 1;
                int b = b0 + s % BS;
                b = b < nb ? b : nb - 1;
                dr[pp][k] = ((const uint16_t *)(w[pp] + q8s_row_d(row, cols)))[b];
            }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int h = 0; h < 2; h++) {
            int ph;
            const int rr = step(h, ph);
            const uint8_t *wh = NP == 2 && ph ? wt[NP - 1] : wt[0];
#pragma unroll
            for (int p = 0; p < KP; p++) {
                int c = c00 + rr * KP + p;
                c = c < np ? c : np - 1;
                q[h][p] = *(const uint4 *)(wh + 64L * c + woff);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        /* the segment's x limbs and scales into LDS (waits for them, not for the weights) */
#pragma unroll
        for (int k = 0; k < XR; k++) {
            const int s = (int)threadIdx.x + 64 * NW * k;
            if (XS % (64 * NW) == 0 || s < XS) {
                const int L = s & 63, bs = s >> 6, tok = L & 15;
                const bool in = tok < t && b0 + bs < nb && bs < 2 * KP * nc;
                const float4 z = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                uint4 h, m, o;
                xsplit8(in ? xr[k][0] : z, in ? xr[k][1] : z, h, m, o);
                xls[(bs * 3 + 0) * 64 + L] = h;
                xls[(bs * 3 + 1) * 64 + L] = m;
                xls[(bs * 3 + 2) * 64 + L] = o;
            }
        }
#pragma unroll
        for (int pp = 0; pp < NP; pp++)
#pragma unroll
            for (int k = 0; k < DR; k++) {
                const int s = (int)threadIdx.x + 64 * NW * k;
                if (DN % (64 * NW) == 0 || s < DN)
                    dls[pp * DL + (s / BS) * DP + s % BS] = dr[pp][k];
            }
        __syncthreads();
        /* the segment's ranges, unrolled whole (a loop back edge would drain the loads in flight):
         * range ch's MFMAs (range ch+1 in flight), then range ch+2 issued into its registers (past
         * the last, range nc-1 again, from L2). A pair's 2 SC steps skip what lies past its last
         * rather than leave the loop: the compiler unrolls a loop with an early exit whole only up
         * to 8 steps */
#pragma unroll
        for (int e = 0; e < NP * SC; e++) {
            if (NP == 1 && e >= nc)
                break;
            if (NP == 2 && e >= 2 * nc)
                continue;
            const int pe = NP == 2 && e >= nc ? 1 : 0, ch = e - pe * nc;
            if (NP == 2 && e == nc) { /* product 1's ranges from here: its sums in acc, product 0's aside */
                const f32x4 a = acc;
                acc = oth;
                oth = a;
            }
            const uint16_t *dl = dls + (NP == 2 && pe ? DL : 0);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int p = 0; p < KP; p++) {
                const int c = c00 + ch * KP + p;
                const bool ok0 = live && c < np, ok1 = live && 2 * c + 1 < nb; /* block 2c, block 2c+1 */
                const uint4 qq = q[e & 1][p];
                /* A block past the matrix (its weights loaded from a clamped index) needs no masking:
                 * its x limbs in LDS are zero, and a bf16 weight is finite, so its MFMAs give exactly
                 * 0; its scale is zeroed below, in case the clamped block's scale is not finite.
                 * Lanes 0-31 hold block 2c, 32-63 block 2c+1: trade dwords 0<->2 and 1<->3 across the halves */
                const auto s02 = __builtin_amdgcn_permlane32_swap(qq.x, qq.z, false, false);
                const auto s13 = __builtin_amdgcn_permlane32_swap(qq.y, qq.w, false, false);
                const bf16x8 wb[2] = {q8_bf16(s02[0], s13[0]), q8_bf16(s02[1], s13[1])};
                const int bs = 2 * (ch * KP + p), lr = wave * 16 + n; /* block 2c in the segment, the lane's row in the workgroup */
                const float d0 = q8_half(dl[lr * DP + bs]), d1 = q8_half(dl[lr * DP + bs + 1]);
                const float d[2] = {ok0 ? d0 : 0.0f, ok1 ? d1 : 0.0f};
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const uint4 *xa = xls + (bs + h) * 3 * 64 + lane;
                    f32x4 pr = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, xa[0]), wb[h], f32x4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
                    pr = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, xa[64]), wb[h], pr, 0, 0, 0);
                    pr = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, xa[128]), wb[h], pr, 0, 0, 0);
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        acc[j] = __builtin_fmaf(pr[j], d[h], acc[j]);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            if (e + 2 < NP * SC) {
                int pn;
                const int nx = step(e + 2, pn);
                const uint8_t *wn = NP == 2 && pn ? wt[NP - 1] : wt[0];
#pragma unroll
                for (int p = 0; p < KP; p++) {
                    int c = c00 + nx * KP + p;
                    c = c < np ? c : np - 1;
                    q[e & 1][p] = *(const uint4 *)(wn + 64L * c + woff);
                }
            }
        }
        if (NP == 2) { /* product 0's sums back in acc for the next segment */
            const f32x4 a = acc;
            acc = oth;
            oth = a;
        }
        __syncthreads(); /* every wave done with the segment's LDS before the next segment writes it */
    }
    /* lane holds D[token 4*kq + j][row 16*rt0 + n], as in gemm_mfma */
    if (!live)
        return;
    const long tp = (t + 15) / 16 * 16;
#pragma unroll
    for (int pp = 0; pp < NP; pp++) {
        const f32x4 a = pp ? oth : acc;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const long tok = 4 * kq + j;
            if (ks == 1) {
                const long i = tok * rows + rt0 * 16 + n;
                if (tok < t)
                    y[pp][i] = res ? res[i] + a[j] : a[j];
            } else if (tok < tp) {
                part[pp][((long)split * tp + tok) * rows + rt0 * 16 + n] = a[j];
            }
        }
    }
}

template <int KP, int NW, int SC>
__global__ __launch_bounds__(64 * NW) void gemm_xres(const uint8_t *w, long rows, long cols, const float *x, long x_stride, long t, int ks, int cps,
                                                     float *part, float *y, const float *res)
{
    const uint8_t *const wv[1] = {w};
    float *const pv[1] = {part}, *const yv[1] = {y};
    xres_body<KP, NW, SC>(wv, rows, cols, x, x_stride, t, ks, cps, pv, yv, res, blockIdx.x);
}

/* A round of products that share x (and t <= 16) as one launch: workgroup b belongs to product p
 * with start[p] <= b < start[p+1] and runs position b - start[p] of that product's grid at this
 * launch's NW, on the product's own K split, so every product gets the bits of its own launch. */
template <int KP, int NW, int SC>
__global__ __launch_bounds__(64 * NW) void gemm_xres_round(q8_gemm_round r, long cols, const float *x, long x_stride, long t)
{
    int p = 0;
#pragma unroll
    for (int k = 1; k < Q8_ROUND_MAX; k++)
        if (k < r.n && (long)blockIdx.x >= r.start[k])
            p = k;
    const uint8_t *const wv[1] = {(const uint8_t *)r.w[p]};
    float *const ov[1] = {r.out[p]};
    xres_body<KP, NW, SC>(wv, r.rows[p], cols, x, x_stride, t, r.ks[p], r.cps[p], ov, ov, nullptr, (unsigned)(blockIdx.x - r.start[p]));
}

/* The two products of a round of one shape (the FFN's gate and up) in one workgroup a tile and
 * split: the split's x limbs go to LDS once for both, and the waves stream product 0's ranges,
 * then product 1's, through the same two register sets (product 1's first ranges in flight during
 * product 0's last). Each product's sums are those of its own launch, in the same order; the
 * workgroups of the pair are half those of the two products' own grids. */
template <int KP, int NW, int SC>
__global__ __launch_bounds__(64 * NW) void gemm_xres_pair(q8_gemm_round r, long cols, const float *x, long x_stride, long t)
{
    const uint8_t *const wv[2] = {(const uint8_t *)r.w[0], (const uint8_t *)r.w[1]};
    float *const ov[2] = {r.out[0], r.out[1]};
    xres_body<KP, NW, SC, 2>(wv, r.rows[0], cols, x, x_stride, t, r.ks[0], r.cps[0], ov, ov, nullptr, blockIdx.x);
}

/* The floor of gemm_xres: its grid, segments, barriers and loads (x, the scales, the weights
 * through two register sets, range ch+2 issued after range ch is used), and no arithmetic but a
 * checksum: the wrapping sum of every x word as loaded, every scale once and every weight word
 * once (a clamped or repeated load is not added: a wave past the last row tile, a pair or block
 * past the row, a scale slot past the segment or the matrix, the re-issue past the last range).
 * Each workgroup adds its sum to sink[0]. */
template <int KP, int NW, int SC>
__global__ __launch_bounds__(64 * NW) void read_xres(const uint8_t *w, long rows, long cols, const float *x, long x_stride, long t, int ks, int cps,
                                                     unsigned *sink)
{
    constexpr int BS = 2 * KP * SC, XS = 64 * BS, XR = (XS + 64 * NW - 1) / (64 * NW);
    constexpr int DN = NW * 16 * BS, DR = (DN + 64 * NW - 1) / (64 * NW);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int nb = (int)(cols / Q8_BLOCK), np = (nb + 1) / 2;
    const long tile = blockIdx.x / ks;
    const int split = (int)(blockIdx.x % ks);
    const long rt0 = tile * NW + wave;
    const bool live = rt0 < rows / 16;
    const int n = lane & 15, kq = lane >> 4;
    const uint8_t *wt = w + q8s_row_q(live ? rt0 * 16 : 0, cols);
    const unsigned woff = (unsigned)(n * cols + 16 * kq);
    unsigned acc = 0;
    const int r0 = split * cps, nr = (np + KP - 1) / KP;
    const int mine = nr - r0 < cps ? nr - r0 : cps;
    for (int sb = 0; sb < mine; sb += SC) {
        const int nc = mine - sb < SC ? mine - sb : SC;
        const int c00 = (r0 + sb) * KP, b0 = 2 * c00;
        uint4 q[2][KP];
        uint4 xr[XR][2];
        uint16_t dr[DR];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int k = 0; k < XR; k++) {
            const int s = (int)threadIdx.x + 64 * NW * k;
            const int L = s & 63, bs = s >> 6, tok = L & 15;
            int b = b0 + (bs < BS ? bs : BS - 1);
            b = b < nb ? b : nb - 1;
            const float *px = x + (tok < t ? tok : t - 1) * x_stride + (long)b * Q8_BLOCK + kcol(L >> 4);
            xr[k][0] = *(const uint4 *)px;
            xr[k][1] = *(const uint4 *)(px + 4);
        }
#pragma unroll
        for (int k = 0; k < DR; k++) {
            const int s = (int)threadIdx.x + 64 * NW * k;
            long row = tile * NW * 16 + s / BS;
            row = row < rows ? row : rows - 1;
            int b = b0 + s % BS;
            b = b < nb ? b : nb - 1;
            dr[k] = ((const uint16_t *)(w + q8s_row_d(row, cols)))[b];
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int p = 0; p < KP; p++) {
                int c = c00 + (h < nc ? h : nc - 1) * KP + p;
                c = c < np ? c : np - 1;
                q[h][p] = *(const uint4 *)(wt + 64L * c + woff);
            }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int k = 0; k < XR; k++)
#pragma unroll
            for (int i = 0; i < 2; i++)
                acc += xr[k][i].x + xr[k][i].y + xr[k][i].z + xr[k][i].w;
#pragma unroll
        for (int k = 0; k < DR; k++) {
            const int s = (int)threadIdx.x + 64 * NW * k, bs = s % BS;
            if ((DN % (64 * NW) == 0 || s < DN) && tile * NW * 16 + s / BS < rows && bs < 2 * KP * nc && b0 + bs < nb)
                acc += dr[k];
        }
        __syncthreads(); /* where gemm_xres waits for its LDS image */
#pragma unroll
        for (int ch = 0; ch < SC; ch++) {
            if (ch >= nc)
                break;
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int p = 0; p < KP; p++) {
                const int c = c00 + ch * KP + p;
                const uint4 v = q[ch & 1][p];
                if (live && c < np && 2 * c + (kq >> 1) < nb)
                    acc += v.x + v.y + v.z + v.w;
            }
            __builtin_amdgcn_sched_barrier(0);
            if (ch + 2 < SC) {
                const int nx = ch + 2 < nc ? ch + 2 : nc - 1;
#pragma unroll
                for (int p = 0; p < KP; p++) {
                    int c = c00 + nx * KP + p;
                    c = c < np ? c : np - 1;
                    q[ch & 1][p] = *(const uint4 *)(wt + 64L * c + woff);
                }
            }
        }
        __syncthreads();
    }
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
        __hip_atomic_fetch_add(sink, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

/* output i's sum of the ks partials (splits step floats apart), in split order: sixteen splits'
 * loads in flight at a time, all issued before the first add (past the last split the index is
 * clamped and the value not added) */
__device__ __forceinline__ float split_sum(const float *__restrict__ part, int ks, long step, long i)
{
    float v = 0.0f;
    for (int s0 = 0; s0 < ks; s0 += 16) {
        float a[16];
#pragma unroll
        for (int k = 0; k < 16; k++)
            a[k] = part[(long)(s0 + k < ks ? s0 + k : ks - 1) * step + i];
#pragma unroll
        for (int k = 0; k < 16; k++)
            if (s0 + k < ks)
                v = s0 + k == 0 ? a[0] : v + a[k];
    }
    return v;
}

/* Y = the sum of the ks partials in split order, one thread an output (the kernel boundary
 * before it makes every split's stores visible), plus the residual when res is given (res may be Y) */
__global__ __launch_bounds__(256) void gemm_sum(const float *__restrict__ part, int ks, long t, long tp, long rows, float *y, const float *res)
{
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= t * rows)
        return;
    const float r = res ? res[i] : 0.0f;
    const float v = split_sum(part, ks, tp * rows, i);
    y[i] = res ? r + v : v;
}

/* the sums of a round's products: output i of the round belongs to product p with ostart[p] <= i <
 * ostart[p+1]; a product of one split wrote its Y itself */
__global__ __launch_bounds__(256) void gemm_sum_round(q8_gemm_round r, long tp)
{
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    int p = 0;
#pragma unroll
    for (int k = 1; k < Q8_ROUND_MAX; k++)
        if (k < r.n && i >= r.ostart[k])
            p = k;
    if (i >= r.ostart[r.n] || r.ks[p] == 1)
        return;
    const long j = i - r.ostart[p];
    r.y[p][j] = split_sum(r.out[p], r.ks[p], tp * r.rows[p], j);
}

/* The fused pair's end: y[i] = SiLU(G[i]) * U[i], with G and U the gate's and the up product's sums
 * (products 0 and 1 of the round, the same shape): their split sums in split order, or the Y a
 * product of one split wrote itself; the same sums and SwiGLU as the two products and the
 * elementwise kernel apart */
__global__ __launch_bounds__(256) void gemm_swiglu_round(q8_gemm_round r, long tp, float *y)
{
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= r.ostart[1])
        return;
    const float g = r.ks[0] > 1 ? split_sum(r.out[0], r.ks[0], tp * r.rows[0], i) : r.y[0][i];
    const float u = r.ks[1] > 1 ? split_sum(r.out[1], r.ks[1], tp * r.rows[1], i) : r.y[1][i];
    y[i] = q8_swiglu(g, u);
}

/* ---------------------------------------------------------------- launchers */

/* The instantiated configurations of gemm_mfma: MG token tiles a workgroup (the product's MT token
 * tiles in groups of MG, over blockIdx.y), RT row tiles a wave, KP pairs a range, NW waves a
 * workgroup. x in LDS is MG * KP * 12 KiB (two ranges). Measured on the 9B FFN matrices (12288 x
 * 4096 and 4096 x 12288): 2-pair ranges and every token tile in one workgroup, so that the
 * weights are read once; 8 waves at two token tiles, 16 at three and four. One token tile runs on
 * gemm_xres (x resident); gemm_mfma<1, 1, 2, 16> computes the same sums and is kept for the tests
 * that hold the two to the same bits. */
struct gemm_cfg {
    int mg, rt, kp, nw;
};
/* 16 waves (256 rows) a workgroup, or 12 (192 rows) for the shapes where that leaves fewer compute
 * units idle (nw_of); the 12-wave instances of one token tile are the streaming twins of the
 * x-resident kernel's */
#define GEMM_CFGS(X) X(1, 1, 2, 16) X(2, 1, 2, 8) X(3, 1, 2, 16) X(4, 1, 2, 16) X(1, 1, 2, 12) X(3, 1, 2, 12) X(4, 1, 2, 12)
/* the streaming configurations that also run as a pair (two products of one shape sharing each
 * range's x and each block's x limb reads), as X(MG, RT, KP, NW, the pair's KP): those whose pair
 * kernel spills nothing and leaves the single kernel's waves a SIMD. The pair may stream ranges of
 * fewer pairs than the plan's (the split's cps ranges of KP pairs as KP / PK times as many ranges:
 * the same blocks in the same order, so the same bits), which halves the weights and x a stage
 * holds. A round of the 9B gate and up: 3 token tiles on 12 waves (152 registers) 49.5-50.5 /
 * 51.6-52.5 us a layer at 40 / 48 tokens against 54.0-55.5 / 56.4-57.8 as two products; 4 tiles
 * on 12 waves in ranges of one pair (112 registers) 67.2 against 70.2 us at 64 (in ranges of two
 * pairs it spilled 18 registers: 82.3 against 68.7). Measured and left out: 2 tiles on 8 waves,
 * 52.3-55.6 / 54.9-58.7 against 43.5-44.4 / 47.0-47.5 us at 24 / 32 tokens in ranges of two pairs
 * (132 registers, half the workgroups a CU) or one (113), and every 16-wave one (spills). */
#define GEMM_PAIR_CFGS(X) X(3, 1, 2, 12, 2) X(4, 1, 2, 12, 1)

/* the x-resident kernel for one token tile: 2-pair ranges, 16 or 12 waves, segments of 8 ranges
 * (x limbs 96 KiB and scales 13-17 KiB of LDS: one workgroup a CU) */
#define XRES_KP 2
#define XRES_SC 8

/* every configuration streams ranges of the same KP pairs, so a K split of cps ranges covers the
 * same blocks in each: the split, and so the bits, do not depend on the kernel */
#define GEMM_KP_CHECK(G, R, P, N) static_assert(P == XRES_KP, "every configuration ranges over XRES_KP pairs");
GEMM_CFGS(GEMM_KP_CHECK)
#undef GEMM_KP_CHECK

/* workgroups of a kernel resident on the device at once (occupancy x compute units), asked of the
 * runtime once a kernel (n caches it) */
template <typename K>
static long resident(K kernel, int threads, long &n)
{
    if (!n) {
        int per = 0, dev = 0, cus = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, kernel, threads, 0) != hipSuccess || hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || per < 1 || cus < 1) {
            fprintf(stderr, "q8_gemm: occupancy query failed\n");
            abort();
        }
        n = (long)per * cus;
    }
    return n;
}

/* a product's kernel and K split */
struct gemm_plan {
    gemm_cfg c;
    bool xres; /* gemm_xres (one token tile) rather than gemm_mfma<c> */
    int ks, cps;
};

/* resident workgroups of the x-resident kernel with nw waves (16 or 12) */
static long resident_xres(int nw)
{
    static long n16 = 0, n12 = 0;
    return nw == 12 ? resident(gemm_xres<XRES_KP, 12, XRES_SC>, 64 * 12, n12) : resident(gemm_xres<XRES_KP, 16, XRES_SC>, 64 * 16, n16);
}

/* The K split of a rows x cols matrix: ks splits of cps ranges of XRES_KP block pairs (the last may
 * hold fewer), a function of the shape alone (nw comes from the shape too), so that a token's
 * output has the same bits whatever the number of tokens it is computed with (5 to 64 a launch,
 * and every 64-token launch of a longer X). As many splits as fill the device with one resident
 * round of the x-resident kernel's workgroups (16 nw rows each), with at least two ranges a split
 * above 256 rows, fewer if the partials of a 64-token launch would not fit the workspace. Above
 * 256 rows one-range splits write and add more partials than their shorter streams save: 1024 x
 * 4096 at 16 splits of two ranges took 10.1 us at 16 tokens and 14.4 at 64, against 10.7 and 15.3
 * at 32 splits of one. At 256 rows or fewer the grid is a few workgroups on an otherwise idle
 * device, the product takes one workgroup's time, and a second range lengthens it (the two
 * 32 x 4096 products of a 64-token round took ~2 us more at two ranges a split). ks_force > 0 sets
 * the split count instead (a test hook: other splits, other bits). */
static void split_of(long rows, long cols, int nw, int ks_force, int *ks, int *cps)
{
    const long tiles = (rows + 16L * nw - 1) / (16L * nw);
    const long np = ((cols / Q8_BLOCK) + 1) / 2;
    const long ranges = (np + XRES_KP - 1) / XRES_KP;
    long split = ks_force > 0 ? ks_force : resident_xres(nw) / tiles;
    if (ks_force <= 0 && rows > 256 && split > ranges / 2)
        split = ranges / 2;
    split = split < 1 ? 1 : split > ranges ? ranges : split;
    long per = (ranges + split - 1) / split;
    while (per < ranges && (ranges + per - 1) / per * 64 * rows > Q8_GEMM_PART_MAX)
        per++;
    *cps = (int)per;
    *ks = (int)((ranges + per - 1) / per);
}

/* The waves a workgroup for a shape, 16 or 12, from the shape alone (so the split, and the bits,
 * stay independent of t): the one whose grid takes the fewest rounds of resident workgroups times
 * the rows and ranges a workgroup streams; 16 on a tie. At 12288 x 4096, 16 waves make 48 row
 * tiles x 5 splits = 240 workgroups of 256 rows x 7 ranges, 16 compute units idle; 12 make 64 x 4
 * = 256 of 192 rows x 8 ranges. At 4096 x 12288 16 waves fill the device (16 x 16 of 256 x 6). A
 * matrix of at most 192 rows is one row tile either way, with the same split and the same rows a
 * workgroup, so it ties and takes 16 waves, as a round's larger products do: the DeltaNet
 * quartet's 32-row products then share their launch. */
static int nw_of(long rows, long cols, int ks_force)
{
    long best = -1;
    int pick = 16;
    for (int nw : {16, 12}) {
        int ks, cps;
        split_of(rows, cols, nw, ks_force, &ks, &cps);
        const long tiles = (rows + 16L * nw - 1) / (16L * nw), res = resident_xres(nw);
        const long cost = (tiles * ks + res - 1) / res * (rows < 16L * nw ? rows : 16L * nw) * cps;
        if (best < 0 || cost < best) {
            best = cost;
            pick = nw;
        }
    }
    return pick;
}

static gemm_plan plan_of(long rows, long cols, long t, q8_gemm_opts o)
{
    const long mt = ((t < 64 ? t : 64) + 15) / 16;
    static const gemm_cfg CFG[5] = {{0, 0, 0, 0}, {1, 1, 2, 16}, {2, 1, 2, 8}, {3, 1, 2, 16}, {4, 1, 2, 16}};
    const int nw = nw_of(rows, cols, o.ks);
    gemm_plan p = {CFG[mt], mt == 1 && !o.streaming, 0, 0};
    if (mt != 2)
        p.c.nw = nw;
    split_of(rows, cols, nw, o.ks, &p.ks, &p.cps);
    return p;
}

long q8_gemm_part_floats(long rows, long cols, long t, q8_gemm_opts o)
{
    const gemm_plan p = plan_of(rows, cols, t, o);
    return p.ks > 1 ? (long)p.ks * (((t < 64 ? t : 64) + 15) / 16) * 16 * rows : 0;
}

/* a round's products: plans, partial regions (from part, or null to count), outputs; the floats of
 * partials it needs in *parts */
static void round_plan(int n, const void *const *w, const long *rows, long cols, long t, float *const *y, float *part, q8_gemm_opts o,
                       q8_gemm_round &all, gemm_plan *pl, long *parts)
{
    const long tp = (t + 15) / 16 * 16;
    long np = 0, outs = 0;
    all = q8_gemm_round{};
    all.n = n;
    for (int p = 0; p < n; p++) {
        pl[p] = plan_of(rows[p], cols, t, o);
        all.w[p] = w ? w[p] : nullptr;
        all.rows[p] = rows[p];
        all.ks[p] = pl[p].ks;
        all.cps[p] = pl[p].cps;
        all.y[p] = y ? y[p] : nullptr;
        all.ostart[p] = outs;
        outs += t * rows[p];
        if (pl[p].ks > 1) {
            all.out[p] = part ? part + np : nullptr;
            np += (long)pl[p].ks * tp * rows[p];
        } else {
            all.out[p] = all.y[p];
        }
    }
    all.ostart[n] = outs;
    *parts = np;
}

long q8_gemm_round_part_floats(int n, const long *rows, long cols, long t, q8_gemm_opts o)
{
    if (t < 1 || t > 64 || n < 2 || n > Q8_ROUND_MAX)
        return 0;
    q8_gemm_round all;
    gemm_plan pl[Q8_ROUND_MAX];
    long parts = 0;
    round_plan(n, nullptr, rows, cols, t, nullptr, nullptr, o, all, pl, &parts);
    return parts;
}

int q8_launch_gemm_round(q8_stream_t stream, int n, const void *const *w, const long *rows, long cols, const float *x, long x_stride, long t,
                         float *const *y, float *part, long part_cap, q8_gemm_opts o, float *pair_y)
{
    if (t < 1 || t > 64 || n < 2 || n > Q8_ROUND_MAX || (pair_y && (n != 2 || rows[0] != rows[1])))
        return -1;
    q8_gemm_round all;
    gemm_plan pl[Q8_ROUND_MAX];
    long parts = 0;
    round_plan(n, w, rows, cols, t, y, part, o, all, pl, &parts);
    if (parts > part_cap || (parts > 0 && !part))
        return -1;
    hipStream_t s = (hipStream_t)stream;
    /* one launch for the products of each kernel configuration (the x-resident kernel, or the
     * streaming kernel's MG, RT and KP: with these plans one launch for the whole round), at the
     * wave count of its largest product, then every product's sums. The waves a workgroup only
     * decide which rows a workgroup streams; each product keeps its own K split, and so the bits
     * of its own launch (the attention layer's K and V, 1024 x 4096, plan 12 waves alone and run
     * at Q's 16 in its round). Two products of one shape on the x-resident kernel (the FFN's gate
     * and up) run as a pair: one workgroup a tile and split for both, x staged once */
    bool launched[Q8_ROUND_MAX] = {};
    const gemm_cfg &q0 = pl[0].c, &q1 = pl[1].c;
    if (n == 2 && rows[0] == rows[1] && pl[0].xres == pl[1].xres && q0.mg == q1.mg && q0.rt == q1.rt && q0.kp == q1.kp && q0.nw == q1.nw &&
        all.ks[0] == all.ks[1] && all.cps[0] == all.cps[1]) {
        const int nw = q0.nw, rowsper = 16 * nw * (pl[0].xres ? 1 : q0.rt);
        const unsigned wgs = (unsigned)((rows[0] + rowsper - 1) / rowsper * all.ks[0]);
        bool ok = false;
        if (pl[0].xres) {
            if (nw == 12)
                Q8_LAUNCH(q8_time_name("gemm_xres_pair", 3, XRES_KP, 12, XRES_SC), (gemm_xres_pair<XRES_KP, 12, XRES_SC>), dim3(wgs), dim3(64 * 12), s,
                          all, cols, x, x_stride, t);
            else
                Q8_LAUNCH(q8_time_name("gemm_xres_pair", 3, XRES_KP, 16, XRES_SC), (gemm_xres_pair<XRES_KP, 16, XRES_SC>), dim3(wgs), dim3(64 * 16), s,
                          all, cols, x, x_stride, t);
            ok = true;
        } else {
            const unsigned groups = (unsigned)(((t + 15) / 16 + q0.mg - 1) / q0.mg);
#define GP(G, R, P, N, PK)                                                                                             \
    if (!ok && q0.mg == G && q0.rt == R && q0.kp == P && nw == N) {                                                    \
        q8_gemm_round pr = all; /* ranges of PK pairs: the split's cps ranges of P pairs as P / PK times as many */    \
        pr.cps[0] *= P / PK;                                                                                           \
        pr.cps[1] *= P / PK;                                                                                           \
        Q8_LAUNCH(q8_time_name("gemm_mfma_pair", 4, G, R, PK, N), (gemm_mfma_pair<G, R, PK, N>), dim3(wgs, groups), dim3(64 * N), s, pr, cols,  \
                  x, x_stride, t);                                                                                     \
        ok = true;                                                                                                     \
    }
            GEMM_PAIR_CFGS(GP)
#undef GP
        }
        launched[0] = launched[1] = ok;
    }
    for (int p0 = 0; p0 < n; p0++) {
        if (launched[p0])
            continue;
        const gemm_plan &c0 = pl[p0];
        auto same = [&](int p) {
            return !launched[p] && pl[p].xres == c0.xres && (c0.xres || (pl[p].c.mg == c0.c.mg && pl[p].c.rt == c0.c.rt && pl[p].c.kp == c0.c.kp));
        };
        int nw = c0.c.nw;
        for (long p = p0 + 1, big = rows[p0]; p < n; p++)
            if (same((int)p) && rows[p] > big) {
                big = rows[p];
                nw = pl[p].c.nw;
            }
        const int rowsper = 16 * nw * (c0.xres ? 1 : c0.c.rt);
        q8_gemm_round g{};
        long wgs = 0;
        for (int p = p0; p < n; p++) {
            if (!same(p))
                continue;
            launched[p] = true;
            const int k = g.n++;
            g.w[k] = all.w[p];
            g.rows[k] = all.rows[p];
            g.ks[k] = all.ks[p];
            g.cps[k] = all.cps[p];
            g.out[k] = all.out[p];
            g.y[k] = all.y[p];
            g.start[k] = wgs;
            wgs += (rows[p] + rowsper - 1) / rowsper * all.ks[p];
        }
        g.start[g.n] = wgs;
        bool ok = false;
        if (c0.xres) {
            if (nw == 12)
                Q8_LAUNCH(q8_time_name("gemm_xres_round", 3, XRES_KP, 12, XRES_SC), (gemm_xres_round<XRES_KP, 12, XRES_SC>), dim3((unsigned)wgs),
                          dim3(64 * 12), s, g, cols, x, x_stride, t);
            else
                Q8_LAUNCH(q8_time_name("gemm_xres_round", 3, XRES_KP, 16, XRES_SC), (gemm_xres_round<XRES_KP, 16, XRES_SC>), dim3((unsigned)wgs),
                          dim3(64 * 16), s, g, cols, x, x_stride, t);
            ok = true;
        } else {
            const unsigned groups = (unsigned)(((t + 15) / 16 + c0.c.mg - 1) / c0.c.mg);
#define GR(G, R, P, N)                                                                                                 \
    if (!ok && c0.c.mg == G && c0.c.rt == R && c0.c.kp == P && nw == N) {                                              \
        Q8_LAUNCH(q8_time_name("gemm_mfma_round", 4, G, R, P, N), (gemm_mfma_round<G, R, P, N>), dim3((unsigned)wgs, groups), dim3(64 * N), s, g,    \
                  cols, x, x_stride, t);                                                                               \
        ok = true;                                                                                                     \
    }
            GEMM_CFGS(GR)
#undef GR
        }
        if (!ok) {
            fprintf(stderr, "q8_gemm: no round kernel for MG %d RT %d KP %d NW %d\n", c0.c.mg, c0.c.rt, c0.c.kp, nw);
            abort();
        }
    }
    if (pair_y)
        gemm_swiglu_round<<<dim3((unsigned)((all.ostart[1] + 255) / 256)), dim3(256), 0, s>>>(all, (t + 15) / 16 * 16, pair_y);
    else if (parts > 0)
        gemm_sum_round<<<dim3((unsigned)((all.ostart[n] + 255) / 256)), dim3(256), 0, s>>>(all, (t + 15) / 16 * 16);
    return 0;
}

int q8_launch_read_gemm(q8_stream_t stream, const void *w, long rows, long cols, const float *x, long x_stride, long t, unsigned *sink,
                        q8_gemm_opts o)
{
    if (t < 5 || t > 16)
        return -1;
    const gemm_plan p = plan_of(rows, cols, t, o);
    if (!p.xres)
        return -1;
    hipStream_t s = (hipStream_t)stream;
    const long tiles = (rows + 16L * p.c.nw - 1) / (16L * p.c.nw);
    if (p.c.nw == 12)
        Q8_LAUNCH(q8_time_name("read_xres", 3, XRES_KP, 12, XRES_SC), (read_xres<XRES_KP, 12, XRES_SC>), dim3((unsigned)(tiles * p.ks)), dim3(64 * 12), s,
                  (const uint8_t *)w, rows, cols, x, x_stride, t, p.ks, p.cps, sink);
    else
        Q8_LAUNCH(q8_time_name("read_xres", 3, XRES_KP, 16, XRES_SC), (read_xres<XRES_KP, 16, XRES_SC>), dim3((unsigned)(tiles * p.ks)), dim3(64 * 16), s,
                  (const uint8_t *)w, rows, cols, x, x_stride, t, p.ks, p.cps, sink);
    return 0;
}

template <int MG, int RT, int KP, int NW>
static void gemm_go(hipStream_t s, const void *w, long rows, long cols, const float *x, long xst, long t, float *y, float *part, int ks, int cps,
                    const float *res)
{
    const long tiles = (rows + 16L * NW * RT - 1) / (16L * NW * RT);
    const long groups = ((t + 15) / 16 + MG - 1) / MG;
    Q8_LAUNCH(q8_time_name("gemm_mfma", 4, MG, RT, KP, NW), (gemm_mfma<MG, RT, KP, NW>), dim3((unsigned)(tiles * ks), (unsigned)groups),
              dim3(64 * NW), s, (const uint8_t *)w, rows, cols, x, xst, t, ks, cps, part, y, res);
}

void q8_launch_gemm_mfma(q8_stream_t stream, const void *w, long rows, long cols, const float *x, long x_stride, long t, float *y, float *part,
                         const float *res, q8_gemm_opts o)
{
    hipStream_t s = (hipStream_t)stream;
    const gemm_plan p = plan_of(rows, cols, t, o);
    const int ks = p.ks, cps = p.cps;
    float *out = ks > 1 ? part : y;
    const float *r1 = ks > 1 ? nullptr : res;
    bool done = false;
    if (p.xres) {
        const long tiles = (rows + 16L * p.c.nw - 1) / (16L * p.c.nw);
        if (p.c.nw == 12)
            Q8_LAUNCH(q8_time_name("gemm_xres", 3, XRES_KP, 12, XRES_SC), (gemm_xres<XRES_KP, 12, XRES_SC>), dim3((unsigned)(tiles * ks)), dim3(64 * 12), s,
                      (const uint8_t *)w, rows, cols, x, x_stride, t, ks, cps, out, out, r1);
        else
            Q8_LAUNCH(q8_time_name("gemm_xres", 3, XRES_KP, 16, XRES_SC), (gemm_xres<XRES_KP, 16, XRES_SC>), dim3((unsigned)(tiles * ks)), dim3(64 * 16), s,
                      (const uint8_t *)w, rows, cols, x, x_stride, t, ks, cps, out, out, r1);
        done = true;
    }
#define GO(G, R, P, N)                                                                                                 \
    if (!done && p.c.mg == G && p.c.rt == R && p.c.kp == P && p.c.nw == N) {                                           \
        gemm_go<G, R, P, N>(s, w, rows, cols, x, x_stride, t, out, part, ks, cps, r1);                                 \
        done = true;                                                                                                   \
    }
    GEMM_CFGS(GO)
#undef GO
    if (!done) {
        fprintf(stderr, "q8_gemm: no kernel for MG %d RT %d KP %d NW %d\n", p.c.mg, p.c.rt, p.c.kp, p.c.nw);
        abort();
    }
    if (ks > 1)
        gemm_sum<<<dim3((unsigned)((t * rows + 255) / 256)), 256, 0, s>>>(part, ks, t, (t + 15) / 16 * 16, rows, y, res);
}
