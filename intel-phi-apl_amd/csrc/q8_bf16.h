/* q8_bf16.h: the pieces of the bf16 matrix-core product (q8_gemm.hip): exact int8 and
 * three-limb F32 operands for v_mfma_f32_16x16x32_bf16, and their column order inside a block. */
#ifndef Q8_BF16_H
#define Q8_BF16_H

#include <hip/hip_runtime.h>

#include <stdint.h>

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

/* 8 F32 values to their three bf16 limbs (8 each): hi = the top 16 bits, r = x - hi exactly,
 * mid = r's top 16 bits, lo = r - mid exactly (at most 8 significant bits). An infinite x is hi
 * alone (x - hi would be NaN), so it reaches the sums as the infinity the F32 product sees; a NaN
 * stays NaN in every limb's path. The infinity test runs only when the largest |x| of the 8 is
 * infinite (a few instructions for 8 values; the per-value test cost the streaming GEMM 2 us at
 * M = 40 and 64). */
__device__ __forceinline__ void xsplit8(float4 a, float4 c, uint4 &h, uint4 &m, uint4 &o)
{
    const float v[8] = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
    float hi[8], mid[8], lo[8];
#pragma unroll
    for (int e = 0; e < 8; e++) {
        hi[e] = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, v[e]) & 0xffff0000u);
        const float r = v[e] - hi[e];
        mid[e] = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, r) & 0xffff0000u);
        lo[e] = r - mid[e];
    }
    const float big = fmaxf(fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))),
                            fmaxf(fmaxf(fabsf(v[4]), fabsf(v[5])), fmaxf(fabsf(v[6]), fabsf(v[7]))));
    if (__builtin_expect(big == __builtin_inff(), 0)) {
#pragma unroll
        for (int e = 0; e < 8; e++)
            if (__builtin_isinf(v[e]))
                mid[e] = lo[e] = 0.0f;
    }
    h = make_uint4(pack_hi(hi[0], hi[1]), pack_hi(hi[2], hi[3]), pack_hi(hi[4], hi[5]), pack_hi(hi[6], hi[7]));
    m = make_uint4(pack_hi(mid[0], mid[1]), pack_hi(mid[2], mid[3]), pack_hi(mid[4], mid[5]), pack_hi(mid[6], mid[7]));
    o = make_uint4(pack_hi(lo[0], lo[1]), pack_hi(lo[2], lo[3]), pack_hi(lo[4], lo[5]), pack_hi(lo[6], lo[7]));
}

/* 8 int8 (two dwords) to 8 bf16 */
__device__ __forceinline__ bf16x8 q8_bf16(uint32_t a, uint32_t b)
{
    return __builtin_bit_cast(bf16x8, make_uint4(pack_hi((float)(int8_t)a, (float)(int8_t)(a >> 8)), pack_hi((float)(int8_t)(a >> 16), (float)(int8_t)(a >> 24)),
                                                 pack_hi((float)(int8_t)b, (float)(int8_t)(b >> 8)), pack_hi((float)(int8_t)(b >> 16), (float)(int8_t)(b >> 24))));
}

#endif
