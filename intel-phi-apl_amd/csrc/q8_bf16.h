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
 * stays NaN in every limb's path. */
__device__ __forceinline__ void xsplit8(float4 a, float4 c, uint4 &h, uint4 &m, uint4 &o)
{
    const float v[8] = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
    uint32_t hh[4], mm[4], oo[4];
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
        float hi[2], mid[2], lo[2];
#pragma unroll
        for (int e = 0; e < 2; e++) {
            hi[e] = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, v[j + e]) & 0xffff0000u);
            const float r = __builtin_isinf(v[j + e]) ? 0.0f : v[j + e] - hi[e];
            mid[e] = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, r) & 0xffff0000u);
            lo[e] = r - mid[e];
        }
        hh[j / 2] = pack_hi(hi[0], hi[1]);
        mm[j / 2] = pack_hi(mid[0], mid[1]);
        oo[j / 2] = pack_hi(lo[0], lo[1]);
    }
    h = make_uint4(hh[0], hh[1], hh[2], hh[3]);
    m = make_uint4(mm[0], mm[1], mm[2], mm[3]);
    o = make_uint4(oo[0], oo[1], oo[2], oo[3]);
}

/* 8 int8 (two dwords) to 8 bf16 */
__device__ __forceinline__ bf16x8 q8_bf16(uint32_t a, uint32_t b)
{
    return __builtin_bit_cast(bf16x8, make_uint4(pack_hi((float)(int8_t)a, (float)(int8_t)(a >> 8)), pack_hi((float)(int8_t)(a >> 16), (float)(int8_t)(a >> 24)),
                                                 pack_hi((float)(int8_t)b, (float)(int8_t)(b >> 8)), pack_hi((float)(int8_t)(b >> 16), (float)(int8_t)(b >> 24))));
}

#endif
