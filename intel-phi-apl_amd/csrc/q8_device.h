/* q8_device.h: what every kernel of the library shares: the form S addressing, the exact
 * conversions, the reductions, and the launchers' declarations (host side).
 *
 * Form S (include/q8_rt.h), per 16-row group g at g*17*cols bytes:
 *   16*cols int8 q, row by row (row 16g+r at r*cols);
 *   then cols bytes of binary16 d, row by row (row 16g+r at 16*cols + r*cols/16).
 * Like the reference's form I (src/card/gemv.c:23-40) it is 17/16 bytes per weight and a
 * 16-row group holds everything of its rows, so a prefix of groups is a smaller matrix. Unlike
 * form I, a row's 32 weights of a block lie in column order, contiguous: a lane's 16-byte load
 * is 16 columns of one row, and 64 lanes read 1 KiB of one row at once. */
#ifndef Q8_DEVICE_H
#define Q8_DEVICE_H

#include <stddef.h>
#include <stdint.h>

#define Q8_GROUP 16
#define Q8_BLOCK 32
#define Q8_BLOCK_BYTES 34

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>

/* bytes from the handle to the start of row r's int8 weights / binary16 scales */
__device__ __forceinline__ size_t q8s_row_q(long r, long cols)
{
    return (size_t)(r >> 4) * 17u * (size_t)cols + (size_t)(r & 15) * (size_t)cols;
}
__device__ __forceinline__ size_t q8s_row_d(long r, long cols)
{
    return (size_t)(r >> 4) * 17u * (size_t)cols + 16u * (size_t)cols + (size_t)(r & 15) * (size_t)(cols / 16);
}

/* byte k of w as a signed integer, to binary32: exact (|q| <= 128). One v_cvt_f32_i32 with an
 * SDWA sign-extended byte select on gfx950. */
__device__ __forceinline__ float q8_s8(uint32_t w, int k)
{
    return (float)(int8_t)(uint8_t)(w >> (8 * k));
}

/* binary16 to binary32: v_cvt_f32_f16, exact for every pattern (subnormals kept: the f16
 * denormal mode is on for HIP kernels). */
__device__ __forceinline__ float q8_half(uint16_t h)
{
    return (float)__builtin_bit_cast(_Float16, h);
}

/* sum over the 64 lanes, the same pairing on every call: the result in every lane */
__device__ __forceinline__ float q8_wave_sum(float v)
{
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1)
        v += __shfl_xor(v, off, 64);
    return v;
}

#define Q8_DPP(v, ctrl) __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, (v)), (ctrl), 0xf, 0xf, false))

/* sum over the 64 lanes by DPP within each row of 16 lanes (pairs i^1, i^2, then the half-row
 * and row mirrors), then the four rows' sums read from lanes 15, 31, 47, 63 and added as
 * (r0 + r1) + (r2 + r3): the same order on every call; the result is wave-uniform */
__device__ __forceinline__ float q8_wave_sum_dpp(float v)
{
    v += Q8_DPP(v, 0xb1);  /* quad_perm [1,0,3,2] */
    v += Q8_DPP(v, 0x4e);  /* quad_perm [2,3,0,1] */
    v += Q8_DPP(v, 0x141); /* row_half_mirror */
    v += Q8_DPP(v, 0x140); /* row_mirror */
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 15));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 31));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 47));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
    return (r0 + r1) + (r2 + r3);
}

/* the least power of two >= n (n >= 1) */
__host__ __device__ constexpr int q8_pow2ceil(int n)
{
    return n <= 1 ? 1 : 2 * q8_pow2ceil((n + 1) / 2);
}

/* The sums over the 64 lanes of V values a lane (V a power of two), by a butterfly over the lane
 * bits 5, 4, 3 and then 0, 1, 2: the same lane pairs in the same order for every V, so a value's
 * sum has the same bits whatever V is. While two or more values are left, a step over bit 5, 4 or
 * 3 is transposed: lanes with the bit clear keep the first half of the values and the others the
 * second half, each adding its partner's copy of the values it keeps, so a step costs one add a
 * kept value instead of one a value. A single value is summed in place. Bit 5 pairs lanes with
 * v_permlane32_swap (the upper 32 lanes of its first operand trade places with the lower 32 of
 * its second), bit 4 with v_permlane16_swap (the odd rows of 16 lanes of the first with the even
 * rows of the second), bit 3 with DPP row_ror:8; bits 0, 1, 2 within each group of 8 lanes with
 * DPP quad_perm [1,0,3,2], [2,3,0,1] and row_half_mirror (exact pairs once each quad holds equal
 * values). On return, with T = min(3, log2 V) transposed steps, v[k] (k < V >> T) of lane l is the
 * sum of value q8_wave_sums_index<V>(l, k); lanes with q8_wave_sums_owner<V>(l) hold each value
 * once. The two results of a swap pass through q8_swap_sum, which hides the second from the
 * optimiser: summed directly, this compiler folds their sum into twice the first result (checked
 * in its gfx950 assembly: v_permlane32_swap_b32 v1, v2 then v_add_f32 v1, v1, v1). */
__device__ __forceinline__ float q8_swap_sum(uint32_t a, uint32_t b)
{
    asm volatile("" : "+v"(b));
    return __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
}
template <int V>
__device__ __forceinline__ constexpr int q8_wave_sums_steps()
{
    return V >= 8 ? 3 : V >= 4 ? 2 : V >= 2 ? 1 : 0;
}
template <int V>
__device__ __forceinline__ int q8_wave_sums_index(int l, int k)
{
    constexpr int T = q8_wave_sums_steps<V>();
    return (T > 0 && (l & 32) ? V / 2 : 0) + (T > 1 && (l & 16) ? V / 4 : 0) + (T > 2 && (l & 8) ? V / 8 : 0) + k;
}
template <int V>
__device__ __forceinline__ bool q8_wave_sums_owner(int l)
{
    constexpr int T = q8_wave_sums_steps<V>();
    return (l & 7) == 0 && (T > 2 || !(l & 8)) && (T > 1 || !(l & 16)) && (T > 0 || !(l & 32));
}
template <int V>
__device__ __forceinline__ void q8_wave_sums(float (&v)[V], int lane)
{
    static_assert((V & (V - 1)) == 0, "a power of two");
    /* bit 5 */
    if constexpr (V >= 2) {
#pragma unroll
        for (int i = 0; i < V / 2; i++) {
            const auto s = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, v[i]), __builtin_bit_cast(uint32_t, v[i + V / 2]), false, false);
            v[i] = q8_swap_sum(s[0], s[1]);
        }
    } else {
        const auto s = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, v[0]), __builtin_bit_cast(uint32_t, v[0]), false, false);
        v[0] = q8_swap_sum(s[0], s[1]);
    }
    constexpr int N4 = V >= 2 ? V / 2 : 1; /* values left */
    /* bit 4 */
    if constexpr (N4 >= 2) {
#pragma unroll
        for (int i = 0; i < N4 / 2; i++) {
            const auto s = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, v[i]), __builtin_bit_cast(uint32_t, v[i + N4 / 2]), false, false);
            v[i] = q8_swap_sum(s[0], s[1]);
        }
    } else {
        const auto s = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, v[0]), __builtin_bit_cast(uint32_t, v[0]), false, false);
        v[0] = q8_swap_sum(s[0], s[1]);
    }
    constexpr int N3 = N4 >= 2 ? N4 / 2 : 1;
    /* bit 3 */
    if constexpr (N3 >= 2) {
        const bool hi = (lane & 8) != 0;
#pragma unroll
        for (int i = 0; i < N3 / 2; i++) {
            const float keep = hi ? v[i + N3 / 2] : v[i], give = hi ? v[i] : v[i + N3 / 2];
            v[i] = keep + Q8_DPP(give, 0x128); /* row_ror:8 */
        }
    } else {
        v[0] += Q8_DPP(v[0], 0x128);
    }
    constexpr int N = N3 >= 2 ? N3 / 2 : 1;
    /* bits 0, 1, 2 */
#pragma unroll
    for (int k = 0; k < N; k++) {
        v[k] += Q8_DPP(v[k], 0xb1);  /* quad_perm [1,0,3,2] */
        v[k] += Q8_DPP(v[k], 0x4e);  /* quad_perm [2,3,0,1] */
        v[k] += Q8_DPP(v[k], 0x141); /* row_half_mirror */
    }
}

/* SiLU(g) * u (src/apl/qwen35.apl:38; docs/model.md:29: Sig = 1 / (1 + exp(min(700, -g)))):
 * in binary32 exp(min(700, -g)) overflows to inf for -g > 88.7 exactly as exp(-g) does, so
 * the clamp changes nothing and is left out. */
__device__ __forceinline__ float q8_swiglu(float g, float u)
{
    return g / (1.0f + __expf(-g)) * u;
}
#endif

/* ---- launchers (q8_kernels.hip), all asynchronous on `stream` */
#ifdef __cplusplus
struct ihipStream_t;
typedef struct ihipStream_t *q8_stream_t;

/* Kernel timing: when set, the next product kernel launched takes these two events as its own
 * start and end (hipExtLaunchKernelGGL) and writes its name, as rocprof prints it (for example
 * "gemv_k<1, 4, 1, 1>"), into name[64] and its grid in threads into *grid; then the slot
 * clears. Host side, one thread. */
void q8_time_next(void *start_event, void *stop_event, char *name, long *grid);
/* "base<a, b, ...>" for the n integers that follow, into the timing slot's name */
void q8_time_name(const char *base, int n, ...);

#if defined(__HIPCC__)
#include <hip/hip_ext.h>
extern void *q8_next_start, *q8_next_stop;
extern long *q8_next_grid;
/* kernel<<<grid, block, 0, stream>>>(args...), or the timed launch when a slot is set; NAME is
 * evaluated only then (a call of q8_time_name) */
#define Q8_LAUNCH(NAME, kernel, grid, block, stream, ...)                                                              \
    do {                                                                                                               \
        if (q8_next_start) {                                                                                           \
            NAME;                                                                                                      \
            *q8_next_grid = (long)(grid).x * (grid).y * (grid).z * (block).x * (block).y * (block).z;                 \
            hipExtLaunchKernelGGL(kernel, grid, block, 0, stream, (hipEvent_t)q8_next_start, (hipEvent_t)q8_next_stop, 0, \
                                  __VA_ARGS__);                                                                        \
            q8_next_start = q8_next_stop = nullptr;                                                                    \
        } else {                                                                                                       \
            kernel<<<grid, block, 0, stream>>>(__VA_ARGS__);                                                           \
        }                                                                                                              \
    } while (0)
#endif

/* Y = X W^T, t tokens, the fast kernels; W form S. w1 != NULL: the fused pair, Y = SiLU(X W0^T) * (X W1^T). */
void q8_launch_gemv(q8_stream_t stream, const void *w0, const void *w1, long rows, long cols, const float *x, long x_stride, long t, float *y);
/* An epilogue on either side of a product (src/apl/qwen35.apl:49, 131-139). nw != NULL: the RMS
 * norm first, per token xn[k] = nw[k] * (x[k] * s) with s = 1 / sqrt(eps + sum_k x[k]^2 / cols);
 * res != NULL: Y = res + the product, res laid out as Y (it may be Y: the residual stream updated
 * in place). One of the two at a time. */
struct q8_epi {
    const float *nw;
    float eps;
    const float *res;
};
/* The decode product with the epilogue fused into its kernel (t <= 4): 0, or -1 when no fused
 * kernel takes the shape (nothing launched; the caller runs the epilogue apart). */
int q8_launch_gemv_epi(q8_stream_t stream, const void *w0, const void *w1, long rows, long cols, const float *x, long x_stride, long t, float *y,
                       q8_epi e);
/* The RMS norm apart: xn [t cols] (rows cols floats apart) from x [t cols] (x_stride apart). */
void q8_launch_rmsnorm(q8_stream_t stream, const float *x, long x_stride, long t, long cols, const float *nw, float eps, float *xn);
/* y[i] = a[i] + b[i], i < n (y may be a or b). */
void q8_launch_add(q8_stream_t stream, const float *a, const float *b, long n, float *y);
/* A round of products sharing x as one launch (t <= 4, cols % 1024 == 0, every rows % 8 == 0):
 * 0, or -1 (nothing launched: the caller runs them one by one). */
#define Q8_ROUND_MAX 8
struct q8_round {
    int n;
    const void *w[Q8_ROUND_MAX];
    float *y[Q8_ROUND_MAX];
    long rows[Q8_ROUND_MAX];
    long start[Q8_ROUND_MAX + 1]; /* first workgroup of each product; start[n] = the grid */
};
int q8_launch_gemv_round(q8_stream_t stream, int n, const void *const *w, const long *rows, long cols, const float *x, long x_stride, long t, float *const *y);
/* The same with the RMS norm of x fused (e.nw != NULL, e.res NULL): 0, or -1 (nothing launched). */
int q8_launch_gemv_round_epi(q8_stream_t stream, int n, const void *const *w, const long *rows, long cols, const float *x, long x_stride, long t,
                             float *const *y, q8_epi e);
/* The reference's order, every y bit-identical to the reference's F32 host path. */
void q8_launch_exact(q8_stream_t stream, const void *w, long rows, long cols, const float *x, long x_stride, long t, float *y);
/* Y = X W^T for 1 <= t <= 64 on the matrix cores (and the sum of the K split's partials); the
 * runtime sends every product of t >= 5 tokens here, 64 tokens a launch. part holds
 * q8_gemm_part_floats(rows, cols, t, o) floats, at most Q8_GEMM_PART_MAX. The K split is a
 * function of (rows, cols) alone, so a token's output does not depend on t. o: test hooks, zero
 * for the planner's choices (ks > 0: that many K splits; streaming: one token tile on the
 * streaming kernel instead of the x-resident one, the same sums). */
#define Q8_GEMM_PART_MAX (8L << 20)
struct q8_gemm_opts {
    int ks;
    int streaming;
};
void q8_launch_gemm_mfma(q8_stream_t stream, const void *w, long rows, long cols, const float *x, long x_stride, long t, float *y, float *part,
                         const float *res, q8_gemm_opts o);
long q8_gemm_part_floats(long rows, long cols, long t, q8_gemm_opts o);
/* A round of products sharing x at 1 <= t <= 64 tokens (one 64-token chunk of a longer X, so the
 * last chunk of one with 65 to 68 tokens holds fewer than 5; rounds of fewer than 5 tokens in all
 * run on the decode kernel): one matrix-core launch for the products (the x-resident kernel at
 * t <= 16, the streaming one above, at the largest product's wave count; two products of one shape
 * as a pair kernel where one is built for the configuration) and one launch of every
 * product's partial sums, each product on its own K split (its single launch's bits, as
 * q8_launch_gemm_mfma's at any t): 0, or -1 (nothing launched: the partials need more than part_cap floats
 * of part, q8_gemm_round_part_floats; the caller runs them one by one). pair_y != NULL: the fused
 * pair, n == 2 (gate, up; one shape): pair_y = SiLU(G) * U from the two products' sums in one
 * launch, y[] then only receiving what a product of one split writes itself. */
struct q8_gemm_round {
    int n;
    const void *w[Q8_ROUND_MAX];
    float *out[Q8_ROUND_MAX]; /* the product's partials (ks > 1) or its Y */
    float *y[Q8_ROUND_MAX];
    long rows[Q8_ROUND_MAX];
    int ks[Q8_ROUND_MAX], cps[Q8_ROUND_MAX];
    long start[Q8_ROUND_MAX + 1];  /* first workgroup of each product; start[n] = the grid */
    long ostart[Q8_ROUND_MAX + 1]; /* first output (t x rows a product); ostart[n] = the outputs */
};
int q8_launch_gemm_round(q8_stream_t stream, int n, const void *const *w, const long *rows, long cols, const float *x, long x_stride, long t,
                         float *const *y, float *part, long part_cap, q8_gemm_opts o, float *pair_y = nullptr);
long q8_gemm_round_part_floats(int n, const long *rows, long cols, long t, q8_gemm_opts o);
/* The floor of the x-resident product at 5 <= t <= 16 tokens: its loads on its grid (the plan for
 * these options), no arithmetic, a checksum added to sink[0]; -1 when the plan is not the
 * x-resident kernel. */
int q8_launch_read_gemm(q8_stream_t stream, const void *w, long rows, long cols, const float *x, long x_stride, long t, unsigned *sink,
                        q8_gemm_opts o);
/* y[i] = SiLU(g[i]) * u[i] (the exact fused pair's epilogue). */
void q8_launch_swiglu_ew(q8_stream_t stream, const float *g, const float *u, long n, float *y);
/* z[i] = row rows[i] of w dequantised (q * d, exact), i < n; rows and z device arrays; an index
 * outside [0, nrows) gives a row of NaN. */
void q8_launch_rows(q8_stream_t stream, const void *w, long cols, long nrows, const long *rows, long n, float *z);
/* *out = the lowest i with a[i] bit-equal to the fmaxf fold of a[0..n); cm, ci hold
 * q8_argmax_chunks(n) candidates. */
long q8_argmax_chunks(long n);
void q8_launch_argmax(q8_stream_t stream, const float *a, long n, float *cm, long *ci, long *out);
/* GGUF Q8_0 rows to form S, both device. */
void q8_launch_repack(q8_stream_t stream, const void *q8, long rows, long cols, void *out);
/* Synthetic GGUF rows and F32 values on the device. */
void q8_launch_fill(q8_stream_t stream, void *dst, long rows, long cols, uint64_t seed, int dist, float mu, float sigma);
void q8_launch_fill_f32(q8_stream_t stream, float *dst, long n, uint64_t seed);
/* The decode product's loads at t tokens (x rows x_stride apart), nothing computed: the floor of a
 * product of that shape (w1: the fused pair's two matrices). sink[b] (device, rows entries)
 * receives workgroup b's checksum of the words it read (added, wrapping). 0, or -1 when the shape
 * has no such kernel (nothing launched). */
int q8_launch_read(q8_stream_t stream, const void *w0, const void *w1, long rows, long cols, const float *x, long x_stride, long t, unsigned *sink);
/* dst = src, n16 16-byte words, both device. */
void q8_launch_copy(q8_stream_t stream, void *dst, const void *src, long n16);
/* *flag = seq once the kernels before it on the stream are done; flag in pinned host memory. */
void q8_launch_flag(q8_stream_t stream, unsigned *flag, unsigned seq);
/* The primitive conversions of the product kernels, lane by lane (the reference's gate 2.1
 * s8 and f16 sets, src/gate/upconv_kernel.c:18-57). */
void q8_launch_prims(q8_stream_t stream, const int8_t *q, const float *x8, const float *c8, float *o8, long n8, const uint16_t *h,
                     const float *xf, const float *cf, float *of, long nf);
#endif

#endif
