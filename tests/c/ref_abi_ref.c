/* Compiled against the reference's own src/card/rt.h (found with -I at test time, never copied):
 * the product entry points as the reference's generated code declares them, and struct rt's layout
 * as it sees it. Linked by tests/test_abi.py with ref_abi_own.c under -flto -Werror=lto-type-mismatch,
 * so a declaration in include/q8_rt.h that differs from the reference's in any parameter or return
 * type fails the link. */
#include <stddef.h>

#include "rt.h"

void *const ref_side[] = {(void *)rt_init, (void *)rt_gemv, (void *)rt_gemv_q, (void *)rt_gemv_open,
                          (void *)rt_gemv_go, (void *)rt_gemm, (void *)rt_gemm_q, (void *)rt_q8_row};

/* every product entry point called with the reference's argument types */
void ref_calls(struct rt *R, const void *w, const float *x, float *y)
{
    rt_gemv(R, w, 16, 32, x, y);
    rt_gemv_q(R, w, 16, 32, x, y);
    rt_gemv_open(R);
    rt_gemv_go(R);
    rt_gemm(R, w, 16, 32, x, 2, y);
    rt_gemm_q(R, w, 16, 32, x, 2, y);
    rt_q8_row(w, 32, 0, y);
}

int ref_init(struct rt *R, int threads) { return rt_init(R, threads); }

const long ref_layout[] = {sizeof(struct rt), offsetof(struct rt, team), offsetof(struct rt, frame), offsetof(struct rt, chain),
                           offsetof(struct rt, gemm_chain), offsetof(struct rt, threads), offsetof(struct rt, last), RT_BATCH};
