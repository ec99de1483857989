/* The other half of the reference-header check (ref_abi_ref.c): the same entry points through
 * include/q8_rt.h, and struct rt's layout as this library declares it. main() compares the two
 * layouts and calls rt_init through the reference's declaration (0 with a GPU, -1 without). */
#include <stddef.h>
#include <stdio.h>

#include "q8_rt.h"

void *const own_side[] = {(void *)rt_init, (void *)rt_gemv, (void *)rt_gemv_q, (void *)rt_gemv_open,
                          (void *)rt_gemv_go, (void *)rt_gemm, (void *)rt_gemm_q, (void *)rt_q8_row};

void own_calls(struct rt *R, const void *w, const float *x, float *y)
{
    rt_gemv(R, w, 16, 32, x, y);
    rt_gemv_q(R, w, 16, 32, x, y);
    rt_gemv_open(R);
    rt_gemv_go(R);
    rt_gemm(R, w, 16, 32, x, 2, y);
    rt_gemm_q(R, w, 16, 32, x, 2, y);
    rt_q8_row(w, 32, 0, y);
}

static const long own_layout[] = {sizeof(struct rt), offsetof(struct rt, team), offsetof(struct rt, frame), offsetof(struct rt, chain),
                                  offsetof(struct rt, gemm_chain), offsetof(struct rt, threads), offsetof(struct rt, last), RT_BATCH};
extern const long ref_layout[];
extern void *const ref_side[];
int ref_init(struct rt *R, int threads);

int main(void)
{
    for (int i = 0; i < (int)(sizeof(own_layout) / sizeof(own_layout[0])); i++)
        if (own_layout[i] != ref_layout[i]) {
            printf("layout item %d: reference %ld, here %ld\n", i, ref_layout[i], own_layout[i]);
            return 1;
        }
    for (int i = 0; i < 8; i++)
        if (own_side[i] != ref_side[i]) {
            printf("entry point %d resolves differently\n", i);
            return 1;
        }
    struct rt R = {0};
    const int rc = ref_init(&R, 1);
    printf("layout identical; rt_init through the reference's declaration: %d\n", rc);
    if (rc == 0)
        rt_fini(&R);
    return rc == 0 || rc == -1 ? 0 : 1;
}
