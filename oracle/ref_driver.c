/* ref_driver.c: TEST INFRASTRUCTURE ONLY. Calls the reference's own Q8_0 product code,
 * compiled unchanged from its sources (src/card/gemv.c, gemm.c, team.c with the host model
 * of knc.h), so the oracle and the GPU can be held to it bit for bit. Built by
 * oracle/Makefile into oracle/_ref/, which is never committed.
 *
 *   ref_repack_i    gemv_i_repack (gemv.c:23-40): GGUF rows to form I
 *   ref_gemv        gemv_i_thread at one thread, no chain (gemv.c:165-181): whole groups
 *   ref_gemm        gemm_i_thread at one thread, no chain (gemm.c:271-294)
 *   ref_team_*      the same on the reference's pinned team (team.c:90-129), its threads on
 *                   the first n CPUs this process may use; for the CPU baseline */
#define _GNU_SOURCE
#include <sched.h>
#include <stdint.h>
#include <stdlib.h>

#include "gemm.h"
#include "gemv.h"
#include "team.h"

void ref_repack_i(const uint8_t *q8, long rows, long cols, void *out) { gemv_i_repack(q8, rows, cols, out); }

void ref_gemv_i(const void *form_i, long rows, long cols, const float *x, float *y)
{
    struct gemv_job j = {.w = form_i, .rows = rows, .cols = cols, .x = x, .y = y};
    gemv_i_thread(&j, 0, 1);
}

void ref_gemm_i(const void *form_i, long rows, long cols, const float *x, long t, float *y)
{
    struct gemm_job j = {.w = form_i, .rows = rows, .cols = cols, .t = t, .x = x, .x_stride = cols, .y = y};
    gemm_i_thread(&j, 0, 1);
}

void ref_gemv(const uint8_t *q8, long rows, long cols, const float *x, float *y)
{
    void *w = malloc((size_t)gemv_i_bytes(rows, cols));
    if (!w)
        abort();
    gemv_i_repack(q8, rows, cols, w);
    ref_gemv_i(w, rows, cols, x, y);
    free(w);
}

void ref_gemm(const uint8_t *q8, long rows, long cols, const float *x, long t, float *y)
{
    void *w = malloc((size_t)gemv_i_bytes(rows, cols));
    if (!w)
        abort();
    gemv_i_repack(q8, rows, cols, w);
    ref_gemm_i(w, rows, cols, x, t, y);
    free(w);
}

/* The CPUs this thread may use before the first team: the team pins its calling thread to its
 * first CPU, so later teams read the set from here, and ref_team_destroy gives the thread the
 * whole set back (a second team, in the same process, sees the same CPUs as the first). */
static cpu_set_t first_allowed;
static int have_allowed;

void *ref_team_create(int n)
{
    cpu_set_t allowed;
    int *cpus = malloc(sizeof(int) * (size_t)n), k = 0;
    if (!cpus)
        abort();
    if (!have_allowed) {
        CPU_ZERO(&first_allowed);
        sched_getaffinity(0, sizeof first_allowed, &first_allowed);
        have_allowed = 1;
    }
    allowed = first_allowed;
    for (int c = 0; c < CPU_SETSIZE && k < n; c++)
        if (CPU_ISSET((size_t)c, &allowed))
            cpus[k++] = c;
    if (k < n) {
        free(cpus);
        return NULL;
    }
    struct team *t = team_create(cpus, n, 1);
    free(cpus);
    return t;
}

void ref_team_destroy(void *t)
{
    team_destroy(t);
    if (have_allowed)
        sched_setaffinity(0, sizeof first_allowed, &first_allowed);
}

void ref_team_gemv_i(void *team, const void *form_i, long rows, long cols, const float *x, float *y)
{
    struct gemv_job j = {.w = form_i, .rows = rows, .cols = cols, .x = x, .y = y};
    team_run(team, gemv_i_thread, &j);
}

void ref_team_gemm_i(void *team, const void *form_i, long rows, long cols, const float *x, long t, float *y)
{
    struct gemm_job j = {.w = form_i, .rows = rows, .cols = cols, .t = t, .x = x, .x_stride = cols, .y = y};
    team_run(team, gemm_i_thread, &j);
}
