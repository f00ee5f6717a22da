/* cpu_gemm.c -- the host GEMMs: ork_i8_mm_run_cpu, the public CPU int8 GEMM (reference include/ork/run.h:132,
 * src/npu/core/buf.c:578-580 forwarding to orki_cpu_gemm_i32, :428-477), and the offline context's runs.
 *
 * ork_i8_mm_run_cpu is an explicitly-CPU API the reference exports so a caller can time the CPU side of a
 * routing decision. An OFFLINE context (ork_npu_init_offline: no device) runs its weights here, as the
 * reference's offline branches do (src/npu/i8/run.c:140, src/npu/i4/run.c:236, the CPU chains
 * src/npu/core/buf.c:483-487 / :560-564, the grouped accumulate :501-520): an offline weight keeps its int8
 * codes [K][N] on the host. A device context never comes here: its runs launch the HIP kernels or fail.
 * Exact int32: the k-outer AXPY keeps the C row hot while B streams, skips zero activations, and
 * parallelises over M rows on the host pool. */
#include <stdlib.h>
#include <string.h>

#include "internal.h"

struct cpu_gemm { int K, N; const int8_t *A, *B; int32_t *C; };

static void rows(int lo, int hi, void *arg) {
    const struct cpu_gemm *g = arg;
    for (int m = lo; m < hi; m++) {
        const int8_t *a = g->A + (size_t)m * g->K;
        int32_t *c = g->C + (size_t)m * g->N;
        memset(c, 0, (size_t)g->N * sizeof *c);
        for (int k = 0; k < g->K; k++) {
            const int32_t av = a[k];
            if (!av) continue;
            const int8_t *b = g->B + (size_t)k * g->N;
            for (int n = 0; n < g->N; n++) c[n] += av * (int32_t)b[n];
        }
    }
}

void ork_i8_mm_run_cpu(int M, int K, int N, const int8_t *A, const int8_t *B, int32_t *C) {
    if (M <= 0 || K <= 0 || N <= 0 || !A || !B || !C) return;
    struct cpu_gemm g = {K, N, A, B, C};
    if (M == 1) rows(0, 1, &g);
    else orki_parallel_for(M, rows, &g);
}

/* Per-K-group accumulate (src/npu/core/buf.c:501-520): each group's exact int32 partial, scaled as
 * ((float)P * aScale[m*Sk+g]) * bScale[g*N+n], is added to C in ascending g from 0.0f. Built without FMA
 * contraction (-ffp-contract=off), so the float sequence is the reference's. Returns -1 on bad
 * arguments or allocation failure. */
struct cpu_grouped { int K, N, G; const int8_t *A, *B; const float *aS, *bS; float *C; int fail; };

static void grouped_rows(int lo, int hi, void *arg) {
    struct cpu_grouped *g = arg;
    const int Sk = g->K / g->G;
    int32_t *acc = malloc((size_t)g->N * sizeof *acc);
    if (!acc) { g->fail = 1; return; }
    for (int m = lo; m < hi; m++) {
        float *cr = g->C + (size_t)m * g->N;
        for (int n = 0; n < g->N; n++) cr[n] = 0.0f;
        for (int q = 0; q < Sk; q++) {
            /* row m of A restricted to group q, times the group's K-rows of B: an exact int32 partial */
            const int8_t *a = g->A + (size_t)m * g->K + (size_t)q * g->G;
            const int8_t *bq = g->B + (size_t)q * g->G * g->N;
            memset(acc, 0, (size_t)g->N * sizeof *acc);
            for (int k = 0; k < g->G; k++) {
                const int32_t av = a[k];
                if (!av) continue;
                const int8_t *b = bq + (size_t)k * g->N;
                for (int n = 0; n < g->N; n++) acc[n] += av * (int32_t)b[n];
            }
            const float as = g->aS[(size_t)m * Sk + q];
            const float *bs = g->bS + (size_t)q * g->N;
            for (int n = 0; n < g->N; n++) cr[n] += (float)acc[n] * as * bs[n];
        }
    }
    free(acc);
}

int orki_cpu_gemm_grouped(int M, int K, int N, int G, const int8_t *A, const int8_t *B_kn, const float *aS,
                          const float *bS, float *C) {
    if (M < 1 || K < 1 || N < 1 || G < 1 || K % G || !A || !B_kn || !aS || !bS || !C) return -1;
    struct cpu_grouped g = {K, N, G, A, B_kn, aS, bS, C, 0};
    if (M == 1) grouped_rows(0, 1, &g);
    else orki_parallel_for(M, grouped_rows, &g);
    return g.fail ? -1 : 0;
}
