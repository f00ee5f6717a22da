/* cpu_gemm.c -- ork_i8_mm_run_cpu: the public CPU int8 GEMM (reference include/ork/run.h:132,
 * src/npu/core/buf.c:578-580 forwarding to orki_cpu_gemm_i32, :428-477).
 *
 * An explicitly-CPU API the reference exports so a caller can time the CPU side of a routing decision;
 * it is not a fallback of any device entry point. Exact int32: the k-outer AXPY keeps the C row hot
 * while B streams, skips zero activations, and parallelises over M rows on the host pool. */
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
