/* Prints the planner's choice for each "kind M K N" argument quadruple on a 256-CU device, one line each, named as
 * the library names its launches (orkh_mm_variant). Built from the host planner source alone, with no GPU code. */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "internal.h"

/* the planner's one call into the HIP layer (grouped runs: the LDS-ring kernel's ring size); not reached here */
int orkh_tiled2_ring_lds(int kind, int bm, int bn) {
    (void)kind, (void)bm, (void)bn;
    return 163840;
}

/* the LDS-ring kernel's two-slot ring: the tiles the kernel builds it for (its LDS arithmetic, restated: int8 and
 * fp16 on 64 x 192, 128 x 128 and 128 x 96; uniform int4 on 128 x 128 only, its 64 x 192 and 128 x 96 stages being
 * 41 and 45 KiB; never NF4) */
int orkh_tiled2_ring2_ok(int kind, int bm, int bn) {
    const int big = (bm == 128 && (bn == 128 || bn == 96)) || (bm == 64 && bn == 192);
    if (kind == ORKH_I8 || kind == ORKH_F16) return big;
    if (kind == ORKH_I4U) return bm == 128 && bn == 128;
    return 0;
}

static const char *name(int kind, const orkh_plan *q) {
    static char b[96];
    static const char *kn[] = {"i8", "i4u", "nf4", "f16"};
    const char *k = kn[kind];
    if (q->algo == ORKH_ALGO_GEMV)
        snprintf(b, sizeof b, "%s_%s_w%d_kbw%d_ks%d", q->half ? "gemvh" : "gemv", k, q->wpg, q->kbw, q->ksplit);
    else if (q->algo == ORKH_ALGO_STREAM)
        snprintf(b, sizeof b, "stream_%s_mt%d_w%d_kbw%d_ks%d%s", k, q->mt, q->wpg, q->kbw, q->ksplit,
                 q->np == 2 ? "_p2" : q->half ? "_h" : "");
    else if (q->ksplit > 1)
        snprintf(b, sizeof b, "%s_%s_%dx%d_ks%d%s%s", q->algo == ORKH_ALGO_TILED2 ? "tiled2" : "tiled", k, q->bm, q->bn,
                 q->ksplit, q->algo == ORKH_ALGO_TILED2 && q->aline ? "_al" : "",
                 q->algo == ORKH_ALGO_TILED2 && q->ring == 2 ? "_r2" : "");
    else
        snprintf(b, sizeof b, "%s_%s_%dx%d%s%s", q->algo == ORKH_ALGO_TILED2 ? "tiled2" : "tiled", k, q->bm, q->bn,
                 q->algo == ORKH_ALGO_TILED2 && q->aline ? "_al" : "", q->algo == ORKH_ALGO_TILED2 && q->ring == 2 ? "_r2" : "");
    return b;
}

int main(int argc, char **argv) {
    ork_npu c;
    memset(&c, 0, sizeof c);
    c.cores = 256;
    for (int i = 1; i + 3 < argc; i += 4) {
        const int kind = atoi(argv[i]), M = atoi(argv[i + 1]), K = atoi(argv[i + 2]), N = atoi(argv[i + 3]);
        const int kpb = kind == ORKH_I8 ? 64 : kind == ORKH_F16 ? 32 : 128;
        orkh_plan q;
        size_t ws = 0;
        orki_plan(&c, kind, M, K, N, (K + kpb - 1) / kpb, &q, &ws);
        printf("%d %d %d %d %s %zu\n", kind, M, K, N, name(kind, &q), ws);
    }
    return 0;
}
