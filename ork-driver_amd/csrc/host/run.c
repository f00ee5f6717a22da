/* run.c -- matmul entry points: argument checks, operand residency, plan, launch.
 *
 * Reference entry points: ork_i8_mm_run (src/npu/i8/run.c:139-180), ork_i4_mm_run (src/npu/i4/run.c:235-365),
 * ork_f16_mm_run (src/npu.c:1824-1832); the A/C overlap guard orki_check_overlap
 * (src/npu/core/submit.c:532-539) and its -1. Behaviour kept: run dtype must match the pack dtype,
 * overlapping A and C are refused, C is valid on return. What changes: one HIP launch (plus a split-K
 * reduce when planned) replaces the per-slice NPU submits and the host K-slice accumulate; operands
 * already in HBM (ork_dev_alloc) are used in place, host operands move by async copies on the
 * context's stream. There is no CPU fallback: an offline context or a device error returns -1. */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "internal.h"

int orki_check_overlap(const char *name, uintptr_t a0, uintptr_t a1, uintptr_t c0, uintptr_t c1) {
    if (a0 < c1 && c0 < a1) {
        fprintf(stderr, "[ork] ERROR [%s]: memory overlap detected! A [%p, %p) overlaps with C [%p, %p).\n",
                name, (void *)a0, (void *)a1, (void *)c0, (void *)c1);
        return 1;
    }
    return 0;
}

static const char *dt_name(int dt) { return dt == DT_F16 ? "fp16" : dt == DT_I8 ? "int8" : "int4"; }

/* esz_a: bytes per A element; C is always 4 bytes per element. */
static int run_common(const char *who, ork_npu *c, ork_w *w, int want_dt, int M, const void *A, void *C, int esz_a) {
    if (!c || !w || !A || !C) { orki_err("%s: NULL argument", who); return -1; }
    if (orki_need_device(c, who)) return -1;
    if (w->dtype != want_dt || !w->dB) {
        orki_err("%s: weight is %s, run needs %s", who, w->dB ? dt_name(w->dtype) : "offline", dt_name(want_dt));
        return -1;
    }
    if (M < 1) { orki_err("%s: M=%d", who, M); return -1; }
    const int K = w->K, N = w->N;
    if ((w->rkind == ORKH_I4U || w->rkind == ORKH_NF4) && K > 131072) {
        orki_err("%s: K=%d exceeds the int4 path's exact-accumulation bound (131072)", who, K);
        return -1;
    }
    const size_t abytes = (size_t)M * K * esz_a, cbytes = (size_t)M * N * 4;
    if (abytes >= ORKH_MAX_OPERAND_BYTES || w->dbytes >= ORKH_MAX_OPERAND_BYTES) {
        orki_err("%s: operand too large for 32-bit buffer offsets (A %zu B, weight %zu B)", who, abytes, w->dbytes);
        return -1;
    }
    if (orki_check_overlap(who, (uintptr_t)A, (uintptr_t)A + abytes, (uintptr_t)C, (uintptr_t)C + cbytes)) return -1;

    const int a_dev = orki_dev_find(c, A, abytes) && ((uintptr_t)A % 16 == 0);
    const int c_dev = orki_dev_find(c, C, cbytes);
    const void *dA = A;
    void *dC = C;
    if (!a_dev) {
        void *s = orki_stage(c, &c->sA, abytes);
        if (!s || orkh_h2d(s, A, abytes, c->stream)) { orki_hip_fail(who); return -1; }
        dA = s;
    }
    if (!c_dev) {
        dC = orki_stage(c, &c->sC, cbytes);
        if (!dC) { orki_hip_fail(who); return -1; }
    }

    orkh_plan q;
    size_t ws = 0;
    orki_plan(c, w->rkind, M, K, N, w->KB, &q, &ws);
    if (ws) {
        q.ws = orki_stage(c, &c->sW, ws);
        if (!q.ws) { orki_hip_fail(who); return -1; }
    }
    orkh_mm p;
    memset(&p, 0, sizeof p);
    p.kind = w->rkind;
    p.M = M;
    p.K = K;
    p.N = N;
    p.KB = w->KB;
    p.A = dA;
    p.lda = K;
    p.B = w->dB;
    p.C = dC;
    p.ldc = N;
    memcpy(p.lut, w->lut, sizeof p.lut);
    if (orkh_mm_launch(&p, &q, c->stream)) { orki_hip_fail(who); return -1; }
    if (!c_dev && orkh_d2h(C, dC, cbytes, c->stream)) { orki_hip_fail(who); return -1; }
    if (c->async && a_dev && c_dev) return 0;
    if (orkh_sync(c->stream)) { orki_hip_fail(who); return -1; }
    return 0;
}

int ork_i8_mm_run(ork_npu *c, ork_w *w, int M, const int8_t *A, int32_t *C) {
    return run_common("ork_i8_mm_run", c, w, DT_I8, M, A, C, 1);
}

int ork_i4_mm_run(ork_npu *c, ork_w *w, int M, const int8_t *A, int32_t *C) {
    return run_common("ork_i4_mm_run", c, w, DT_I4, M, A, C, 1);
}

int ork_f16_mm_run(ork_npu *c, ork_w *w, int M, const ork_f16 *A, float *C) {
    return run_common("ork_f16_mm_run", c, w, DT_F16, M, A, C, 2);
}

const char *ork_w_plan_name(ork_npu *c, const ork_w *w, int M) {
    if (!c || !w || w->rkind < 0 || M < 1) return "none";
    orkh_plan q;
    size_t ws;
    orki_plan(c, w->rkind, M, w->K, w->N, w->KB, &q, &ws);
    orkh_mm p;
    memset(&p, 0, sizeof p);
    p.kind = w->rkind;
    return orkh_mm_variant(&p, &q);
}
