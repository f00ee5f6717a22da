/* run.c -- matmul entry points: argument checks, operand residency, plan, launch.
 *
 * Reference entry points: ork_i8_mm_run (src/npu/i8/run.c:139-180), ork_i4_mm_run (src/npu/i4/run.c:235-365),
 * ork_f16_mm_run (src/npu.c:1824-1832); the A/C overlap guard orki_check_overlap
 * (src/npu/core/submit.c:532-539) and its -1. Behaviour kept: run dtype must match the pack dtype,
 * overlapping A and C are refused, C is valid on return. What changes: one HIP launch (plus a split-K
 * reduce when planned) replaces the per-slice NPU submits and the host K-slice accumulate; operands
 * already in HBM (ork_dev_alloc) are used in place; a host A is uploaded from pinned staging by one DMA
 * copy on the context's stream, and a host C up to 1 MiB is written by the kernels straight into pinned,
 * device-mapped memory (larger ones come back by one D2H copy). An offline context (no device) runs an offline
 * weight's host codes on the CPU, exactly, as the reference's offline branches do (src/npu/i8/run.c:140,
 * src/npu/i4/run.c:236, :368-369); a device context never falls back: a device error returns -1. */
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
    if (c->offline && w->codes && want_dt != DT_F16) {
        /* OFFLINE: the exact CPU MAC on the weight's codes [K][N], whatever its pack dtype, as the reference */
        if (M > 0) ork_i8_mm_run_cpu(M, w->K, w->N, (const int8_t *)A, w->codes, (int32_t *)C);
        return 0;
    }
    if (orki_need_device(c, who)) return -1;
    if (w->dtype != want_dt || !w->dB) {
        orki_err("%s: weight is %s, run needs %s", who, w->dB ? dt_name(w->dtype) : "offline", dt_name(want_dt));
        return -1;
    }
    if (M < 1) { orki_err("%s: M=%d", who, M); return -1; }
    const int K = w->K, N = w->N;
    if ((w->rkind == ORKH_I4U || w->rkind == ORKH_NF4) && K > ORKI_I4_K_MAX) {
        orki_err("%s: K=%d exceeds the int4 path's exact-accumulation bound (K <= 131040)", who, K);
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
    int cmode = ORKI_C_INPLACE;
    if (!a_dev && !(dA = orki_host_a(c, A, abytes))) { orki_hip_fail(who); return -1; }
    if (!c_dev && !(dC = orki_host_c(c, C, cbytes, &cmode))) { orki_hip_fail(who); return -1; }

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
    if (!c_dev && orki_host_c_post(c, C, dC, cbytes, cmode)) { orki_hip_fail(who); return -1; }
    if (c->async && a_dev && c_dev) return 0;
    if (orkh_sync(c->stream)) { orki_hip_fail(who); return -1; }
    if (!c_dev) orki_host_c_done(c, C, cbytes, cmode);
    return 0;
}

int ork_i8_mm_run(ork_npu *c, ork_w *w, int M, const int8_t *A, int32_t *C) {
    return run_common("ork_i8_mm_run", c, w, DT_I8, M, A, C, 1);
}

/* ork_i8_mm_run for callers that cannot allocate (code under HIP graph capture, serving loops that forbid
 * hipMalloc): A and C must already be device memory, and a split-K plan's partials go to the library's static
 * per-GPU scratch array (ORKH_SCRATCH_BYTES) instead of the context's grown-on-demand workspace. Nothing here
 * allocates, frees or calls an allocating routine. -1 on a NULL argument, an offline context, a weight that
 * is not an int8-run weight, host A or C, A/C overlap, a plan whose partials exceed the scratch array, or a
 * device failure. Returns after the launch in async mode, else after the stream sync, like ork_i8_mm_run.
 * Calls that overlap on one GPU share its scratch array and race. */
int ork_i8_mm_run_noalloc(ork_npu *c, ork_w *w, int M, const int8_t *A, int32_t *C) {
    const char *who = "ork_i8_mm_run_noalloc";
    if (!c || !w || !A || !C) { orki_err("%s: NULL argument", who); return -1; }
    if (orki_need_device(c, who)) return -1;
    if (w->dtype != DT_I8 || !w->dB) { orki_err("%s: weight is not a resident int8-run weight", who); return -1; }
    if (M < 1) { orki_err("%s: M=%d", who, M); return -1; }
    const int K = w->K, N = w->N;
    if ((w->rkind == ORKH_I4U || w->rkind == ORKH_NF4) && K > ORKI_I4_K_MAX) {
        orki_err("%s: K=%d exceeds the int4 path's exact-accumulation bound (K <= 131040)", who, K);
        return -1;
    }
    const size_t abytes = (size_t)M * K, cbytes = (size_t)M * N * 4;
    if (abytes >= ORKH_MAX_OPERAND_BYTES || w->dbytes >= ORKH_MAX_OPERAND_BYTES) {
        orki_err("%s: operand too large for 32-bit buffer offsets (A %zu B, weight %zu B)", who, abytes, w->dbytes);
        return -1;
    }
    if ((uintptr_t)A % 16 || !orkh_ptr_is_device(A) || !orkh_ptr_is_device(C)) {
        orki_err("%s: A (16-byte aligned) and C must be device memory", who);
        return -1;
    }
    if (orki_check_overlap(who, (uintptr_t)A, (uintptr_t)A + abytes, (uintptr_t)C, (uintptr_t)C + cbytes)) return -1;
    orkh_plan q;
    size_t ws = 0;
    orki_plan(c, w->rkind, M, K, N, w->KB, &q, &ws);
    if (ws > ORKH_SCRATCH_BYTES) {
        orki_err("%s: the plan's split-K partials need %zu B, above the %u B scratch array", who, ws,
                 (unsigned)ORKH_SCRATCH_BYTES);
        return -1;
    }
    if (ws) q.ws = c->dev.scratch;
    orkh_mm p;
    memset(&p, 0, sizeof p);
    p.kind = w->rkind;
    p.M = M;
    p.K = K;
    p.N = N;
    p.KB = w->KB;
    p.A = A;
    p.lda = K;
    p.B = w->dB;
    p.C = C;
    p.ldc = N;
    memcpy(p.lut, w->lut, sizeof p.lut);
    if (orkh_mm_launch(&p, &q, c->stream)) { orki_hip_fail(who); return -1; }
    if (c->async) return 0;
    if (orkh_sync(c->stream)) { orki_hip_fail(who); return -1; }
    return 0;
}

int ork_i4_mm_run(ork_npu *c, ork_w *w, int M, const int8_t *A, int32_t *C) {
    return run_common("ork_i4_mm_run", c, w, DT_I4, M, A, C, 1);
}

int ork_f16_mm_run(ork_npu *c, ork_w *w, int M, const ork_f16 *A, float *C) {
    return run_common("ork_f16_mm_run", c, w, DT_F16, M, A, C, 2);
}

/* Grouped runs: ork_i8_mm_run_grouped (src/npu/i8/run.c:45-137) and ork_i4_mm_run_grouped
 * (src/npu/i4/run.c:367-459). C f32[M][N] = the per-K-group int32 partials, each scaled by
 * aScale[m*(K/G)+g] and bScale[g*N+n] and summed in ascending g (src/npu/core/buf.c:501-520), so the result
 * is bit-identical to the reference's offline path. -1 on a NULL argument, a weight of the wrong kind or
 * without a group size, A/C overlap, an offline context or a device failure (the reference's -1 cases);
 * -3 for a group size the kernels cannot split at (G % 32), as the reference answers -3 for a device group
 * size it does not support. Operands and scales may be host memory or ork_dev_alloc buffers. */
static int run_grouped(const char *who, ork_npu *c, ork_w *w, int want_dt, int M, const int8_t *A, const float *aS,
                       const float *bS, float *C) {
    if (!c || !w || !A || !aS || !bS || !C || M < 1) { orki_err("%s: NULL argument or M < 1", who); return -1; }
    if (c->offline && w->codes) {
        /* OFFLINE: the per-group accumulate on the CPU (src/npu/i8/run.c:48-49, src/npu/i4/run.c:368-369) */
        if (w->gsize < 1 || w->K % w->gsize) { orki_err("%s: weight has no group size", who); return -1; }
        return orki_cpu_gemm_grouped(M, w->K, w->N, w->gsize, A, w->codes, aS, bS, C);
    }
    if (orki_need_device(c, who)) return -1;
    if (w->dtype != want_dt || !w->dB || w->rkind == ORKH_F16) {
        orki_err("%s: weight is %s, this run needs %s", who, w->dB ? dt_name(w->dtype) : "offline", dt_name(want_dt));
        return -1;
    }
    const int K = w->K, N = w->N, G = w->gsize;
    if (G < 1 || K % G) {
        orki_err("%s: weight has no group size (ork_i4_mm_pack_grouped / ork_w_set_group)", who);
        return -1;
    }
    if (G % 32) {
        orki_err("%s: G=%d unsupported on the device: a group must be whole 32-k chunks", who, G);
        return -3;
    }
    if ((w->rkind == ORKH_I4U || w->rkind == ORKH_NF4) && K > ORKI_I4_K_MAX) {
        orki_err("%s: K=%d exceeds the int4 path's exact-accumulation bound (K <= 131040)", who, K);
        return -1;
    }
    const int Sk = K / G;
    const size_t abytes = (size_t)M * K, cbytes = (size_t)M * N * 4, asz = (size_t)M * Sk * 4,
                 bsz = (size_t)Sk * N * 4;
    if (abytes >= ORKH_MAX_OPERAND_BYTES || w->dbytes >= ORKH_MAX_OPERAND_BYTES) {
        orki_err("%s: operand too large for 32-bit buffer offsets", who);
        return -1;
    }
    if (orki_check_overlap(who, (uintptr_t)A, (uintptr_t)A + abytes, (uintptr_t)C, (uintptr_t)C + cbytes)) return -1;

    const int a_dev = orki_dev_find(c, A, abytes) && ((uintptr_t)A % 16 == 0);
    const int c_dev = orki_dev_find(c, C, cbytes);
    const int as_dev = orki_dev_find(c, aS, asz), bs_dev = orki_dev_find(c, bS, bsz);
    const void *dA = A;
    const float *dAS = aS, *dBS = bS;
    float *dC = C;
    if (!a_dev && !(dA = orki_host_a(c, A, abytes))) { orki_hip_fail(who); return -1; }
    if (!as_dev || !bs_dev) {
        const size_t boff = (asz + 255) & ~(size_t)255;
        uint8_t *st = orki_stage(c, &c->sS, boff + bsz);
        if (!st) { orki_hip_fail(who); return -1; }
        if (!as_dev) {
            if (orkh_h2d(st, aS, asz, c->stream)) { orki_hip_fail(who); return -1; }
            dAS = (const float *)st;
        }
        if (!bs_dev) {
            if (orkh_h2d(st + boff, bS, bsz, c->stream)) { orki_hip_fail(who); return -1; }
            dBS = (const float *)(st + boff);
        }
    }
    int cmode = ORKI_C_INPLACE;
    if (!c_dev && !(dC = orki_host_c(c, C, cbytes, &cmode))) { orki_hip_fail(who); return -1; }
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
    p.ldc = N;
    memcpy(p.lut, w->lut, sizeof p.lut);
    orkh_plan q;
    orki_plan_grouped(c, w->rkind, M, K, N, w->KB, G, &q);
    const int rc = orkh_mm_launch_grouped(&p, &q, G, dAS, dBS, dC, N, c->stream);
    if (rc) { orki_hip_fail(who); return -1; }
    if (!c_dev && orki_host_c_post(c, C, dC, cbytes, cmode)) { orki_hip_fail(who); return -1; }
    if (c->async && a_dev && c_dev && as_dev && bs_dev) return 0;
    if (orkh_sync(c->stream)) { orki_hip_fail(who); return -1; }
    if (!c_dev) orki_host_c_done(c, C, cbytes, cmode);
    return 0;
}

int ork_i8_mm_run_grouped(ork_npu *c, ork_w *w, int M, const int8_t *A, const float *aScale, const float *bScale, float *C) {
    return run_grouped("ork_i8_mm_run_grouped", c, w, DT_I8, M, A, aScale, bScale, C);
}

int ork_i4_mm_run_grouped(ork_npu *c, ork_w *w, int M, const int8_t *A, const float *aScale, const float *bScale, float *C) {
    return run_grouped("ork_i4_mm_run_grouped", c, w, DT_I4, M, A, aScale, bScale, C);
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

const char *ork_w_grouped_plan_name(ork_npu *c, const ork_w *w, int M) {
    static _Thread_local char b[64];
    if (!c || !w || w->rkind < 0 || w->rkind == ORKH_F16 || M < 1 || w->gsize < 1) return "none";
    orkh_plan q;
    orki_plan_grouped(c, w->rkind, M, w->K, w->N, w->KB, w->gsize, &q);
    const char *k = w->rkind == ORKH_I8 ? "i8" : w->rkind == ORKH_I4U ? "i4u" : "nf4";
    if (q.algo == ORKH_ALGO_TILED2) snprintf(b, sizeof b, "tiled2g_%s_%dx%d", k, q.bm, q.bn);
    else if (q.algo == ORKH_ALGO_GEMV) snprintf(b, sizeof b, "grouped_%s_gemvh_w%d", k, q.wpg);
    else snprintf(b, sizeof b, "grouped_%s_mt%d", k, q.mt);
    return b;
}
