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
    orki_ptok pt;
    if (c->offline && w->codes && want_dt != DT_F16) {
        /* OFFLINE: the exact CPU MAC on the weight's codes [K][N], whatever its pack dtype, as the reference */
        orki_prof_begin(c, &pt, 0);
        if (M > 0) ork_i8_mm_run_cpu(M, w->K, w->N, (const int8_t *)A, w->codes, (int32_t *)C);
        orki_prof_end(c, &pt, who, "cpu");
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
    orki_prof_begin(c, &pt, 1);
    if (!a_dev && !(dA = orki_host_a(c, A, abytes))) { orki_hip_fail(who); return -1; }
    if (!c_dev && !(dC = orki_host_c(c, C, cbytes, &cmode))) { orki_hip_fail(who); return -1; }

    orkh_plan q;
    size_t ws = 0;
    orki_plan(c, w->rkind, M, K, N, w->KB, &q, &ws);
    if (ws) {
        q.ws = orki_ws_stage(c, ws, NULL);
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
    orki_prof_launched(c, &pt);
    if (c->async && a_dev && c_dev && !(ws && c->ws_guard)) {
        orki_prof_end(c, &pt, who, c->prof ? orkh_mm_variant(&p, &q) : NULL);
        return 0;
    }
    if (orkh_sync(c->stream)) { orki_hip_fail(who); return -1; }
    if (!c_dev) orki_host_c_done(c, C, cbytes, cmode);
    if (ws && orki_ws_check(c, q.ws, ws, who)) return -1;
    orki_prof_end(c, &pt, who, c->prof ? orkh_mm_variant(&p, &q) : NULL);
    orki_prof_settle(c);
    return 0;
}

int ork_i8_mm_run(ork_npu *c, ork_w *w, int M, const int8_t *A, int32_t *C) {
    return run_common("ork_i8_mm_run", c, w, DT_I8, M, A, C, 1);
}

/* ork_i8_mm_run for callers that cannot allocate (code under HIP graph capture, serving loops that forbid
 * hipMalloc): A (16-byte aligned) and C must already be device memory, and a split-K plan's partials go to the
 * library's static per-GPU scratch array (ORKH_SCRATCH_BYTES) instead of the context's grown-on-demand workspace.
 * Nothing here allocates, frees or calls an allocating routine. -1 on a NULL argument, an offline context, a
 * weight that is not an int8-run weight, host A or C, an A that is not 16-byte aligned (ork_i8_mm_run stages such
 * an A; this entry point cannot), A/C overlap, a plan whose partials exceed the scratch array, a call outside
 * async mode on a stream that is being captured, or a device failure. Returns after the launch in async mode,
 * else after the stream sync, like ork_i8_mm_run. Calls that overlap on one GPU share its scratch array and race. */
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
    /* Outside async mode the call ends with a stream synchronisation, which would invalidate a capture in progress */
    if (!c->async && orkh_stream_capturing(c->stream) != 0) {
        orki_err("%s: the stream is being captured (or its state is unknown): async mode is required there", who);
        return -1;
    }
    orkh_plan q;
    size_t ws = 0;
    orki_plan(c, w->rkind, M, K, N, w->KB, &q, &ws);
    if (ws > ORKH_SCRATCH_BYTES) {
        orki_err("%s: the plan's split-K partials need %zu B, above the %u B scratch array", who, ws,
                 (unsigned)ORKH_SCRATCH_BYTES);
        return -1;
    }
    if (ws && c->ws_guard && ws + 2 * ORKI_WS_GUARD > ORKH_SCRATCH_BYTES) {
        orki_err("%s: the plan's split-K partials and their guard bands exceed the scratch array", who);
        return -1;
    }
    if (ws && !(q.ws = orki_ws_stage(c, ws, c->dev.scratch))) { orki_hip_fail(who); return -1; }
    orki_ptok pt;
    orki_prof_begin(c, &pt, 0);
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
    if (c->async && !(ws && c->ws_guard)) {
        orki_prof_end(c, &pt, who, c->prof ? orkh_mm_variant(&p, &q) : NULL);
        return 0;
    }
    if (orkh_sync(c->stream)) { orki_hip_fail(who); return -1; }
    if (ws && orki_ws_check(c, q.ws, ws, who)) return -1;
    orki_prof_end(c, &pt, who, c->prof ? orkh_mm_variant(&p, &q) : NULL);
    return 0;
}

/* The one-row run with a fused prologue and epilogue (include/ork/hip.h): checks, then one k_gemv_row launch with
 * the M = 1 planner's panel rule (half a panel per workgroup unless whole panels already spread evenly over the
 * CUs). */
static int dev_ok(ork_npu *c, const void *p, size_t n) { return p && (orki_dev_find(c, p, n) || orkh_ptr_is_device(p)); }

static int spans_overlap(const void *a, size_t na, const void *b, size_t nb) {
    return (uintptr_t)a < (uintptr_t)b + nb && (uintptr_t)b < (uintptr_t)a + na;
}

int ork_i8_mm_run_row(ork_npu *c, int S, ork_w *const *w, const ork_row_op *op) {
    const char *who = "ork_i8_mm_run_row";
    if (!c || !w || !op || S < 1 || S > 3) { orki_err("%s: NULL argument or S outside 1..3", who); return -2; }
    if (orki_need_device(c, who)) return -1;
    const int epi = op->epilogue, pro = op->prologue;
    if ((epi == ORK_COL_RESID && S != 1) || (epi == ORK_COL_SWIGLU && S != 2) ||
        (epi != ORK_COL_STORE && epi != ORK_COL_RESID && epi != ORK_COL_SWIGLU) ||
        (pro != ORK_ROW_RMSNORM && pro != ORK_ROW_QUANT)) {
        orki_err("%s: prologue %d / epilogue %d with %d weights is not a built combination", who, pro, epi, S);
        return -2;
    }
    const int K = w[0] ? w[0]->K : 0;
    for (int i = 0; i < S; i++) {
        const ork_w *wi = w[i];
        if (!wi || !wi->dB || wi->dtype != DT_I8 || wi->rkind == ORKH_F16 || wi->K != K) {
            orki_err("%s: weight %d is not a resident int8-run weight of K=%d", who, i, K);
            return -2;
        }
        if ((size_t)wi->KB * (wi->rkind == ORKH_I8 ? 64 : 128) > ORK_ROW_KMAX) {
            orki_err("%s: K=%d exceeds the row bound (%d)", who, K, ORK_ROW_KMAX);
            return -2;
        }
    }
    if (epi == ORK_COL_SWIGLU && (w[1]->N != w[0]->N || w[1]->rkind != w[0]->rkind || w[1]->KB != w[0]->KB ||
                                  memcmp(w[1]->lut, w[0]->lut, sizeof w[0]->lut))) {
        orki_err("%s: gate and up weights differ in shape or kind", who);
        return -2;
    }
    const size_t rb = (size_t)K * 4, nb0 = (size_t)w[0]->N * 4;
    int ok = dev_ok(c, op->row, rb) && (pro != ORK_ROW_RMSNORM || dev_ok(c, op->norm_w, rb)) &&
             (!op->row_scale || dev_ok(c, op->row_scale, 4));
    if (epi == ORK_COL_STORE) {
        for (int i = 0; i < S; i++)
            ok = ok && dev_ok(c, op->C[i], (size_t)w[i]->N * 4) && !spans_overlap(op->C[i], (size_t)w[i]->N * 4, op->row, rb);
    } else {
        ok = ok && dev_ok(c, op->w_scale[0], nb0) && (epi != ORK_COL_SWIGLU || dev_ok(c, op->w_scale[1], nb0)) &&
             dev_ok(c, op->out, nb0) && !spans_overlap(op->out, nb0, op->row, rb);
    }
    if (!ok) {
        orki_err("%s: every operand must be device memory, and the outputs must not overlap the row", who);
        return -2;
    }
    orkh_row r;
    memset(&r, 0, sizeof r);
    r.kind = w[0]->rkind;
    r.K = K;
    r.KB = w[0]->KB;
    memcpy(r.lut, w[0]->lut, sizeof r.lut);
    r.pro = pro == ORK_ROW_RMSNORM ? ORKH_ROW_RMSNORM : ORKH_ROW_QUANT;
    r.epi = epi == ORK_COL_STORE ? ORKH_COL_STORE : epi == ORK_COL_RESID ? ORKH_COL_RESID : ORKH_COL_SWIGLU;
    r.nt = S;
    int P = 0;
    for (int i = 0; i < S; i++) {
        if (w[i]->KB != r.KB) {
            orki_err("%s: the weights differ in K-blocks", who);
            return -2;
        }
        r.B[i] = w[i]->dB;
        r.nb[i] = w[i]->N / 16;
        r.C[i] = op->C[i];
        if (epi != ORK_COL_SWIGLU || i == 0) P += r.nb[i];
    }
    r.row = op->row;
    r.nw = op->norm_w;
    r.eps = op->eps;
    r.as_out = op->row_scale;
    r.ws0 = op->w_scale[0];
    r.ws1 = op->w_scale[1];
    r.x = epi == ORK_COL_RESID ? op->out : NULL;
    r.y = epi == ORK_COL_SWIGLU ? op->out : NULL;
    const int cu = c->cores > 0 ? c->cores : 256;
    r.half = !(P >= cu && (2 * P + cu - 1) / cu >= 2 * ((P + cu - 1) / cu));
    orki_ptok pt;
    orki_prof_begin(c, &pt, 1);
    const int rc = orkh_row_launch(&r, c->stream);
    if (rc == -2) {
        orki_err("%s: prologue %d / epilogue %d is not built for this weight kind", who, pro, epi);
        return -2;
    }
    if (rc) { orki_hip_fail(who); return -1; }
    orki_prof_launched(c, &pt);
    if (!c->async && orkh_sync(c->stream)) { orki_hip_fail(who); return -1; }
    orki_prof_end(c, &pt, who, r.half ? "gemv_row_half" : "gemv_row");
    if (!c->async) orki_prof_settle(c);
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
    orki_ptok pt;
    if (c->offline && w->codes) {
        /* OFFLINE: the per-group accumulate on the CPU (src/npu/i8/run.c:48-49, src/npu/i4/run.c:368-369) */
        if (w->gsize < 1 || w->K % w->gsize) { orki_err("%s: weight has no group size", who); return -1; }
        orki_prof_begin(c, &pt, 0);
        const int rc = orki_cpu_gemm_grouped(M, w->K, w->N, w->gsize, A, w->codes, aS, bS, C);
        if (!rc) orki_prof_end(c, &pt, who, "cpu");
        return rc;
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
    orki_prof_begin(c, &pt, 1);
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
    orki_prof_launched(c, &pt);
    if (c->async && a_dev && c_dev && as_dev && bs_dev) {
        orki_prof_end(c, &pt, who, c->prof ? ork_w_grouped_plan_name(c, w, M) : NULL);
        return 0;
    }
    if (orkh_sync(c->stream)) { orki_hip_fail(who); return -1; }
    if (!c_dev) orki_host_c_done(c, C, cbytes, cmode);
    orki_prof_end(c, &pt, who, c->prof ? ork_w_grouped_plan_name(c, w, M) : NULL);
    orki_prof_settle(c);
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
