/* chain.c -- multi-matmul submit: ork_{i8,i4}_mm_run_chain / _run_stream, ork_f16_mm_run_stream.
 *
 * Reference: ork_i8_mm_run_chain (src/npu/i8/chain.c:56-71, validation :197-250), ork_i8_mm_run_stream
 * (src/npu/i8/run.c:712-740), ork_i4_mm_run_chain (src/npu/i4/chain.c:106), ork_i4_mm_run_stream
 * (src/npu/i4/stream.c:116), ork_f16_mm_run_stream (src/npu/f16/stream.c:170). Behaviour kept: S
 * independent matmuls, each result equal to its single run; -2 for bad arguments (S outside 1..1024,
 * NULL weight, M < 1, wrong dtype), -1 for A/C overlap; C row stride override (cstride) for int8.
 * What changes: no PC-chained NPU programs, cores or doorbells. Every M = 1 task of one resident kind
 * goes into a grouped GEMV launch (ORKH_GROUP_MAX tasks each); tasks of one integer kind, M > 1 and K whose summed
 * columns plan to the LDS-ring kernel unsplit go into one grouped tiled launch (ORKH_TGROUP_MAX each: a
 * prefill's q/k/v or gate/up); the remaining tasks launch back to back
 * on the context's stream with their normal plans, and host operands move in one pinned staging pass. An
 * offline context runs each task's host codes on the CPU (cpu_chain below), as the reference's int8 chain
 * and int4 chain / stream do; its int8 stream and fp16 stream have no offline branch and return -1 here too. */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "internal.h"

typedef struct {
    ork_w *w;
    int M;
    const void *A;
    void *C;
    int ldc;        /* C row stride in elements */
    int a_dev, c_dev;
    const void *dA; /* device pointer used by the kernel */
    void *dC;
    size_t abytes, cbytes;
} ctask;

static size_t al256(size_t n) { return (n + 255) & ~(size_t)255; }

/* An fp16 GEMV task whose own plan splits K exactly as the grouped whole-panel launch would (wpg waves, each over
 * one run of ceil(KB / wpg) blocks): its fp32 results in a group equal its single run's bit for bit. */
static int f16_groupable(const orkh_plan *q, int KB, int wpg) {
    return !q->half && q->wpg == wpg && q->kbw == (KB + wpg - 1) / wpg;
}

/* esz_a: bytes per A element. tasks arrive as (w, M, A, C, cstride) in a normalised array. */
static int chain_common(const char *who, ork_npu *c, int S, ctask *t, int want_dt, int esz_a) {
    if (orki_need_device(c, who)) return -1;
    for (int i = 0; i < S; i++) {
        ork_w *w = t[i].w;
        if (!w || !w->dB || w->dtype != want_dt || t[i].M < 1 || !t[i].A || !t[i].C) {
            orki_err("%s: task %d: bad weight, dtype, M or pointer", who, i);
            return -2;
        }
        if (t[i].ldc < w->N) {
            orki_err("%s: task %d: cstride %d < N %d", who, i, t[i].ldc, w->N);
            return -2;
        }
        if ((w->rkind == ORKH_I4U || w->rkind == ORKH_NF4) && w->K > ORKI_I4_K_MAX) {
            orki_err("%s: task %d: K=%d exceeds the int4 path's exact-accumulation bound (K <= 131040)", who, i, w->K);
            return -2;
        }
        t[i].abytes = (size_t)t[i].M * w->K * esz_a;
        t[i].cbytes = ((size_t)(t[i].M - 1) * t[i].ldc + w->N) * 4;
        if (t[i].abytes >= ORKH_MAX_OPERAND_BYTES || (size_t)t[i].M * t[i].ldc * 4 >= ORKH_MAX_OPERAND_BYTES) {
            orki_err("%s: task %d: operand too large for 32-bit buffer offsets", who, i);
            return -2;
        }
        if (orki_check_overlap(who, (uintptr_t)t[i].A, (uintptr_t)t[i].A + t[i].abytes, (uintptr_t)t[i].C,
                               (uintptr_t)t[i].C + t[i].cbytes))
            return -1;
    }

    orki_ptok pt;
    orki_prof_begin(c, &pt, 1);
    /* residency: device buffers are used in place, host operands go through one staging pass */
    size_t ha = 0, hc = 0, ws = 0;
    for (int i = 0; i < S; i++) {
        t[i].a_dev = orki_dev_find(c, t[i].A, t[i].abytes) && ((uintptr_t)t[i].A % 16 == 0);
        t[i].c_dev = orki_dev_find(c, t[i].C, t[i].cbytes);
        if (!t[i].a_dev) ha += al256(t[i].abytes);
        if (!t[i].c_dev) hc += al256((size_t)t[i].M * t[i].w->N * 4);
    }
    /* host A: gathered by the CPU into pinned staging, uploaded by one DMA copy; host C: written by the kernels
     * into pinned, device-mapped staging when it all fits ORKI_HOST_C_DIRECT (copied out by the CPU after the
     * sync), else into HBM staging brought back by strided D2H copies */
    char *sa = NULL, *ha_h = NULL, *sc = NULL, *hc_h = NULL;
    const int c_pinned = hc && hc <= ORKI_HOST_C_DIRECT;
    if (ha && (!(sa = orki_stage(c, &c->sA, ha)) || !(ha_h = orki_hstage(c, &c->hA, ha)))) { orki_hip_fail(who); return -1; }
    if (c_pinned) {
        if (!(hc_h = orki_hstage(c, &c->hC, hc)) || !(sc = orkh_host_devptr(hc_h))) { orki_hip_fail(who); return -1; }
    } else if (hc && !(sc = orki_stage(c, &c->sC, hc))) { orki_hip_fail(who); return -1; }
    size_t oa = 0, oc = 0;
    for (int i = 0; i < S; i++) {
        if (t[i].a_dev) t[i].dA = t[i].A;
        else {
            t[i].dA = sa + oa;
            memcpy(ha_h + oa, t[i].A, t[i].abytes);
            oa += al256(t[i].abytes);
        }
        if (t[i].c_dev) t[i].dC = t[i].C;
        else {
            t[i].dC = sc + oc;
            oc += al256((size_t)t[i].M * t[i].w->N * 4);
        }
    }
    if (ha && orkh_h2d(sa, ha_h, oa, c->stream)) { orki_hip_fail(who); return -1; }

    /* plans; split-K workspace shared by the individually launched tasks (stream-ordered) */
    orkh_plan *q = calloc((size_t)S, sizeof *q);
    if (!q) { orki_err("%s: out of memory", who); return -1; }
    for (int i = 0; i < S; i++) {
        size_t wsi = 0;
        orki_plan(c, t[i].w->rkind, t[i].M, t[i].w->K, t[i].w->N, t[i].w->KB, &q[i], &wsi);
        if (wsi > ws) ws = wsi;
    }
    void *dws = NULL;
    if (ws && !(dws = orki_ws_stage(c, ws, NULL))) { free(q); orki_hip_fail(who); return -1; }

    int rc = 0;
    char *done = calloc((size_t)S, 1);
    if (!done) { free(q); orki_err("%s: out of memory", who); return -1; }
    /* grouped launches: M = 1 GEMV tasks of one resident kind, in task order, ORKH_GROUP_MAX at a time. The grouped
     * kernel runs whole panels with one wave split per launch; integer sums are exact under any split, but an fp16
     * task joins only when its own plan has that same geometry (whole panels, the same waves and K-blocks per wave),
     * so that its fp32 sums run in the order of its single run. Others launch below with their own plans. */
    for (int i = 0; i < S && !rc; i++) {
        if (done[i] || q[i].algo != ORKH_ALGO_GEMV || q[i].ksplit != 1) continue;
        orkh_group g;
        memset(&g, 0, sizeof g);
        /* the grouped kernel runs whole panels: their wave count, whatever geometry the task's own plan has */
        const int wpg = orki_gemv_panel_wpg(c, t[i].w->rkind, t[i].w->KB, t[i].w->N / 16);
        if (t[i].w->rkind == ORKH_F16 && !f16_groupable(&q[i], t[i].w->KB, wpg)) continue;
        int wg = 0;
        for (int j = i; j < S && g.n < ORKH_GROUP_MAX; j++) {
            if (done[j] || q[j].algo != ORKH_ALGO_GEMV || q[j].ksplit != 1 || t[j].w->rkind != t[i].w->rkind) continue;
            if (t[j].w->rkind == ORKH_F16 && !f16_groupable(&q[j], t[j].w->KB, wpg)) continue;
            orkh_gtask *gt = &g.t[g.n++];
            gt->p.kind = t[j].w->rkind;
            gt->p.M = 1;
            gt->p.K = t[j].w->K;
            gt->p.N = t[j].w->N;
            gt->p.KB = t[j].w->KB;
            gt->p.A = t[j].dA;
            gt->p.lda = t[j].w->K;
            gt->p.B = t[j].w->dB;
            gt->p.C = t[j].dC;
            gt->p.ldc = t[j].c_dev ? t[j].ldc : t[j].w->N;
            memcpy(gt->p.lut, t[j].w->lut, sizeof gt->p.lut);
            gt->kbw = (t[j].w->KB + wpg - 1) / wpg;
            gt->wg0 = wg;
            wg += t[j].w->N / 16;
            done[j] = 1;
        }
        if (orkh_mm_launch_group(&g, wpg, c->stream)) { orki_hip_fail(who); rc = -1; }
    }
    /* grouped tiled launches: tasks of one integer resident kind, M > 1 and K whose columns together plan to the
     * LDS-ring kernel unsplit, ORKH_TGROUP_MAX at a time, under the tile planned for their summed N (integer results
     * are exact under any tile; fp16 tasks keep their own tiles, so each result still equals its single run) */
    for (int i = 0; i < S && !rc; i++) {
        if (done[i] || t[i].M == 1 || t[i].w->rkind == ORKH_F16) continue;
        int mem[ORKH_TGROUP_MAX], n = 0, nsum = 0;
        for (int j = i; j < S && n < ORKH_TGROUP_MAX; j++) {
            if (done[j] || t[j].M != t[i].M || t[j].w->rkind != t[i].w->rkind || t[j].w->K != t[i].w->K ||
                t[j].w->KB != t[i].w->KB)
                continue;
            mem[n++] = j;
            nsum += t[j].w->N;
        }
        if (n < 2) continue;
        orkh_plan gq;
        size_t gws = 0;
        orki_plan(c, t[i].w->rkind, t[i].M, t[i].w->K, nsum, t[i].w->KB, &gq, &gws);
        if (gq.algo != ORKH_ALGO_TILED2 || gq.ksplit > 1) continue;
        orkh_mm ps[ORKH_TGROUP_MAX];
        memset(ps, 0, sizeof ps);
        for (int k = 0; k < n; k++) {
            const ctask *tk = &t[mem[k]];
            ps[k].kind = tk->w->rkind;
            ps[k].M = tk->M;
            ps[k].K = tk->w->K;
            ps[k].N = tk->w->N;
            ps[k].KB = tk->w->KB;
            ps[k].A = tk->dA;
            ps[k].lda = tk->w->K;
            ps[k].B = tk->w->dB;
            ps[k].C = tk->dC;
            ps[k].ldc = tk->c_dev ? tk->ldc : tk->w->N;
            memcpy(ps[k].lut, tk->w->lut, sizeof ps[k].lut);
        }
        if (orkh_mm_launch_tgroup(ps, n, &gq, c->stream)) { orki_hip_fail(who); rc = -1; }
        for (int k = 0; k < n; k++) done[mem[k]] = 1;
    }
    for (int i = 0; i < S && !rc; i++) {
        if (done[i]) continue;
        orkh_mm p;
        memset(&p, 0, sizeof p);
        p.kind = t[i].w->rkind;
        p.M = t[i].M;
        p.K = t[i].w->K;
        p.N = t[i].w->N;
        p.KB = t[i].w->KB;
        p.A = t[i].dA;
        p.lda = t[i].w->K;
        p.B = t[i].w->dB;
        p.C = t[i].dC;
        p.ldc = t[i].c_dev ? t[i].ldc : t[i].w->N;
        memcpy(p.lut, t[i].w->lut, sizeof p.lut);
        q[i].ws = dws;
        if (orkh_mm_launch(&p, &q[i], c->stream)) { orki_hip_fail(who); rc = -1; }
    }
    free(done);
    free(q);
    if (rc) return rc;

    int all_dev = 1;
    for (int i = 0; i < S; i++) {
        if (t[i].c_dev) continue;
        all_dev = 0;
        const size_t row = (size_t)t[i].w->N * 4;
        if (!c_pinned && orkh_d2h_2d(t[i].C, (size_t)t[i].ldc * 4, t[i].dC, row, row, (size_t)t[i].M, c->stream)) {
            orki_hip_fail(who);
            return -1;
        }
    }
    for (int i = 0; i < S; i++) all_dev &= t[i].a_dev;
    orki_prof_launched(c, &pt);
    char pname[32];
    snprintf(pname, sizeof pname, "%d tasks", S);
    if (c->async && all_dev && !(ws && c->ws_guard)) {
        orki_prof_end(c, &pt, who, pname);
        return 0;
    }
    if (orkh_sync(c->stream)) { orki_hip_fail(who); return -1; }
    if (ws && orki_ws_check(c, dws, ws, who)) return -1;
    size_t o = 0;
    if (c_pinned)
        for (int i = 0; i < S; i++) {
            if (t[i].c_dev) continue;
            const size_t row = (size_t)t[i].w->N * 4;
            for (int m = 0; m < t[i].M; m++)
                memcpy((char *)t[i].C + (size_t)m * t[i].ldc * 4, hc_h + o + (size_t)m * row, row);
            o += al256((size_t)t[i].M * row);
        }
    orki_prof_end(c, &pt, who, pname);
    orki_prof_settle(c);
    return 0;
}

static ctask *tasks_new(int S) { return calloc((size_t)S, sizeof(ctask)); }

/* OFFLINE chain (src/npu/core/buf.c:483-487, :560-564): each task exactly on the CPU, in task order, from the
 * weight's host codes; -1 if a task's weight is not an offline one. As the reference's CPU chain, C is written
 * with row stride N (an int8 task's cstride applies on the device only). */
static int cpu_chain(int S, const void *tasks, size_t tsz) {
    /* ork_mm_task_i8 begins with the four fields of ork_mm_task_i4 (w, M, A, C), in the same order */
    if (S < 1) return 0; /* the reference's task loop runs nothing */
    if (!tasks) return -2;
    for (int i = 0; i < S; i++) {
        const ork_mm_task_i4 *t = (const ork_mm_task_i4 *)((const char *)tasks + (size_t)i * tsz);
        if (!t->w || !t->w->codes) return -1;
        if (t->M > 0) ork_i8_mm_run_cpu(t->M, t->w->K, t->w->N, t->A, t->w->codes, t->C);
    }
    return 0;
}

static int i8_chain(const char *who, ork_npu *c, int S, const ork_mm_task_i8 *tasks) {
    if (!c) return -1;
    if (S < 1 || S > 1024 || !tasks) return -2;
    ctask *t = tasks_new(S);
    if (!t) return -1;
    for (int i = 0; i < S; i++) {
        t[i].w = tasks[i].w;
        t[i].M = tasks[i].M;
        t[i].A = tasks[i].A;
        t[i].C = tasks[i].C;
        t[i].ldc = tasks[i].cstride > 0 ? tasks[i].cstride : (tasks[i].w ? tasks[i].w->N : 0);
    }
    const int rc = chain_common(who, c, S, t, DT_I8, 1);
    free(t);
    return rc;
}

static int i4_chain(const char *who, ork_npu *c, int S, const ork_mm_task_i4 *tasks) {
    if (!c) return -1;
    if (S < 1 || S > 1024 || !tasks) return -2;
    ctask *t = tasks_new(S);
    if (!t) return -1;
    for (int i = 0; i < S; i++) {
        t[i].w = tasks[i].w;
        t[i].M = tasks[i].M;
        t[i].A = tasks[i].A;
        t[i].C = tasks[i].C;
        t[i].ldc = tasks[i].w ? tasks[i].w->N : 0;
    }
    const int rc = chain_common(who, c, S, t, DT_I4, 1);
    free(t);
    return rc;
}

int ork_i8_mm_run_chain(ork_npu *c, int S, const ork_mm_task_i8 *tasks) {
    if (c && c->offline) return cpu_chain(S, tasks, sizeof *tasks);
    return i8_chain("ork_i8_mm_run_chain", c, S, tasks);
}

int ork_i8_mm_run_stream(ork_npu *c, int S, const ork_mm_task_i8 *tasks) {
    if (!c) return -2; /* src/npu/i8/run.c:713 */
    return i8_chain("ork_i8_mm_run_stream", c, S, tasks);
}

int ork_i4_mm_run_chain(ork_npu *c, int S, const ork_mm_task_i4 *tasks) {
    if (c && c->offline) return cpu_chain(S, tasks, sizeof *tasks);
    return i4_chain("ork_i4_mm_run_chain", c, S, tasks);
}

int ork_i4_mm_run_stream(ork_npu *c, int S, const ork_mm_task_i4 *tasks) {
    if (c && c->offline) return cpu_chain(S, tasks, sizeof *tasks);
    if (!c) return -2;
    return i4_chain("ork_i4_mm_run_stream", c, S, tasks);
}

int ork_f16_mm_run_stream(ork_npu *c, int S, const ork_mm_task_f16 *tasks) {
    if (!c || S < 1 || S > 1024 || !tasks) return -2;
    ctask *t = tasks_new(S);
    if (!t) return -1;
    for (int i = 0; i < S; i++) {
        t[i].w = tasks[i].w;
        t[i].M = tasks[i].M;
        t[i].A = tasks[i].A;
        t[i].C = tasks[i].C;
        t[i].ldc = tasks[i].w ? tasks[i].w->N : 0;
    }
    const int rc = chain_common("ork_f16_mm_run_stream", c, S, t, DT_F16, 2);
    free(t);
    return rc;
}
