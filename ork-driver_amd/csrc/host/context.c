/* context.c -- context lifecycle, buffer registries, diagnostics, worker pool.
 *
 * Reference roles: ork_npu_init / ork_npu_init_offline (src/npu/core/sched.c:41-117, :137-145),
 * ork_npu_free (src/npu/core/device.c:239-300), introspection (src/npu/core/device.c:315-321, :377-385),
 * ork_dma_alloc / ork_dma_free / orki_dma_find (src/npu/core/buf.c:271-280, :298), ork_parallel_for
 * (src/npu/core/sched.c:192). On MI355X the context opens one HIP device, creates one in-order stream
 * and owns every device allocation made through it. */
#define _GNU_SOURCE
#include <stdarg.h>
#include <stdatomic.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include "internal.h"

static atomic_long g_io_fail;

void orki_err(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    fputs("[ork] ", stderr);
    vfprintf(stderr, fmt, ap);
    fputc('\n', stderr);
    va_end(ap);
}

void orki_hip_fail(const char *what) {
    atomic_fetch_add(&g_io_fail, 1);
    const char *le = orkh_launch_error();
    if (le && le[0]) orki_err("HIP failure in %s: %s", what, le);
    else orki_err("HIP failure in %s: %s", what, orkh_last_error());
}

long ork_io_failures(void) { return atomic_load(&g_io_fail); }
/* reference include/ork/context.h:149, src/npu/core/submit.c:74: failures a recovery path provokes on purpose.
 * No path of this build provokes one, so the count stays 0. */
long ork_io_expected_failures(void) { return 0; }

const char *ork_npu_version(void) { return ORK_NPU_VERSION "+mi355x"; }
uint32_t ork_pack_format_version(void) { return ORK_PACK_FORMAT_VERSION; }

/* ---- worker pool ------------------------------------------------------------------------------ */
struct pf_job { void (*fn)(int, int, void *); void *arg; int lo, hi; };
static void *pf_run(void *p) {
    struct pf_job *j = p;
    j->fn(j->lo, j->hi, j->arg);
    return NULL;
}

void orki_parallel_for(int n, void (*fn)(int lo, int hi, void *arg), void *arg) {
    if (n <= 0) return;
    long nc = sysconf(_SC_NPROCESSORS_ONLN);
    const char *e = getenv("ORK_PACK_THREADS");
    if (e && atoi(e) > 0) nc = atoi(e);
    int nt = (int)(nc < 1 ? 1 : nc > 64 ? 64 : nc);
    if (nt > n) nt = n;
    if (nt <= 1) { fn(0, n, arg); return; }
    pthread_t th[64];
    struct pf_job jobs[64];
    int joined[64] = {0};
    for (int t = 0; t < nt; t++) {
        jobs[t] = (struct pf_job){fn, arg, (int)((long)n * t / nt), (int)((long)n * (t + 1) / nt)};
        if (t == 0) continue;
        if (pthread_create(&th[t], NULL, pf_run, &jobs[t]) == 0) joined[t] = 1;
        else fn(jobs[t].lo, jobs[t].hi, arg); /* no thread: run the chunk here */
    }
    fn(jobs[0].lo, jobs[0].hi, arg);
    for (int t = 1; t < nt; t++)
        if (joined[t]) pthread_join(th[t], NULL);
}

/* ---- lifecycle --------------------------------------------------------------------------------- */
static ork_npu *ctx_new(void) {
    ork_npu *c = calloc(1, sizeof *c);
    if (!c) return NULL;
    pthread_mutex_init(&c->mu, NULL);
    const char *dbg = getenv("ORK_PLAN_DEBUG");
    c->plan_knobs = dbg && *dbg && strcmp(dbg, "0") != 0;
    const char *gd = getenv("ORK_WS_GUARD");
    c->ws_guard = c->plan_knobs && gd && *gd && strcmp(gd, "0") != 0;
    return c;
}

ork_npu *ork_npu_init(void) {
    if (orkh_device_count() < 1) {
        orki_err("ork_npu_init: no HIP device visible");
        return NULL;
    }
    int ord = 0;
    const char *e = getenv("ORK_HIP_DEVICE");
    if (e) ord = atoi(e);
    ork_npu *c = ctx_new();
    if (!c) return NULL;
    if (orkh_init(ord, &c->dev, &c->stream) != 0) {
        orki_err("ork_npu_init: %s", orkh_last_error());
        pthread_mutex_destroy(&c->mu);
        free(c);
        return NULL;
    }
    /* "gfx950:sramecc+:xnack-" -> "gfx950" */
    size_t i = 0;
    while (c->dev.arch[i] && c->dev.arch[i] != ':' && i + 1 < sizeof c->soc) { c->soc[i] = c->dev.arch[i]; i++; }
    c->soc[i] = 0;
    c->cores = c->dev.cu_count;
    c->core_budget = c->cores;
    orki_prof_init(c);
    if (strcmp(c->soc, "gfx950") != 0)
        orki_err("ork_npu_init: device is %s, kernels are built for gfx950 only", c->soc);
    return c;
}

ork_npu *ork_npu_init_offline(const char *soc_id) {
    static const struct { const char *id; int cores; } known[] = {
        {"gfx950", 256}, {"mi355x", 256}, {"rk3588", 3}, {"rk3576", 2}};
    int hit = -1;
    for (int i = 0; soc_id && i < (int)(sizeof known / sizeof known[0]); i++)
        if (!strcmp(soc_id, known[i].id)) hit = i;
    if (hit < 0) {
        orki_err("ERROR: ork_npu_init_offline: unknown SoC id \"%s\"", soc_id ? soc_id : "(null)");
        return NULL;
    }
    ork_npu *c = ctx_new();
    if (!c) return NULL;
    c->offline = 1;
    snprintf(c->soc, sizeof c->soc, "%s", known[hit].id);
    c->cores = known[hit].cores;
    c->core_budget = c->cores;
    orki_prof_init(c);
    return c;
}

void ork_npu_free(ork_npu *c) {
    if (!c) return;
    orki_prof_dump(c);
    if (!c->offline) {
        if (c->stream) (void)orkh_sync(c->stream);
        orkh_free(c->sA.p);
        orkh_free(c->sC.p);
        orkh_free(c->sW.p);
        orkh_free(c->sS.p);
        orkh_host_free(c->hA.p);
        orkh_host_free(c->hC.p);
        for (int i = 0; i < c->dma_n; i++) orkh_host_free(c->dma[i].p);
        for (int i = 0; i < c->devb_n; i++) orkh_free(c->devb[i].p);
        for (int i = 0; i < c->orphan_n; i++) orkh_free(c->orphan[i]);
        orkh_stream_destroy(c->stream);
    }
    free(c->devb);
    free(c->orphan);
    pthread_mutex_destroy(&c->mu);
    free(c);
}

const char *ork_npu_soc(const ork_npu *c) { return c ? c->soc : NULL; }
const char *ork_npu_soc_id(ork_npu *c) { return c ? c->soc : NULL; }
int ork_npu_cores(const ork_npu *c) { return c ? c->cores : 0; }
int ork_npu_validated(const ork_npu *c) { return c && !strcmp(c->soc, "gfx950"); }
void ork_npu_set_core_budget(ork_npu *c, int n) {
    if (!c) return;
    c->core_budget = (n > 0 && n <= c->cores) ? n : c->cores;
}

int orki_need_device(const ork_npu *c, const char *who) {
    if (!c) { orki_err("%s: NULL context", who); return -1; }
    if (c->offline) {
        orki_err("%s: offline context has no device (this build has no CPU fallback)", who);
        return -1;
    }
    return 0;
}

/* ---- staging / registries ---------------------------------------------------------------------- */
void *orki_stage(ork_npu *c, struct ork_buf *b, size_t n) {
    if (b->n >= n && b->p) return b->p;
    size_t want = n < 65536 ? 65536 : n;
    want = (want + 4095) & ~(size_t)4095;
    if (b->p) {
        if (orkh_sync(c->stream) != 0) orki_hip_fail("stage sync");
        orkh_free(b->p);
    }
    b->p = orkh_malloc(want);
    b->n = b->p ? want : 0;
    if (!b->p) orki_hip_fail("staging alloc");
    return b->p;
}

/* The guard pattern: a byte sequence no kernel's partials produce by accident in a whole band. */
static unsigned char g_guard_pat[ORKI_WS_GUARD];
static pthread_once_t g_guard_once = PTHREAD_ONCE_INIT;
static void guard_pat_init(void) {
    for (int i = 0; i < ORKI_WS_GUARD; i++) g_guard_pat[i] = (unsigned char)(0xA5 ^ (i * 31) ^ (i >> 8));
}

void *orki_ws_stage(ork_npu *c, size_t ws, void *fixed) {
    if (!c->ws_guard) return fixed ? fixed : orki_stage(c, &c->sW, ws);
    pthread_once(&g_guard_once, guard_pat_init);
    char *base = fixed ? fixed : orki_stage(c, &c->sW, ws + 2 * ORKI_WS_GUARD);
    if (!base) return NULL;
    if (orkh_h2d(base, g_guard_pat, ORKI_WS_GUARD, c->stream) ||
        orkh_h2d(base + ORKI_WS_GUARD + ws, g_guard_pat, ORKI_WS_GUARD, c->stream))
        return NULL;
    return base + ORKI_WS_GUARD;
}

int orki_ws_check(ork_npu *c, const void *ws_base, size_t ws, const char *who) {
    if (!c->ws_guard || !ws_base) return 0;
    unsigned char got[2][ORKI_WS_GUARD];
    const char *b = ws_base;
    if (orkh_d2h(got[0], b - ORKI_WS_GUARD, ORKI_WS_GUARD, c->stream) ||
        orkh_d2h(got[1], b + ws, ORKI_WS_GUARD, c->stream) || orkh_sync(c->stream)) {
        orki_hip_fail(who);
        return -1;
    }
    for (int s = 0; s < 2; s++)
        for (int i = 0; i < ORKI_WS_GUARD; i++)
            if (got[s][i] != g_guard_pat[i]) {
                orki_err("%s: split-K partials overran their workspace: guard byte %s%d changed", who,
                         s ? "+" : "-", s ? i : ORKI_WS_GUARD - i);
                return -1;
            }
    return 0;
}

/* Pinned, device-mapped host staging, grown on demand like orki_stage. */
void *orki_hstage(ork_npu *c, struct ork_buf *b, size_t n) {
    if (b->n >= n && b->p) return b->p;
    size_t want = n < 65536 ? 65536 : n;
    want = (want + 4095) & ~(size_t)4095;
    if (b->p) {
        if (orkh_sync(c->stream) != 0) orki_hip_fail("stage sync");
        orkh_host_free(b->p);
    }
    b->p = orkh_host_alloc(want);
    b->n = b->p ? want : 0;
    if (!b->p) orki_hip_fail("pinned staging alloc");
    return b->p;
}

/* The [p, p+n) span inside one ork_dma_alloc buffer: its base, or NULL. */
static const struct ork_buf *dma_span(ork_npu *c, const void *p, size_t n) {
    for (int i = 0; i < c->dma_n; i++) {
        const char *b = c->dma[i].p;
        if ((const char *)p >= b && (const char *)p + n <= b + c->dma[i].n) return &c->dma[i];
    }
    return NULL;
}

/* A pageable host A would be staged a second time inside the runtime's copy, which also blocks the caller; one
 * CPU memcpy into pinned staging makes the upload a plain DMA on the stream. An A inside an ork_dma_alloc
 * buffer is already pinned. The staging is reused by the next run: every run with a host A syncs its stream
 * before returning, so no upload from it is still pending then. */
const void *orki_host_a(ork_npu *c, const void *A, size_t n) {
    void *s = orki_stage(c, &c->sA, n);
    if (!s) return NULL;
    const void *src = A;
    if (!dma_span(c, A, n)) {
        void *h = orki_hstage(c, &c->hA, n);
        if (!h) return NULL;
        memcpy(h, A, n);
        src = h;
    }
    return orkh_h2d(s, src, n, c->stream) ? NULL : s;
}

/* Where the kernels write a host C:
 *   ORKI_C_INPLACE  C lies in an ork_dma_alloc buffer (pinned, device-mapped): written in place;
 *   ORKI_C_PINNED   up to ORKI_HOST_C_DIRECT bytes: written across PCIe into pinned staging, copied to C by
 *                   the CPU after the sync -- no device-to-host copy command and its completion round trip;
 *   ORKI_C_HBM      larger: HBM staging, brought back by one D2H copy on the stream. */
void *orki_host_c(ork_npu *c, void *C, size_t n, int *mode) {
    const struct ork_buf *d = dma_span(c, C, n);
    if (d) {
        char *base = orkh_host_devptr(d->p);
        *mode = ORKI_C_INPLACE;
        return base ? base + ((char *)C - (char *)d->p) : NULL;
    }
    if (n <= ORKI_HOST_C_DIRECT) {
        void *h = orki_hstage(c, &c->hC, n);
        *mode = ORKI_C_PINNED;
        return h ? orkh_host_devptr(h) : NULL;
    }
    *mode = ORKI_C_HBM;
    return orki_stage(c, &c->sC, n);
}

int orki_host_c_post(ork_npu *c, void *C, const void *dC, size_t n, int mode) {
    return mode == ORKI_C_HBM ? orkh_d2h(C, dC, n, c->stream) : 0;
}

void orki_host_c_done(ork_npu *c, void *C, size_t n, int mode) {
    if (mode == ORKI_C_PINNED) memcpy(C, c->hC.p, n);
}

void *ork_dma_alloc(ork_npu *c, size_t size) {
    if (!c || c->offline || !size) return NULL;
    pthread_mutex_lock(&c->mu);
    void *p = NULL;
    if (c->dma_n < ORK_DMA_MAX) {
        p = orkh_host_alloc(size);
        if (p) c->dma[c->dma_n++] = (struct ork_buf){p, size};
        else orki_hip_fail("ork_dma_alloc");
    }
    pthread_mutex_unlock(&c->mu);
    return p;
}

void ork_dma_free(ork_npu *c, void *ptr) {
    if (!c || !ptr) return;
    pthread_mutex_lock(&c->mu);
    for (int i = 0; i < c->dma_n; i++)
        if (c->dma[i].p == ptr) {
            (void)orkh_sync(c->stream);
            orkh_host_free(ptr);
            c->dma[i] = c->dma[--c->dma_n];
            break;
        }
    pthread_mutex_unlock(&c->mu);
}

int orki_dma_find(ork_npu *c, const void *p) {
    for (int i = 0; i < c->dma_n; i++) {
        const char *b = c->dma[i].p;
        if ((const char *)p >= b && (const char *)p < b + c->dma[i].n) return 1;
    }
    return 0;
}

void *ork_dev_alloc(ork_npu *c, size_t size) {
    if (!c || c->offline || !size) return NULL;
    void *p = orkh_malloc(size);
    if (!p) { orki_hip_fail("ork_dev_alloc"); return NULL; }
    pthread_mutex_lock(&c->mu);
    if (c->devb_n == c->devb_cap) {
        int nc = c->devb_cap ? 2 * c->devb_cap : 16;
        struct ork_buf *nb = realloc(c->devb, (size_t)nc * sizeof *nb);
        if (!nb) { pthread_mutex_unlock(&c->mu); orkh_free(p); return NULL; }
        c->devb = nb;
        c->devb_cap = nc;
    }
    c->devb[c->devb_n++] = (struct ork_buf){p, size};
    pthread_mutex_unlock(&c->mu);
    return p;
}

void ork_dev_free(ork_npu *c, void *ptr) {
    if (!c || !ptr) return;
    pthread_mutex_lock(&c->mu);
    for (int i = 0; i < c->devb_n; i++)
        if (c->devb[i].p == ptr) {
            (void)orkh_sync(c->stream);
            orkh_free(ptr);
            c->devb[i] = c->devb[--c->devb_n];
            break;
        }
    pthread_mutex_unlock(&c->mu);
}

int orki_dev_find(ork_npu *c, const void *p, size_t n) {
    for (int i = 0; i < c->devb_n; i++) {
        const char *b = c->devb[i].p;
        if ((const char *)p >= b && (const char *)p + n <= b + c->devb[i].n) return 1;
    }
    return 0;
}

int ork_dev_upload(ork_npu *c, void *dst, const void *src, size_t n) {
    if (orki_need_device(c, "ork_dev_upload")) return -1;
    if (orkh_h2d(dst, src, n, c->stream) || orkh_sync(c->stream)) { orki_hip_fail("ork_dev_upload"); return -1; }
    return 0;
}

int ork_npu_mark(ork_npu *c, void *dev_u64) {
    if (orki_need_device(c, "ork_npu_mark")) return -1;
    if (orkh_mark(dev_u64, c->stream)) { orki_err("ork_npu_mark: %s", orkh_last_error()); return -1; }
    return 0;
}

int ork_npu_wallclock_khz(const ork_npu *c) { return (c && !c->offline) ? c->dev.wall_khz : 0; }

long long ork_npu_read_probe(ork_npu *c, const void *dev, size_t bytes, uint32_t *dev_sink) {
    if (orki_need_device(c, "ork_npu_read_probe")) return -1;
    if (!orkh_ptr_is_device(dev) || !orkh_ptr_is_device(dev_sink)) {
        orki_err("ork_npu_read_probe: the bytes and the sink must be device memory");
        return -1;
    }
    const long long n = orkh_read_probe(dev, bytes, dev_sink, c->stream);
    if (n < 0) { orki_err("ork_npu_read_probe: %s", orkh_last_error()); return -1; }
    if (!c->async && orkh_sync(c->stream)) { orki_hip_fail("ork_npu_read_probe"); return -1; }
    return n;
}

int ork_dev_download(ork_npu *c, void *dst, const void *src, size_t n) {
    if (orki_need_device(c, "ork_dev_download")) return -1;
    if (orkh_d2h(dst, src, n, c->stream) || orkh_sync(c->stream)) { orki_hip_fail("ork_dev_download"); return -1; }
    return 0;
}

void ork_npu_set_async(ork_npu *c, int on) { if (c) c->async = on ? 1 : 0; }

int ork_npu_sync(ork_npu *c) {
    if (orki_need_device(c, "ork_npu_sync")) return -1;
    if (orkh_sync(c->stream)) { orki_hip_fail("ork_npu_sync"); return -1; }
    orki_prof_settle(c);
    return 0;
}

void *ork_npu_stream(ork_npu *c) { return (c && !c->offline) ? c->stream : NULL; }

void orki_orphan(ork_npu *c, void *dptr) {
    if (!c || !dptr) return;
    pthread_mutex_lock(&c->mu);
    if (c->orphan_n == c->orphan_cap) {
        int nc = c->orphan_cap ? 2 * c->orphan_cap : 16;
        void **no = realloc(c->orphan, (size_t)nc * sizeof *no);
        if (!no) { pthread_mutex_unlock(&c->mu); (void)orkh_sync(c->stream); orkh_free(dptr); return; }
        c->orphan = no;
        c->orphan_cap = nc;
    }
    c->orphan[c->orphan_n++] = dptr;
    pthread_mutex_unlock(&c->mu);
}
