/* prof.c -- ORK_PROFILE: per-call timing of the run entry points, printed when the context is freed.
 *
 * Reference: ORK_PROFILE is read when the context is made (src/npu/core/sched.c:53); the int8 and int4 runs count
 * their calls and host wall time (src/npu.c:82-91) and ork_npu_free prints "[ork PROFILE] run_i8: N calls, T ms
 * total, U us/call" with the submit-ioctl counts (src/npu/core/device.c:257-263). Kept: the switch, the moment
 * of printing, the prefix, calls and host wall time per call. What changes: one row per (entry point, kernel
 * plan) instead of per dtype, and in place of the ioctl split the device time of each call's launches, taken by
 * two HIP events on the context's stream around them (none while the stream is being captured into a graph,
 * where events do not time; none for ork_i8_mm_run_noalloc, which makes no runtime objects). Event pairs are
 * read back once the stream has been synchronised, so an async run is not made to wait. */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "internal.h"

#define PROF_ROWS 64
#define PROF_PEND 256 /* event pairs in flight (async runs) before the oldest is waited for */

struct prof_row {
    const char *who;
    char plan[64];
    long calls, dev_n;
    double host_us, dev_us;
};

struct orki_prof {
    struct prof_row row[PROF_ROWS];
    int nrow;
    void *ev[2 * PROF_PEND]; /* created on first use */
    int pend_row[PROF_PEND]; /* row of each pending pair, -1 = free */
    int head, npend;         /* ring of pending pairs, oldest at head */
};

static double now_us(void) {
    struct timespec t;
    clock_gettime(CLOCK_MONOTONIC, &t);
    return (double)t.tv_sec * 1e6 + (double)t.tv_nsec * 1e-3;
}

void orki_prof_init(ork_npu *c) {
    if (!getenv("ORK_PROFILE")) return;
    c->prof = calloc(1, sizeof *c->prof);
    if (!c->prof) orki_err("ORK_PROFILE: out of memory, profiling off");
}

static int row_of(struct orki_prof *p, const char *who, const char *plan) {
    for (int i = 0; i < p->nrow; i++)
        if (p->row[i].who == who && !strcmp(p->row[i].plan, plan)) return i;
    if (p->nrow == PROF_ROWS) return PROF_ROWS - 1; /* the last row absorbs the overflow */
    struct prof_row *r = &p->row[p->nrow];
    r->who = who;
    snprintf(r->plan, sizeof r->plan, "%s", plan);
    return p->nrow++;
}

/* Read back the oldest pending pair (waits for it when the stream has not reached it yet). */
static void settle_one(struct orki_prof *p) {
    const int k = p->head;
    const float ms = orkh_event_ms(p->ev[2 * k], p->ev[2 * k + 1]);
    if (ms >= 0.f && p->pend_row[k] >= 0) {
        p->row[p->pend_row[k]].dev_us += 1e3 * ms;
        p->row[p->pend_row[k]].dev_n++;
    }
    p->pend_row[k] = -1;
    p->head = (p->head + 1) % PROF_PEND;
    p->npend--;
}

void orki_prof_settle(ork_npu *c) {
    if (!c || !c->prof) return;
    while (c->prof->npend) settle_one(c->prof);
}

void orki_prof_begin(ork_npu *c, orki_ptok *t, int device) {
    t->t0 = 0;
    t->pair = -1;
    if (!c->prof) return;
    t->t0 = now_us();
    struct orki_prof *p = c->prof;
    if (!device || c->offline || orkh_stream_capturing(c->stream) != 0) return;
    if (!p->ev[0]) {
        for (int i = 0; i < 2 * PROF_PEND; i++)
            if (!(p->ev[i] = orkh_event_new())) return;
        for (int i = 0; i < PROF_PEND; i++) p->pend_row[i] = -1;
    }
    if (p->npend == PROF_PEND) settle_one(p);
    const int k = (p->head + p->npend) % PROF_PEND;
    if (orkh_event_record(p->ev[2 * k], c->stream)) return;
    t->pair = k;
}

void orki_prof_launched(ork_npu *c, orki_ptok *t) {
    if (!c->prof || t->pair < 0) return;
    if (orkh_event_record(c->prof->ev[2 * t->pair + 1], c->stream)) t->pair = -1;
}

void orki_prof_end(ork_npu *c, orki_ptok *t, const char *who, const char *plan) {
    if (!c->prof) return;
    struct orki_prof *p = c->prof;
    const int r = row_of(p, who, plan ? plan : "");
    p->row[r].calls++;
    p->row[r].host_us += now_us() - t->t0;
    if (t->pair >= 0) {
        p->pend_row[t->pair] = r;
        p->npend++;
    }
}

void orki_prof_dump(ork_npu *c) {
    struct orki_prof *p = c ? c->prof : NULL;
    if (!p) return;
    if (!c->offline && c->stream) (void)orkh_sync(c->stream);
    orki_prof_settle(c);
    for (int i = 0; i < p->nrow; i++) {
        const struct prof_row *r = &p->row[i];
        if (r->dev_n)
            fprintf(stderr, "[ork PROFILE] %s %s: %ld calls, %.3f ms total, %.2f us/call; device %.2f us/call over %ld\n",
                    r->who, r->plan, r->calls, r->host_us / 1e3, r->host_us / r->calls, r->dev_us / r->dev_n, r->dev_n);
        else
            fprintf(stderr, "[ork PROFILE] %s %s: %ld calls, %.3f ms total, %.2f us/call\n", r->who, r->plan, r->calls,
                    r->host_us / 1e3, r->host_us / r->calls);
    }
    for (int i = 0; i < 2 * PROF_PEND; i++) orkh_event_free(p->ev[i]);
    free(p);
    c->prof = NULL;
}
