/* plan.c -- the MI355X matmul planner: which kernel, what grid, how K is split.
 *
 * Replaces the reference's K-split / N-tile / M-tile / core-count policy (orki_int8_ks, orki_budget,
 * orki_run_loop_chunk, the mg_max*64 M-tile: src/npu.c:131-160, :1598-1610, :1693-1694;
 * orki_f16_ks, src/npu/f16/regcmd.c:120-125). The NPU needed K cut into 1024-wide slices, N into
 * 8192-wide outputs and M into CBUF-sized row groups, each a separate submit with a host int32
 * accumulate. On MI355X every shape is one launch (plus a reduce pass when K is split across
 * workgroups); the planner only decides how to fill 256 CUs:
 *   M <= 64  stream: one 16-column panel per workgroup, waves split K in runs of 1 KiB blocks (8 per
 *            run for the int8/fp16 GEMV); K is split across workgroups only for long-K, few-panel
 *            shapes that leave the machine underfilled. ORK_KSPLIT=n forces a split (tests).
 *   M >  64  tiled: the BM x BN tile (128x96, 128x128 or 64x64) and K split with the least modelled
 *            time (operand bytes per workgroup-round, plus partials and a reduce launch when split). */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "internal.h"

static int cdiv(int a, int b) { return (a + b - 1) / b; }

int orki_plan(const ork_npu *c, int rkind, int M, int K, int N, int KB, orkh_plan *q, size_t *ws_bytes) {
    (void)K;
    memset(q, 0, sizeof *q);
    *ws_bytes = 0;
    const int cu = (c && c->cores > 0) ? c->cores : 256;
    const int NB = N / 16;
    int stream = M <= 64;
    const char *force = getenv("ORK_PLAN");
    if (force && !strcmp(force, "tiled")) stream = 0;
    if (force && !strcmp(force, "stream") && M <= 64) stream = 1;

    if (stream) {
        /* M = 1 takes the VALU-dot GEMV (same grid and fields); ORK_PLAN=stream keeps the MFMA kernel. */
        q->algo = (M == 1 && !(force && !strcmp(force, "stream"))) ? ORKH_ALGO_GEMV : ORKH_ALGO_STREAM;
        q->mt = cdiv(M, 16);
        /* Run length per wave: 8 KiB in flight per wave for the int8/fp16 GEMV (M = 1); more waves with
         * shorter runs where each block costs more issue (more rows, int4 decode). Measured on the
         * K=2048, N=6144 panels; the run lengths on either side were within 2-4%. */
        const int kbw_target = (rkind == ORKH_I4U || rkind == ORKH_NF4) ? 2 : (M > 1 ? 4 : 8);
        const int need = cdiv(KB, kbw_target); /* waves per panel at the target run length */
        const int wpg = need <= 4 ? 4 : 8;
        /* K is split across workgroups only when the panels leave the machine underfilled (< 4 waves
         * per CU) AND each wave would otherwise stream more than two runs back to back: the split
         * costs a second launch (the fixed-order reduce, ~2 us), which a one-run wave never repays. */
        int ksplit = 1;
        const int runs = cdiv(cdiv(KB, wpg), kbw_target);
        if ((long)NB * wpg < 4L * cu && runs > 2) {
            ksplit = cdiv(4 * cu, NB * wpg);
            if (ksplit > runs) ksplit = runs; /* every wave keeps a full run */
        }
        const char *fks = getenv("ORK_KSPLIT");
        if (fks && atoi(fks) > 0) ksplit = atoi(fks);
        if (ksplit > KB) ksplit = KB;
        if (ksplit < 1) ksplit = 1;
        const int kbs = cdiv(KB, ksplit);
        ksplit = cdiv(KB, kbs);
        q->wpg = wpg;
        q->kbs = kbs;
        q->kbw = cdiv(kbs, wpg);
        q->ksplit = ksplit;
        if (ksplit > 1) *ws_bytes = (size_t)ksplit * M * N * 4;
        return 0;
    }

    const char *tf = getenv("ORK_TILE"); /* testing / A-B: "BMxBN" forces that tile of the LDS-ring kernel */
    int fbm, fbn;
    if (tf && sscanf(tf, "%dx%d", &fbm, &fbn) == 2) {
        const char *fks2 = getenv("ORK_KSPLIT");
        int ks = fks2 ? atoi(fks2) : 1;
        if (ks < 1) ks = 1;
        if (ks > KB) ks = KB;
        q->algo = ORKH_ALGO_TILED2;
        q->bm = fbm;
        q->bn = fbn;
        q->kbs = cdiv(KB, ks);
        q->ksplit = cdiv(KB, q->kbs);
        if (q->ksplit > 1) *ws_bytes = (size_t)q->ksplit * M * N * 4;
        return 0;
    }
    const char *fks = getenv("ORK_KSPLIT");
    int ks_force = fks ? atoi(fks) : 0;
    if (ks_force > 0) ks_force = cdiv(KB, cdiv(KB, ks_force < KB ? ks_force : KB)); /* as a split can realise it */
    double best = -1;

    /* The LDS-ring kernel (k_tiled2) for int8, fp16 and uniform int4. Each workgroup is bound by how fast its
     * operand tiles reach the CU (measured ~15 B/clk per CU, i.e. ~0.027 us per KiB) plus ~1.5 us of
     * set-up, so a round of workgroups costs about 1.5 + 0.027 * (A + B + C KiB of one workgroup) us.
     * Measured on K=2048..6144, M=128..4096 int8 / fp16 / W4A4 shapes to within ~15%. A K split adds
     * the partials' round trip and the reduce launch (~3 us + 2 * ks * M * N * 4 B at 4 TB/s).
     * NF4 keeps k_tiled: four waves share each decoded B block here, and the codebook decode is not
     * cheap enough to repeat. */
    if (rkind != ORKH_NF4 && !(force && !strcmp(force, "tiled"))) {
        static const int cfg2[][2] = {{256, 256}, {128, 128}, {64, 192}, {64, 64}};
        const int kpb = rkind == ORKH_I8 ? 64 : rkind == ORKH_F16 ? 32 : 128;
        const int abpk = rkind == ORKH_F16 ? 2 * kpb : kpb; /* A bytes per row per K-block */
        for (int i = 0; i < 4; i++) {
            const int bm = cfg2[i][0], bn = cfg2[i][1];
            const long tiles = (long)cdiv(M, bm) * cdiv(NB, bn / 16);
            for (int ks = ks_force > 0 ? ks_force : 1; ks <= (ks_force > 0 ? ks_force : 8); ks *= (ks_force > 0 ? 8 : 2)) {
                const int kbs = cdiv(KB, ks);
                if (ks_force <= 0 && (cdiv(KB, kbs) != ks || (ks > 1 && kbs < 4))) continue;
                const long wgs = tiles * ks;
                const long rounds = (wgs + cu - 1) / cu;
                const double kib = ((double)bm * abpk * kbs + (double)bn / 16 * 1024 * kbs + (double)bm * bn * 4) / 1024;
                double t = rounds * (1.5 + 0.027 * kib);
                if (ks > 1) t += 3.0 + 2.0 * ks * (double)M * N * 4 / 4e6;
                if (best < 0 || t < best - 1e-9) {
                    best = t;
                    q->algo = ORKH_ALGO_TILED2;
                    q->bm = bm;
                    q->bn = bn;
                    q->ksplit = ks;
                    q->kbs = kbs;
                }
            }
        }
        if (q->ksplit > 1) *ws_bytes = (size_t)q->ksplit * M * N * 4;
        return 0;
    }

    /* k_tiled (NF4, or ORK_PLAN=tiled): each CU pulls its tiles' A and B rows through L2 at a roughly fixed
     * rate, so the time of a round of workgroups is about the operand bytes one workgroup loads. K is split
     * across workgroups when that cuts the per-workgroup bytes by more than the partial sums and the extra
     * reduce launch (~2 us) cost. Model units: us at ~48 KB/us per CU (measured order of magnitude),
     * 5 TB/s for the partials' HBM round trip. */
    static const int cfg[][2] = {{128, 96}, {128, 128}, {64, 64}};
    const int bpk = 64;                                                  /* B bytes per column per K-block, every kind */
    const int apk = (rkind == ORKH_I4U || rkind == ORKH_NF4) ? 128 : 64; /* A bytes per row per K-block */
    for (int i = 0; i < 3; i++) {
        const int bm = cfg[i][0], bn = cfg[i][1];
        const long tiles = (long)cdiv(M, bm) * cdiv(NB, bn / 16);
        for (int ks = ks_force > 0 ? ks_force : 1; ks <= (ks_force > 0 ? ks_force : 8); ks++) {
            const int kbs = cdiv(KB, ks);
            if (ks_force <= 0 && (cdiv(KB, kbs) != ks || (ks > 1 && kbs < 4))) continue;
            const long wgs = tiles * ks;
            const long rounds = (wgs + cu - 1) / cu;
            double t = rounds * (double)(bm * apk + bn * bpk) * kbs / 48e3;
            if (ks > 1) t += 2.0 + 2.0 * ks * (double)M * N * 4 / 5e6;
            if (best < 0 || t < best - 1e-9) {
                best = t;
                q->bm = bm;
                q->bn = bn;
                q->ksplit = ks;
                q->kbs = kbs;
            }
        }
    }
    q->algo = ORKH_ALGO_TILED;
    if (q->ksplit > 1) *ws_bytes = (size_t)q->ksplit * M * N * 4;
    return 0;
}
