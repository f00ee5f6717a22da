/* plan.c -- the MI355X matmul planner: which kernel, what grid, how K is split.
 *
 * Replaces the reference's K-split / N-tile / M-tile / core-count policy (orki_int8_ks, orki_budget,
 * orki_run_loop_chunk, the mg_max*64 M-tile: src/npu.c:131-160, :1598-1610, :1693-1694;
 * orki_f16_ks, src/npu/f16/regcmd.c:120-125). The NPU needed K cut into 1024-wide slices, N into
 * 8192-wide outputs and M into CBUF-sized row groups, each a separate submit with a host int32
 * accumulate. On MI355X every shape is one launch (plus a reduce pass when K is split across
 * workgroups); the planner only decides how to fill 256 CUs:
 *   M = 1    GEMV: half a 16-column panel per workgroup (whole panels where those already spread evenly over
 *            the CUs), waves split K in runs of ~8 KiB; K is split across workgroups only for long-K,
 *            few-panel shapes that leave the machine underfilled.
 *   M <= 64  the streaming kernel (same grid, runs of 1-4 KiB) or the LDS-ring tiled kernel, whichever a
 *            delivery model of both prices lower, each with its best K split.
 *   M >  64  the LDS-ring tiled kernel: the tile and K split with the least modelled time.
 *   NF4      (M > 1) the streaming kernel, k_tiled and the LDS-ring kernel, every tile and split, each priced by
 *            its own fit (nf4_best).
 * Both time models charge a workgroup for a fixed set-up, the operand bytes that must reach its CU and
 * its multiply-accumulates; a K split adds its partials' round trip and the reduce launch.
 * ORK_PLAN=stream|tiled, ORK_TILE=BMxBN (with ORK_PLAN=tiled: a k_tiled tile) and ORK_KSPLIT=n force a kernel,
 * tile or split (tests, A/B); they and
 * the other overrides below are read only on a context made with ORK_PLAN_DEBUG set (knob()), so a stray
 * variable cannot change the kernels of a production context. */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "internal.h"

static int cdiv(int a, int b) { return (a + b - 1) / b; }

/* A planner test override: the environment variable on a context made with ORK_PLAN_DEBUG, else nothing. */
static const char *knob(const ork_npu *c, const char *name) { return (c && c->plan_knobs) ? getenv(name) : NULL; }

/* A bytes per activation row per 1 KiB weight block (K-block of the panel layout) */
static int a_bytes_per_kb(int rkind) { return rkind == ORKH_F16 ? 64 : (rkind == ORKH_I8 ? 64 : 128); }
static int kpb_of(int rkind) { return rkind == ORKH_I8 ? 64 : rkind == ORKH_F16 ? 32 : 128; }

/* Streaming-kernel geometry for a K split of ks (1 = unsplit). Run length per wave: 8 KiB in flight per
 * wave for the int8/fp16 GEMV (M = 1); more waves with shorter runs where each block costs more issue
 * (more rows, int4 decode). Measured on the K=2048, N=6144 panels; the run lengths on either side were
 * within 2-4%. */
/* Paired panels for the streaming kernel: with more panels than CUs (but fewer than two per CU), one round of
 * cu workgroups, the first NB - cu owning two adjacent panels, balances the bytes per CU, and each wave loads
 * an A chunk once for both panels. Measured (K=2048 N=6144, us, single -> paired): int8 M=16 4.81 -> 4.43,
 * M=32 7.39 -> 5.60; fp16 M=16 8.17 -> 6.71; W4A8 M=16 4.25 -> 3.96, M=32 6.65 -> 4.85; M <= 8 no gain (M=2
 * 4.25 -> 4.43). The kernel holds up to two row tiles per panel. ORK_STREAM_NP=1 / 2 turns it off / on
 * wherever it applies (tests). */
static int stream_paired(const ork_npu *c, int M, int mt, int NB, int cu, int ks) {
    if (ks != 1 || mt > 2 || NB <= cu || NB >= 2 * cu || M < 2) return 0;
    const char *e = knob(c, "ORK_STREAM_NP");
    if (e) return atoi(e) == 2;
    return M > 8;
}

static void stream_geom(const ork_npu *c, int rkind, int M, int KB, int NB, int cu, int ks, orkh_plan *q) {
    const int kbw_target = (rkind == ORKH_I4U || rkind == ORKH_NF4) ? 2 : (M > 1 ? 4 : 8);
    const int need = cdiv(KB, kbw_target); /* waves per panel at the target run length */
    int wpg = need <= 4 ? 4 : 8;
    /* an int8 GEMV with fewer panels than CUs runs 8 shorter waves per panel: 2.94 -> 2.84 us at K=N=2048,
     * 2.80 -> 2.67 us at N=1024; with more panels than CUs 4 stay ahead (3.94 vs 4.04 us at N=6144) */
    if (M == 1 && rkind == ORKH_I8 && NB < cu) wpg = 8;
    const char *fw = knob(c, "ORK_WPG"); /* testing / A-B: waves per panel of the GEMV (4 or 8) */
    if (M == 1 && fw && (atoi(fw) == 4 || atoi(fw) == 8)) wpg = atoi(fw);
    if (ks > KB) ks = KB;
    if (ks < 1) ks = 1;
    const int kbs = cdiv(KB, ks);
    q->mt = cdiv(M, 16);
    q->wpg = wpg;
    q->kbs = kbs;
    q->kbw = cdiv(kbs, wpg);
    q->ksplit = cdiv(KB, kbs);
    q->np = stream_paired(c, M, q->mt, NB, cu, q->ksplit) ? 2 : 1;
    q->npg = q->np == 2 ? cu : NB;
}

/* The GEMV's split rule: split only when the panels leave the machine underfilled (< 4 waves per CU) AND
 * each wave would otherwise stream more than two runs back to back; the split costs a second launch
 * (the fixed-order reduce), which a one-run wave never repays. */
static int stream_rule_ks(const ork_npu *c, int rkind, int M, int KB, int NB, int cu) {
    orkh_plan g;
    stream_geom(c, rkind, M, KB, NB, cu, 1, &g);
    const int kbw_target = (rkind == ORKH_I4U || rkind == ORKH_NF4) ? 2 : (M > 1 ? 4 : 8);
    const int runs = cdiv(cdiv(KB, g.wpg), kbw_target);
    int ks = 1;
    if ((long)NB * g.wpg < 4L * cu && runs > 2) {
        ks = cdiv(4 * cu, NB * g.wpg);
        if (ks > runs) ks = runs; /* every wave keeps a full run */
    }
    return ks;
}

/* The GEMV's half-panel geometry (k_gemv_half: 8 columns per workgroup, so the bytes spread evenly over the CUs
 * whatever N/16 is): waves whose runs are about four load instructions (eight K-blocks; two instructions for
 * NF4, whose codebook decode is heavier), 2, 4 or 8 waves. Measured against whole panels (graph-timed, us):
 *   int8  K=2048 N=6144 3.95 -> 3.82; K=N=2048 2.77 -> 2.50; K=6144 N=2048 4.33 -> 3.77; K=8192 N=512 4.30 -> 3.39;
 *         K=2048 N=151936 (an LM head) 45.9 -> 44.6
 *   fp16  K=N=2048 3.52 -> 3.17
 *   W4A8  uniform K=2048 N=6144 3.14 -> 3.10, K=6144 N=2048 3.94 -> 3.15; NF4 K=2048 N=6144 3.58 -> 3.28,
 *         K=6144 N=2048 4.44 -> 3.35; W4A4 K=N=4096 3.60 -> 3.33
 * Where whole panels already spread evenly (N/16 x the K split a multiple of the CU count) they stay: K=2048
 * N=4096 int8 3.19 whole, 3.22 halves. ORK_GEMV_HALF=0/1 forces either and ORK_WPG=2/4/8 the waves (tests, A/B). */
static void gemv_half_geom(const ork_npu *c, int rkind, int NB, int cu, orkh_plan *q) {
    const char *e = knob(c, "ORK_GEMV_HALF");
    if (e && atoi(e) == 0) return;
    const long wgs = (long)NB * q->ksplit;
    if (!e && wgs >= cu && cdiv((int)(2 * wgs), cu) >= 2 * cdiv((int)wgs, cu)) return;
    const int blocks_per_wave = rkind == ORKH_NF4 ? 4 : 8;
    const int need = cdiv(q->kbs, blocks_per_wave);
    q->half = 1;
    q->wpg = need <= 2 ? 2 : need <= 4 ? 4 : 8;
    const char *fw = knob(c, "ORK_WPG");
    if (fw && (atoi(fw) == 2 || atoi(fw) == 4 || atoi(fw) == 8)) q->wpg = atoi(fw);
    q->kbw = cdiv(q->kbs, q->wpg);
}

int orki_gemv_panel_wpg(const ork_npu *c, int rkind, int KB, int NB) {
    orkh_plan g;
    memset(&g, 0, sizeof g);
    stream_geom(c, rkind, 1, KB, NB, (c && c->cores > 0) ? c->cores : 256, 1, &g);
    return g.wpg;
}

/* Time models (us) of the two MFMA kernels, for int8, fp16 and uniform int4 weights. A workgroup's time is
 * the sum of
 *   a fixed launch / drain cost and a cost per workgroup placed on the busiest CU ("per"),
 *   the operand bytes that must reach its CU (A rows, B blocks, C tile), per KiB: the ~15 B/clk per CU
 *   that L2 delivers, and (LDS-ring kernel) a further share that grows with the number of CUs pulling
 *   at once, and
 *   its multiply-accumulates at the kind's rate (per million MACs: int8 ~0.1 us, fp16 ~0.19 us, int4
 *   with decode ~0.2 us in the LDS-ring kernel -- the MFMA peaks; ~10x that in the streaming kernel,
 *   whose few waves per panel keep dependent MFMA chains);
 * with nothing overlapped between the three. A K split adds the reduce launch and the int32/fp32
 * partials written and read back. Least-squares fits to 588 timed launches (int8, fp16, W4A8, W4A4;
 * M = 16..4096, K = 2048..6144, N = 2048..22016; every tile and split on offer): 4% rms error for the
 * streaming kernel, 7% for the tiled one, and the pick within 1% of the fastest timed candidate. */
static double mac_rate(int rkind, int tiled) {
    if (rkind == ORKH_I8) return tiled ? 0.100 : 0.94;
    if (rkind == ORKH_F16) return tiled ? 0.187 : 1.90;
    if (rkind == ORKH_NF4) return tiled ? 0.40 : 0.91; /* tiled: with the per-stage decode into LDS (12% rms) */
    return tiled ? 0.199 : 0.91;
}

/* Half panels on the streaming kernel (8 columns per workgroup, twice the workgroups): each workgroup loads half
 * of its panel's B but all of its rows of A. Offered for int8 and fp16, whose panel bytes are a large share of a
 * workgroup's; priced by the same model with the halved B and C bytes. Measured against whole panels (graph-timed,
 * best split of each, us): fp16 K=N=2048 M=16 4.98 -> 4.41, M=8 4.18 -> 3.94; K=2048 N=768 M=16 4.74 -> 4.17; int8
 * K=N=2048 M=32 4.54 -> 4.13, K=6144 N=2048 M=16 6.74 -> 5.87, K=8192 N=1024 M=8 5.88 -> 5.21; where the halves
 * need a second round of the CUs they lose (int8 K=N=4096 M=16 5.55 -> 6.79). The uniform-int4 and NF4 nibbles are
 * a small share of a workgroup's bytes next to its int8 rows of A: half panels lost 2-8% below 32 rows and gained
 * 2-5% above, so they keep whole panels. Over 72 int8 / fp16 shapes (K x N = 2048 x 2048, 2048 x 768, 4096 x 4096,
 * 6144 x 2048, 8192 x 1024, 2048 x 6144; M = 2..64) the model's picks come within 3% of the fastest streaming
 * candidate of each. */
static int stream_half_offered(int rkind) { return rkind == ORKH_I8 || rkind == ORKH_F16; }

static double stream_us(const ork_npu *c, int rkind, int M, int N, int KB, int cu, int ks, int half) {
    orkh_plan g;
    stream_geom(c, rkind, M, KB, N / 16, cu, ks, &g);
    if (half && g.np == 2) return -1; /* paired and half panels exclude each other */
    const int pp = g.np == 2 ? 2 : 1; /* panels of the busiest workgroup */
    const long wgs = g.np == 2 ? g.npg : (long)(N / 16) * g.ksplit * (half ? 2 : 1);
    const double per = (double)((wgs + cu - 1) / cu);
    const double kib = ((double)M * a_bytes_per_kb(rkind) * g.kbs +
                        pp * ((half ? 512.0 : 1024.0) * g.kbs + (half ? 32.0 : 64.0) * M)) / 1024;
    const double mmac = (double)pp * g.mt * 16 * 16 * g.kbs * kpb_of(rkind) / 1e6;
    double t = 1.74 + per * (0.103 + 0.017 * kib + mac_rate(rkind, 0) * mmac);
    if (g.ksplit > 1) t += 2.81 + 0.327 * g.ksplit * (double)M * N * 4 / 1e6;
    return t;
}

/* NF4 above one row. Its codebook decode shifts each kernel's balance of operand delivery and VALU work differently
 * per tile, so every candidate has its own least-squares fit (relative error, non-negative terms) to graph-timed
 * launches on MI355X: 45 shapes (K x N = 2048 x 6144, 6144 x 2048, 4096 x 4096, 2048 x 2048, 2048 x 12288;
 * M = 32..1024), 1007 kernel / tile / split candidates in all (tests/golden/nf4_plan_sweep.json),
 *   t = a + rounds * (b + c * KiB) + [ks > 1] (d + e * ks * M * N * 4 / 1e6)   us,
 * KiB being the A and B bytes one workgroup loads (the streaming kernel: the form of stream_us). The fits are
 * within 4-7% rms per candidate; over the 45 shapes the picks total within 0.6% of the fastest timed candidate of
 * each. Refitted after the LDS-ring kernel's stage loads moved behind the first K-block of stage work (128 x 128
 * and 64 x 64 ran 2-7% faster) and with its 128 x 96 tile offered: the earlier fits, without it, totalled 2.2%
 * above the fastest on the same launches (K=4096 N=4096 M=384 24.1 us against 22.8 on 128 x 96, K=2048 N=6144
 * M=128 10.0 on k_tiled against 9.5 on the LDS ring's 64 x 64). */
static const struct nf4_fit {
    int algo, bm, bn, ksmax;
    double a, b, c, d, e;
} nf4_fits[] = {
    {ORKH_ALGO_TILED2, 128, 128, 4, 4.1310, 0.6805, 0.0272, 1.7563, 0.4771},
    {ORKH_ALGO_TILED2, 128, 96, 4, 2.4251, 2.0721, 0.0268, 2.2542, 0.5308},
    {ORKH_ALGO_TILED2, 64, 64, 4, 3.9420, 0.0000, 0.0287, 2.0167, 0.5399},
    {ORKH_ALGO_TILED2, 32, 64, 4, 1.0803, 2.1819, 0.0297, 2.6830, 0.3840},
    {ORKH_ALGO_TILED, 128, 128, 8, 5.3951, 3.6657, 0.0342, 2.9489, 0.4949},
    {ORKH_ALGO_TILED, 128, 96, 8, 3.8782, 3.9816, 0.0295, 2.9108, 0.4612},
    {ORKH_ALGO_TILED, 64, 64, 8, 3.5590, 1.4223, 0.0257, 2.7922, 0.4108},
};

static void nf4_best(const ork_npu *c, int M, int N, int KB, int cu, orkh_plan *q) {
    const int NB = N / 16;
    const double part = (double)M * N * 4 / 1e6; /* MB of one K slice's partials */
    double best = -1;
    for (int ks = 1; ks <= 8; ks *= 2) {
        const int kbs = cdiv(KB, ks);
        if (cdiv(KB, kbs) != ks || (ks > 1 && kbs < 2)) continue;
        if (M <= 64 && ks <= 4) { /* the streaming kernel holds up to 64 rows */
            orkh_plan g;
            memset(&g, 0, sizeof g);
            stream_geom(c, ORKH_NF4, M, KB, NB, cu, ks, &g);
            const int pp = g.np == 2 ? 2 : 1;
            const long wgs = g.np == 2 ? g.npg : (long)NB * g.ksplit;
            const double per = (double)((wgs + cu - 1) / cu);
            const double kib = ((double)M * 128 * g.kbs + pp * (1024.0 * g.kbs + 64.0 * M)) / 1024;
            const double mmac = (double)pp * g.mt * 16 * 16 * g.kbs * 128 / 1e6;
            double t = 2.0835 + per * (0.0241 * kib + 0.2942 * mmac);
            if (ks > 1) t += 2.0516 + 0.6116 * ks * part;
            if (best < 0 || t < best - 1e-9) {
                best = t;
                *q = g;
                q->algo = ORKH_ALGO_STREAM;
            }
        }
        for (size_t i = 0; i < sizeof nf4_fits / sizeof nf4_fits[0]; i++) {
            const struct nf4_fit *f = &nf4_fits[i];
            if (ks > f->ksmax) continue;
            const long wgs = (long)cdiv(M, f->bm) * cdiv(NB, f->bn / 16) * ks;
            const double rounds = (double)((wgs + cu - 1) / cu);
            const double kib = ((double)f->bm * 128 + (double)f->bn * 64) * kbs / 1024;
            double t = f->a + rounds * (f->b + f->c * kib);
            if (ks > 1) t += f->d + f->e * ks * part;
            if (best < 0 || t < best - 1e-9) {
                best = t;
                memset(q, 0, sizeof *q);
                q->algo = f->algo;
                q->bm = f->bm;
                q->bn = f->bn;
                q->ksplit = ks;
                q->kbs = kbs;
            }
        }
    }
}

/* int8, fp16 and uniform int4 above 64 rows: like NF4, every LDS-ring tile has its own least-squares fit (relative
 * error, non-negative terms) to graph-timed launches on MI355X, in the form of nf4_fits, KiB being the A and B bytes
 * one workgroup loads (tests/golden/mma_plan_sweep.json: every tile and K split of 1, 2 and 4 on offer at
 * K x N = 2048 x 6144, 2048 x 2048, 4096 x 4096, 6144 x 2048, 2048 x 12288 and M = 96..2048; the 32- and 16-row
 * tiles for one round of the CUs only). A tile is priced only where its rows are at most twice M, as timed. */
static const struct mma_fit {
    int rkind, bm, bn, ksmax; /* ksmax: the largest K split timed (and offered) */
    double a, b, c, d, e;
} mma_fits[] = { /* kind, tile, ksmax, a..e; then the launches fitted and the fit's rms relative error */
    {ORKH_I8, 256, 256, 4, 5.8440, 0.0000, 0.0241, 0.0000, 0.3994}, /* 16, 3.1% */
    {ORKH_I8, 128, 128, 4, 2.1719, 1.6437, 0.0156, 2.4427, 0.4431}, /* 82, 7.2% */
    {ORKH_I8, 128, 96, 4, 2.9512, 2.1169, 0.0143, 2.2673, 0.4083}, /* 75, 5.9% */
    {ORKH_I8, 64, 192, 4, 3.4918, 0.7902, 0.0145, 2.0294, 0.4527}, /* 74, 7.5% */
    {ORKH_I8, 64, 64, 4, 2.4453, 0.5219, 0.0160, 2.5433, 0.4340}, /* 79, 4.6% */
    {ORKH_I8, 32, 64, 2, 2.7092, 0.0000, 0.0223, 2.3342, 0.4118}, /* 14, 0.6% */
    {ORKH_I8, 32, 32, 1, 0.0000, 2.2276, 0.0188, 0.0000, 0.0000}, /* 4, 0.2% */
    {ORKH_I8, 16, 64, 1, 0.0000, 2.6950, 0.0192, 0.0000, 0.0000}, /* 4, 0.1% */
    {ORKH_F16, 256, 256, 4, 0.0880, 6.1768, 0.0227, 0.0000, 0.3771}, /* 38, 4.7% */
    {ORKH_F16, 128, 128, 4, 4.0377, 0.2295, 0.0161, 1.6667, 0.4677}, /* 92, 6.6% */
    {ORKH_F16, 128, 96, 4, 5.2807, 0.7426, 0.0150, 0.9779, 0.4447}, /* 91, 6.2% */
    {ORKH_F16, 64, 192, 4, 5.9856, 0.0000, 0.0145, 0.6252, 0.4682}, /* 89, 7.1% */
    {ORKH_F16, 64, 64, 4, 2.8047, 0.0000, 0.0180, 2.8555, 0.4211}, /* 92, 6.4% */
    {ORKH_F16, 32, 64, 2, 2.6572, 0.0000, 0.0223, 2.4686, 0.3812}, /* 13, 1.6% */
    {ORKH_F16, 32, 32, 1, 0.0000, 2.7401, 0.0175, 0.0000, 0.0000}, /* 4, 0.2% */
    {ORKH_F16, 16, 64, 1, 0.0000, 3.4902, 0.0175, 0.0000, 0.0000}, /* 4, 0.3% */
    {ORKH_I4U, 128, 128, 4, 2.1327, 1.8768, 0.0211, 2.5510, 0.4127}, /* 57, 5.8% */
    {ORKH_I4U, 128, 96, 4, 0.7882, 4.7886, 0.0180, 2.3200, 0.4005}, /* 46, 4.9% */
    {ORKH_I4U, 64, 192, 4, 0.1933, 4.9232, 0.0174, 2.4635, 0.3617}, /* 57, 5.8% */
    {ORKH_I4U, 64, 64, 4, 0.3768, 3.0260, 0.0137, 2.3979, 0.4614}, /* 60, 3.8% */
    {ORKH_I4U, 32, 64, 2, 0.0000, 2.8698, 0.0196, 2.1311, 0.5144}, /* 14, 0.5% */
    {ORKH_I4U, 32, 32, 1, 0.0000, 2.7500, 0.0158, 0.0000, 0.0000}, /* 4, 0.1% */
    {ORKH_I4U, 16, 64, 1, 0.0000, 3.0075, 0.0175, 0.0000, 0.0000}, /* 4, 0.1% */
};

static double mma_fit_best(int rkind, int M, int N, int KB, int cu, int ks_force, orkh_plan *q) {
    const int NB = N / 16;
    const double part = (double)M * N * 4 / 1e6;
    double best = -1;
    for (size_t i = 0; i < sizeof mma_fits / sizeof mma_fits[0]; i++) {
        const struct mma_fit *f = &mma_fits[i];
        if (f->rkind != rkind || f->bm > 2 * M) continue;
        for (int ks = 1; ks <= f->ksmax; ks *= 2) {
            if (ks_force > 0 && ks != ks_force) continue;
            const int kbs = cdiv(KB, ks);
            if (cdiv(KB, kbs) != ks || (ks > 1 && kbs < 4)) continue;
            const long wgs = (long)cdiv(M, f->bm) * cdiv(NB, f->bn / 16) * ks;
            if (f->bm <= 32 && wgs > cu) continue;
            const double rounds = (double)((wgs + cu - 1) / cu);
            const double kib = ((double)f->bm * a_bytes_per_kb(rkind) + (double)f->bn * 64) * kbs / 1024;
            double t = f->a + rounds * (f->b + f->c * kib);
            if (ks > 1) t += f->d + f->e * ks * part;
            if (best < 0 || t < best - 1e-9) {
                best = t;
                memset(q, 0, sizeof *q);
                q->algo = ORKH_ALGO_TILED2;
                q->bm = f->bm;
                q->bn = f->bn;
                q->ksplit = ks;
                q->kbs = kbs;
            }
        }
    }
    return best;
}

/* The LDS-ring kernel (k_tiled2): every tile and split on offer priced by the model above; A counts the
 * whole tile height, since rows past M still issue (zero-filled) loads. Returns the modelled time of
 * the best and fills q with it. */
static double tiled2_best(int rkind, int M, int N, int KB, int cu, int ks_force, int cfg_from, orkh_plan *q) {
    /* 32-row tiles split each stage's K-blocks over groups of waves; the model prices them unchanged (measured:
     * fp16 M=128 K=N=2048 32x32 9.0 us vs 9.04 modelled, W4A8 M=64 K=2048 N=6144 32x64 7.27 vs 7.28) */
    static const int cfg2[][2] = {{256, 256}, {128, 128}, {64, 192}, {64, 64}, {32, 64}, {32, 32}, {16, 64}, {16, 32}};
    const int NB = N / 16;
    const int abpk = a_bytes_per_kb(rkind), kpb = kpb_of(rkind);
    double best = -1;
    for (int i = cfg_from; i < (int)(sizeof cfg2 / sizeof cfg2[0]); i++) {
        const int bm = cfg2[i][0], bn = cfg2[i][1];
        /* NF4's decoded (int8) B doubles the LDS reads of the 3-panel wave tile: 22.3 us at M=512 vs 19.8 on
         * 128 x 128, which the model does not see; on 32-row tiles its per-block decode is shared by half the
         * rows the model assumes (not timed: not offered) */
        if (rkind == ORKH_NF4 && (bn == 192 || bm <= 32)) continue;
        const long tiles = (long)cdiv(M, bm) * cdiv(NB, bn / 16);
        for (int ks = ks_force > 0 ? ks_force : 1; ks <= (ks_force > 0 ? ks_force : 8); ks *= (ks_force > 0 ? 8 : 2)) {
            const int kbs = cdiv(KB, ks);
            if (ks_force <= 0 && (cdiv(KB, kbs) != ks || (ks > 1 && kbs < 4))) continue;
            const long wgs = tiles * ks;
            /* the model underprices several rounds of the K-group tiles (W4A8 M=256 K=2048 N=6144 32x64: 18.2 us
             * measured, 14.3 modelled; int8 M=128 N=6144 32x32: 16.4 vs 12.2), so they are offered for one round */
            if (bm <= 32 && wgs > cu) continue;
            /* nor split 8 ways: both such picks ran 24-30% above the model (fp16 K=6144 N=2048 M=16 16 x 64: 12.05 us
             * measured, 9.18 modelled; M=32 32 x 64: 12.03 against 32 x 32 split 4 ways at 11.56), where splits of
             * up to 4 sit at 0.93-0.98 of it */
            if (bm <= 32 && ks > 4) continue;
            const double per = (double)((wgs + cu - 1) / cu);
            const double busy = (double)(wgs < cu ? wgs : cu) / cu;
            const double kib = ((double)bm * abpk * kbs + (double)bn / 16 * 1024 * kbs + (double)bm * bn * 4) / 1024;
            const double mmac = (double)bm * bn * kbs * kpb / 1e6;
            double t = 4.09 + per * (0.35 + (0.0104 + 0.0058 * busy) * kib + mac_rate(rkind, 1) * mmac);
            if (ks > 1) t += 2.11 + 0.456 * ks * (double)M * N * 4 / 1e6;
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
    return best;
}

static int plan_core(const ork_npu *c, int rkind, int M, int K, int N, int KB, orkh_plan *q, size_t *ws_bytes);

/* A-stage layout of the LDS-ring kernel: whole 128-byte row lines (swizzled LDS image; a stage row of 1, 2 or 4
 * lines) or MFMA fragment order. Measured on MI355X, graph-timed, both layouts alternated three times in one run,
 * exact (us, fragment -> line):
 *   one line a stage row:  int8 64x64 K=2048 N=6144 M=128 8.25 -> 7.95, M=256 13.44 -> 11.73, K=N=2048 M=128 7.87 ->
 *                          7.68, M=512 7.88 -> 7.83; int8 64x192 M=256 12.62 -> 11.95, M=512 13.09 -> 12.91; int8
 *                          32x64 M=96 10.90 -> 10.51; int8 128x96 M=512 14.64 -> 12.36; fp16 64x64 K=N=2048 M=128
 *                          12.64 -> 13.05, M=512 12.41 -> 13.18, K=2048 N=6144 M=128 13.83 -> 13.27, M=256 22.92 ->
 *                          20.12; fp16 32x64 M=96 K=N=2048 11.29 -> 11.48, M=256 11.19 -> 11.39; NF4 64x64 M=128
 *                          9.57 -> 9.68, M=256 14.26 -> 14.69
 *   2-4 lines a stage row: W4A4 K=N=4096 64x64 M=256 11.98 -> 10.07, 32x32 M=64 8.19 -> 6.83, 16x32 M=32 6.17 ->
 *                          5.64; W4A8 K=2048 N=6144 64x64 M=128 8.01 -> 7.33, 64x192 M=512 11.78 -> 11.57, 32x64
 *                          M=64 5.84 -> 5.90 (W4A4 M=128 7.91 -> 8.06, M=96 8.40 -> 8.10); NF4 32x64 M=64 6.98 ->
 *                          7.04, M=96 12.43 -> 12.57, 16x64 M=48 11.57 -> 11.65, 32x32 K=N=2048 M=64 5.69 -> 5.55;
 *                          NF4 128x96 M=256 14.29 -> 14.26, M=512 14.96 -> 14.92; int8 32x32 K=N=2048 M=128 5.68 ->
 *                          5.55, 16x32 M=32 5.56 -> 5.34; fp16 32x32 M=128 8.06 -> 7.64, 16x32 M=48 7.35 -> 6.87,
 *                          16x64 M=64 9.49 -> 9.21
 * so lines except: fp16 32x64, and fp16 64x64 unless N > 4096; the nibble kinds' 32x64 tile; NF4's 64x64, 128x96
 * (no gain) and 16-row tiles. ORK_ALINE=0/1 forces it (tests, A/B timing). */
static int aline_rule(const ork_npu *c, int rkind, const orkh_plan *q, int N) {
    /* the kernel has the line layout only where a stage row is whole 128-byte lines: K-blocks per stage as
     * k_tiled2's t2_ks (1 for int4 kinds, 1 for 256 x 256, else 2; at least the tile's K groups of waves) */
    /* k_tiled2's wave grid (t2_xg, t2_wn): 2 x 4 on the uniform-int4 64 x 192 tile, 2 x 2 on its 64 x 64 tile */
    const int xg = (rkind == ORKH_I4U && q->bm == 64) ? (q->bn == 192 ? 1 : q->bn == 64 ? 2 : 0) : 0;
    const int nbt = q->bn / 16, mb = xg ? 2 : (q->bm / 16 < 4 ? q->bm / 16 : 4);
    const int nb = xg == 2 ? 2 : (nbt < 4 ? nbt : (nbt % 4 == 0 ? 4 : 2)), wk = 16 / (mb * nb);
    const int base = (rkind == ORKH_I4U || rkind == ORKH_NF4) ? 1 : (q->bm * q->bn >= 65536 ? 1 : 2);
    const int ks = base > wk ? base : wk;
    const int row_bytes = ks * a_bytes_per_kb(rkind);
    if (row_bytes % 128) return 0;
    const char *e = knob(c, "ORK_ALINE");
    if (e) return atoi(e) != 0;
    if (rkind == ORKH_F16) {
        if (q->bm == 32 && q->bn == 64) return 0;
        if (q->bm == 64 && q->bn == 64) return N > 4096;
    }
    if ((rkind == ORKH_I4U || rkind == ORKH_NF4) && q->bm == 32 && q->bn == 64) return 0;
    if (rkind == ORKH_NF4 && ((q->bm == 64 && q->bn == 64) || q->bm == 16 || (q->bm == 128 && q->bn == 96))) return 0;
    return 1;
}

int orki_plan(const ork_npu *c, int rkind, int M, int K, int N, int KB, orkh_plan *q, size_t *ws_bytes) {
    const int rc = plan_core(c, rkind, M, K, N, KB, q, ws_bytes);
    if (q->algo == ORKH_ALGO_TILED2) q->aline = aline_rule(c, rkind, q, N);
    /* The LDS-ring kernel's two-slot ring (two workgroups per CU, where the kernel has it for the tile) on grids of
     * more than one round of the CUs: one workgroup's set-up, first stage and epilogue overlap the other's loop.
     * Measured against the 4-slot ring (graph-timed, us; K=2048 N=6144 unless given): int8 64x192 M=768 22.95 ->
     * 18.87, M=1024 24.76 -> 21.78; int8 128x128 K=N=4096 M=2048 50.34 -> 45.79, K=N=2048 M=4096 31.6 -> 26.32;
     * fp16 64x192 M=768 41.16 -> 33.48, 128x128 K=N=2048 M=4096 54.95 -> 45.98; uniform int4 128x128 M=2048
     * 43.14 -> 33.87. On one round it loses (int8 64x192 M=512 13.38 -> 14.72, 128x128 K=N=4096 M=1024 25.41 ->
     * 29.11). ORK_RING=0/2 forces either (tests, A/B). */
    if (q->algo == ORKH_ALGO_TILED2) {
        const char *fr = knob(c, "ORK_RING");
        const int cu = (c && c->cores > 0) ? c->cores : 256;
        long wgs = (long)cdiv(M, q->bm) * cdiv(N / 16, q->bn / 16) * (q->ksplit > 1 ? q->ksplit : 1);
        /* uniform int4's 64 x 192 tile has no two-slot form (41 KiB stages): where its grid and 128 x 128's both
         * exceed one round, 128 x 128 with two slots (us, W4A8 K=2048: N=6144 M=768 21.74 -> 19.96, M=1024 22.61
         * -> 20.36; N=12288 M=512 22.43 -> 20.06, M=768 32.23 -> 29.71) */
        const long w128 = (long)cdiv(M, 128) * cdiv(N / 16, 8);
        if (rkind == ORKH_I4U && !fr && !knob(c, "ORK_TILE") && q->bm == 64 && q->bn == 192 && q->ksplit <= 1 &&
            wgs > cu && w128 > cu && orkh_tiled2_ring2_ok(rkind, 128, 128)) {
            q->bm = q->bn = 128;
            q->aline = aline_rule(c, rkind, q, N);
            wgs = w128;
        }
        if (fr) q->ring = atoi(fr) == 2 ? 2 : 0;
        else if (wgs > cu && orkh_tiled2_ring2_ok(rkind, q->bm, q->bn)) q->ring = 2;
        /* C stored write-through (device scope) where the grid is one round of the CUs: every workgroup stores at
         * about the same time, after all the loads, and the L2s pass C on to memory as it comes instead of holding
         * up to 64 MB of it dirty for the end of the kernel. Graph-timed against write-back stores (us): int8 K=2048
         * N=6144 M=512 64 x 192 14.56 -> 13.45, M=256 12.89 -> 12.52; uniform int4 M=512 64 x 192 13.96 -> 12.60;
         * W4A4 K=N=4096 M=256 64 x 64 12.55 -> 12.21; fp16 K=N=2048 M=512 64 x 64 13.00 -> 12.65; int8 M=K=N=4096
         * 256 x 256 67.72 -> 66.35; int8 K=N=2048 M=128 32 x 32 5.66 -> 5.57; W4A8 M=64 32 x 64 6.25 -> 6.06. On
         * grids of several rounds the early writes compete with the later workgroups' loads: int8 M=1024 two-slot
         * 23.37 -> 25.80, fp16 M=768 32.84 -> 36.11. ORK_CWT=0/1 forces either. */
        const char *fc = knob(c, "ORK_CWT");
        q->cwt = fc ? atoi(fc) != 0 : wgs <= cu;
    }
    return rc;
}

static int plan_core(const ork_npu *c, int rkind, int M, int K, int N, int KB, orkh_plan *q, size_t *ws_bytes) {
    (void)K;
    memset(q, 0, sizeof *q);
    *ws_bytes = 0;
    const int cu = (c && c->cores > 0) ? c->cores : 256;
    const int NB = N / 16;
    const char *force = knob(c, "ORK_PLAN");
    const int f_stream = force && !strcmp(force, "stream"), f_tiled = force && !strcmp(force, "tiled");
    const char *fks = knob(c, "ORK_KSPLIT");
    int ks_force = fks ? atoi(fks) : 0;
    if (ks_force > KB) ks_force = KB;
    if (ks_force > 0) ks_force = cdiv(KB, cdiv(KB, ks_force)); /* as a split can realise it */

    const char *tf = knob(c, "ORK_TILE"); /* "BMxBN": that tile of the LDS-ring kernel (of k_tiled with ORK_PLAN=tiled) */
    int fbm, fbn;
    if (tf && sscanf(tf, "%dx%d", &fbm, &fbn) == 2) {
        const int ks = ks_force > 0 ? ks_force : 1;
        q->algo = f_tiled ? ORKH_ALGO_TILED : ORKH_ALGO_TILED2;
        q->bm = fbm;
        q->bn = fbn;
        q->kbs = cdiv(KB, ks);
        q->ksplit = cdiv(KB, q->kbs);
        if (q->ksplit > 1) *ws_bytes = (size_t)q->ksplit * M * N * 4;
        return 0;
    }

    if (rkind == ORKH_NF4 && M > 1 && !f_stream && !f_tiled && ks_force <= 0) {
        nf4_best(c, M, N, KB, cu, q);
        if (q->ksplit > 1) *ws_bytes = (size_t)q->ksplit * M * N * 4;
        return 0;
    }

    if (M <= 64 && !f_tiled) {
        int ks, half = 0;
        if (M == 1 || f_stream || ks_force > 0 || rkind == ORKH_NF4) {
            ks = ks_force > 0 ? ks_force : stream_rule_ks(c, rkind, M, KB, NB, cu);
        } else {
            /* both kernels priced, each at its best split (the streaming kernel also with half panels); the
             * streaming kernel wins ties */
            ks = 1;
            double ts = stream_us(c, rkind, M, N, KB, cu, 1, 0);
            for (int k = 1; k <= 8; k *= 2) {
                if (k > 1 && (cdiv(KB, cdiv(KB, k)) != k || cdiv(KB, k) < 4)) continue;
                for (int h = k == 1 ? 1 : 0; h <= stream_half_offered(rkind); h++) {
                    const double t = stream_us(c, rkind, M, N, KB, cu, k, h);
                    if (t >= 0 && t < ts - 1e-9) { ts = t; ks = k; half = h; }
                }
            }
            orkh_plan t2;
            memset(&t2, 0, sizeof t2);
            if (tiled2_best(rkind, M, N, KB, cu, 0, rkind == ORKH_I4U, &t2) < ts - 1e-9) {
                *q = t2;
                if (q->ksplit > 1) *ws_bytes = (size_t)q->ksplit * M * N * 4;
                return 0;
            }
        }
        /* M = 1 takes the VALU-dot GEMV (same grid and fields); ORK_PLAN=stream keeps the MFMA kernel. */
        q->algo = (M == 1 && !f_stream) ? ORKH_ALGO_GEMV : ORKH_ALGO_STREAM;
        stream_geom(c, rkind, M, KB, NB, cu, ks, q);
        if (q->algo == ORKH_ALGO_GEMV) gemv_half_geom(c, rkind, NB, cu, q);
        if (q->algo == ORKH_ALGO_STREAM) q->half = half && q->np == 1;
        const char *fh = knob(c, "ORK_STREAM_HALF"); /* testing / A-B: half panels on or off on the streaming kernel */
        if (q->algo == ORKH_ALGO_STREAM && q->np == 1 && fh) q->half = atoi(fh) != 0;
        if (q->ksplit > 1) *ws_bytes = (size_t)q->ksplit * M * N * 4;
        return 0;
    }

    /* (NF4 reaches here only with ORK_KSPLIT forced: k_tiled up to 128 rows, the LDS-ring kernel above) */
    if ((rkind != ORKH_NF4 || M > 128) && !f_tiled) {
        /* int8, fp16 and uniform int4: the per-tile fits (uniform int4 has no 256 x 256 fit: with the nibble decode
         * its registers spill, 20 B per lane); a forced split they were not timed at takes the shared model */
        if (rkind == ORKH_NF4 || mma_fit_best(rkind, M, N, KB, cu, ks_force, q) < 0)
            tiled2_best(rkind, M, N, KB, cu, ks_force, rkind == ORKH_I4U, q);
        if (q->ksplit > 1) *ws_bytes = (size_t)q->ksplit * M * N * 4;
        return 0;
    }

    /* k_tiled (NF4 up to 128 rows, or ORK_PLAN=tiled): each CU pulls its tiles' A and B rows through L2 at a roughly fixed
     * rate, so the time of a round of workgroups is about the operand bytes one workgroup loads. K is split
     * across workgroups when that cuts the per-workgroup bytes by more than the partial sums and the extra
     * reduce launch (~2 us) cost. Model units: us at ~48 KB/us per CU (measured order of magnitude),
     * 5 TB/s for the partials' HBM round trip. */
    static const int cfg[][2] = {{128, 96}, {128, 128}, {64, 64}};
    const int bpk = 64;                                                  /* B bytes per column per K-block, every kind */
    const int apk = (rkind == ORKH_I4U || rkind == ORKH_NF4) ? 128 : 64; /* A bytes per row per K-block */
    double best = -1;
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

/* Grouped-scale runs (ork_*_mm_run_grouped). The groups must close in ascending order inside one workgroup, so
 * K is never split. Few rows: k_grouped streams each 16-column panel (and re-reads A per panel). With more
 * rows, int8 and uniform int4 take the LDS-ring kernel at the unsplit 64-row tile (64x192 or 64x64) the time
 * model prices lowest, when the tile's scales fit in LDS beside its ring (else 64x64, else k_grouped):
 *   from 32 rows when every group is whole 128-k spans (G % 128 == 0: the stage runs as in the plain kernel and a
 *   group closes after the K-block that ends it; e.g. W4A4 K=N=4096 G=128: 42.9 -> 21.6 us at M=256, since 18.5
 *   with deeper stages);
 *   from 128 rows otherwise (groups can end inside K-blocks and the kernel walks them K-block by K-block).
 * NF4 stays on k_grouped (its codebook decode would repeat in every wave row).
 * ORK_PLAN=stream|tiled forces either (tests, A/B). */
#define ORKI_GROUPED_TILED_M 32
#define ORKI_GROUPED_TILED_M_PARTIAL 128
void orki_plan_grouped(const ork_npu *c, int rkind, int M, int K, int N, int KB, int G, orkh_plan *q) {
    memset(q, 0, sizeof *q);
    const int cu = (c && c->cores > 0) ? c->cores : 256;
    const char *force = knob(c, "ORK_PLAN");
    int tiled = M >= (G % 128 == 0 ? ORKI_GROUPED_TILED_M : ORKI_GROUPED_TILED_M_PARTIAL);
    if (force && !strcmp(force, "stream")) tiled = 0;
    if (force && !strcmp(force, "tiled")) tiled = 1;
    if (tiled && rkind != ORKH_NF4) {
        const char *tf = knob(c, "ORK_TILE");
        int fbm, fbn;
        if (tf && sscanf(tf, "%dx%d", &fbm, &fbn) == 2 && fbm == 64 && (fbn == 64 || fbn == 192)) {
            q->algo = ORKH_ALGO_TILED2;
            q->bm = fbm;
            q->bn = fbn;
        } else {
            tiled2_best(rkind, M, N, KB, cu, 1, 2, q); /* the 64-row tiles: the larger ones spill with the fp32 sums */
        }
        /* the tile's scales (BM x K/G and K/G x BN floats) sit in LDS beside the stage ring */
        const int Sk = K / G;
        for (int pass = 0; pass < 2 && q->algo == ORKH_ALGO_TILED2; pass++) {
            const long sc = ((long)q->bm * Sk * 4 + 1023) / 1024 * 1024 + ((long)Sk * q->bn * 4 + 1023) / 1024 * 1024;
            const int ring = orkh_tiled2_ring_lds(rkind, q->bm, q->bn);
            if (ring > 0 && ring + sc <= 163840) {
                q->ksplit = 1;
                q->kbs = KB;
                /* A stages as whole row lines where the stage row is whole lines (the kernel checks) */
                const char *fa = knob(c, "ORK_ALINE");
                q->aline = fa ? atoi(fa) != 0 : 1;
                /* write-through C stores on a grid of one round, as for the plain runs */
                const char *fc = knob(c, "ORK_CWT");
                q->cwt = fc ? atoi(fc) != 0 : (long)cdiv(M, q->bm) * cdiv(N / 16, q->bn / 16) <= cu;
                return;
            }
            if (q->bm == 64 && q->bn == 64) break;
            q->bm = 64; /* the smallest ring */
            q->bn = 64;
        }
        memset(q, 0, sizeof *q);
    }
    /* one row: the half-panel VALU kernel (k_grouped_gemv) where the groups' partials fit its LDS (K/G <= 512), runs
     * as the GEMV's (ORK_PLAN=stream keeps k_grouped). Graph-timed against k_grouped (us): W4A4 K=N=4096 G=128
     * 9.6 -> 4.4; int8 K=2048 N=6144 G=128 7.9 -> 4.7; int8 K=2048 N=16384 G=512 8.1 -> 7.5 */
    if (M == 1 && K / G <= 512 && !(force && !strcmp(force, "stream"))) {
        q->algo = ORKH_ALGO_GEMV;
        q->mt = 1;
        q->ksplit = 1;
        q->kbs = KB;
        q->half = 1;
        const int need = cdiv(KB, rkind == ORKH_NF4 ? 4 : 8);
        q->wpg = need <= 2 ? 2 : need <= 4 ? 4 : 8;
        q->kbw = cdiv(KB, q->wpg);
        return;
    }
    q->algo = ORKH_ALGO_STREAM;
    q->mt = M > 16 ? 4 : 1;
    q->ksplit = 1;
    q->kbs = KB;
}
