/* persist.c -- persisted weights: the 4 KiB 'OAPK' header, ork_w_dump, the CPU dumpers and the loaders.
 *
 * Reference: the header and its refusal rules (include/ork/weights.h:159-198, src/npu/core/packhdr.c:48-118),
 * ork_w_dump (src/npu.c:760-774), ork_i8_w_dump_cpu / ork_i8_mm_load (src/npu/i8/pack.c:128-224),
 * ork_i4_w_dump_cpu / ork_i4_mm_load (src/npu/i4/pack.c:489-558), ork_f16_mm_load (src/npu/f16/pack.c:110-123).
 *
 * Kept: the header struct and its size (one 4 KiB page), magic 'OAPK', the fields and their order, the
 * distinct refusal causes (short / unstamped / format / caps / shape) each reported once, "out = NULL ->
 * size", loaders that refuse before reading a payload byte, offline loads that recover the exact codes
 * (ork_w_codes), i4a8 weights dumping as plain int8 (dtype I8), and CPU dumpers byte-identical to
 * pack + dump.
 * What changes: the payload is this build's resident panel layout (../hip/orkh.h), one contiguous run of
 * 1 KiB blocks, not page-padded NPU tiles; the caps identity hashes that layout's geometry and "gfx950",
 * so packs tiled for another chip (the reference's RK tiles included) are refused as foreign caps. There is
 * no Bf (full-K re-tile) and no dma-buf import: ork_i8_w_dump_bf_cpu returns 0 (the reference's "no Bf for
 * this weight") and the _import loaders return NULL (the reference's "import unavailable", on which its
 * callers fall back to the plain loader). */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "internal.h"

/* Bump when the meaning of the geometry changes, so older packs stop matching even on the same chip. */
#define PACK_CAPS_RULE 1u
#define PACK_SOC "gfx950"

/* FNV-1a over the layout's defining constants: the caps rule, the pack format version, the panel
 * geometry (16 columns per panel, 1 KiB blocks, K per block for int8 / fp16 / nibble panels), the SoC id. */
static uint32_t pack_capid(void) {
    uint32_t h = 2166136261u;
    const uint32_t v[] = {PACK_CAPS_RULE, ork_pack_format_version(), 16u, 1024u, 64u, 32u, 128u};
    for (size_t i = 0; i < sizeof v / sizeof v[0]; i++)
        for (int b = 0; b < 4; b++) {
            h ^= (v[i] >> (8 * b)) & 0xffu;
            h *= 16777619u;
        }
    for (const char *p = PACK_SOC; *p; p++) {
        h ^= (unsigned char)*p;
        h *= 16777619u;
    }
    return h ? h : 1u; /* 0 means "unstamped" */
}

size_t ork_pack_hdr_bytes(void) { return ORK_PACK_HDR_BYTES; }

static void pack_stamp(void *out, int dtype, int K, int N) {
    memset(out, 0, ORK_PACK_HDR_BYTES); /* a reproducible blob: the pad is zero */
    ork_pack_hdr h;
    memset(&h, 0, sizeof h);
    h.magic = ORK_PACK_MAGIC;
    h.fmt = ork_pack_format_version();
    h.capid = pack_capid();
    h.dtype = (uint32_t)dtype;
    h.K = K;
    h.N = N;
    h.hdr_bytes = ORK_PACK_HDR_BYTES;
    snprintf(h.soc, sizeof h.soc, "%s", PACK_SOC);
    memcpy(out, &h, sizeof h);
}

/* 0 when the blob's header matches this build and the request; else an ORK_PACKERR_* cause. */
static int pack_check(const void *blob, size_t n, int dtype, int K, int N) {
    static int said_unstamped, said_fmt, said_caps;
    if (!blob || n < ORK_PACK_HDR_BYTES) return ORK_PACKERR_SHORT;
    ork_pack_hdr h;
    memcpy(&h, blob, sizeof h);
    if (h.magic != ORK_PACK_MAGIC) {
        if (!said_unstamped++)
            orki_err("refusing an UNSTAMPED persisted weight (no 'OAPK' header): it predates the pack header "
                     "or was not written by ork_w_dump / ork_*_w_dump_cpu. Rebuild the pack.");
        return ORK_PACKERR_UNSTAMPED;
    }
    if (h.fmt != ork_pack_format_version()) {
        if (!said_fmt++)
            orki_err("refusing a persisted weight from pack format %u (this build writes %u): the layout "
                     "changed. Rebuild the pack.", h.fmt, ork_pack_format_version());
        return ORK_PACKERR_FORMAT;
    }
    if (h.capid != pack_capid()) {
        char soc[sizeof h.soc + 1];
        memcpy(soc, h.soc, sizeof h.soc);
        soc[sizeof h.soc] = 0;
        if (!said_caps++)
            orki_err("refusing a persisted weight built for different caps (pack soc='%s' capid=%08x, this "
                     "build soc='%s' capid=%08x): its tiles follow another layout. Rebuild the pack here.",
                     soc, h.capid, PACK_SOC, pack_capid());
        return ORK_PACKERR_CAPS;
    }
    if (h.hdr_bytes != ORK_PACK_HDR_BYTES) return ORK_PACKERR_FORMAT;
    if ((int)h.dtype != dtype || h.K != K || h.N != N) return ORK_PACKERR_SHAPE;
    return 0;
}

/* ---- panel -> codes (offline loads): the exact inverses of panel.c's tilers ---- */
static void untile_i8(const uint8_t *pan, int K, int N, int KB, int8_t *B_kn) {
    for (int k = 0; k < K; k++)
        for (int n = 0; n < N; n++) {
            const uint8_t *blk = pan + ((size_t)(n / 16) * KB + k / 64) * 1024;
            B_kn[(size_t)k * N + n] = (int8_t)blk[(((k % 64) / 16) * 16 + n % 16) * 16 + k % 16];
        }
}

static void untile_nib(const uint8_t *pan, int K, int N, int KB, int8_t *B_kn) {
    for (int k = 0; k < K; k++) {
        const int r = k % 128, g = r / 32, q = r % 32, d = q / 8, w = q % 8, b = w % 4, hi = w / 4;
        for (int n = 0; n < N; n++) {
            const uint8_t *blk = pan + ((size_t)(n / 16) * KB + k / 128) * 1024;
            const unsigned v = (blk[(g * 16 + n % 16) * 16 + d * 4 + b] >> (hi * 4)) & 0xf;
            B_kn[(size_t)k * N + n] = (int8_t)(v >= 8 ? (int)v - 16 : (int)v); /* sign-extend, as the reference */
        }
    }
}

static int8_t *codes_of_store(const ork_w *w) { /* int8 codes [K][N] of an i4a8 weight's compact store */
    int8_t *codes = malloc((size_t)w->K * w->N);
    if (!codes) return NULL;
    int8_t lut[16];
    orki_nf4_lut(lut);
    for (int n = 0; n < w->N; n++) {
        const uint8_t *nb = w->Bi4 + (size_t)n * (w->K / 2);
        for (int k = 0; k < w->K; k++) {
            const unsigned ix = (k & 1) ? (nb[k >> 1] >> 4) : (nb[k >> 1] & 0xf);
            codes[(size_t)k * w->N + n] = w->quant_kind == ORK_QK_CODEBOOK_NF4 ? lut[ix]
                                                                             : (int8_t)(ix >= 8 ? (int)ix - 16 : (int)ix);
        }
    }
    return codes;
}

/* ---- dumps ---- */
static size_t dump_tiled(int dtype, int rkind, int K, int N, const int8_t *B_kn, void *out, size_t cap) {
    int KB;
    const size_t body = orki_panel_bytes(rkind, K, N, &KB), need = ORK_PACK_HDR_BYTES + body;
    if (!out) return need;
    if (cap < need) return 0;
    pack_stamp(out, dtype, K, N);
    uint8_t *pan = (uint8_t *)out + ORK_PACK_HDR_BYTES;
    if (rkind == ORKH_I8) orki_tile_i8_kn(B_kn, K, N, KB, pan);
    else orki_tile_nib_kn(B_kn, K, N, KB, pan);
    return need;
}

size_t ork_i8_w_dump_cpu(ork_npu *c, int K, int N, const int8_t *B, void *out, size_t cap) {
    if (!c || !B || K <= 0 || N <= 0 || K % 32 || N % 32) return 0;
    return dump_tiled(DT_I8, ORKH_I8, K, N, B, out, cap);
}

size_t ork_i4_w_dump_cpu(ork_npu *c, int K, int N, const int8_t *B, void *out, size_t cap) {
    if (!c || !B || K <= 0 || N <= 0 || K % 32 || N % 64) return 0;
    return dump_tiled(DT_I4, ORKH_I4U, K, N, B, out, cap);
}

size_t ork_i8_w_dump_bf_cpu(ork_npu *c, int K, int N, const int8_t *B, void *out, size_t cap) {
    (void)c, (void)K, (void)N, (void)B, (void)out, (void)cap;
    return 0; /* the panel layout serves every run; there is no separate full-K copy to persist */
}

size_t ork_w_dump(const ork_w *w, void *out, size_t cap) {
    if (!w) return 0;
    if (w->codes) /* offline weight: tile its codes, byte-identical to what a device pack would dump */
        return w->dtype == DT_I4 ? dump_tiled(DT_I4, ORKH_I4U, w->K, w->N, w->codes, out, cap)
                                 : dump_tiled(DT_I8, ORKH_I8, w->K, w->N, w->codes, out, cap);
    if (w->Bi4 && (w->rkind == ORKH_I4U || w->rkind == ORKH_NF4) && w->dtype == DT_I8) {
        /* i4a8: the int8 codes the weight multiplies with, as a plain int8 pack */
        if (!out) return ORK_PACK_HDR_BYTES + orki_panel_bytes(ORKH_I8, w->K, w->N, NULL);
        int8_t *codes = codes_of_store(w);
        if (!codes) return 0;
        const size_t r = dump_tiled(DT_I8, ORKH_I8, w->K, w->N, codes, out, cap);
        free(codes);
        return r;
    }
    if (!w->dB) return 0;
    /* the stamp names the payload's layout: W4A4 nibble panels load back through ork_i4_mm_load or
     * ork_i4a8_mm_load_tiled, whichever entry point the weight ran through */
    const int dt = w->rkind == ORKH_F16 ? DT_F16 : w->rkind == ORKH_I8 ? DT_I8 : w->rkind == ORKH_I4U ? DT_I4 : -1;
    if (dt < 0) return 0;
    const size_t need = ORK_PACK_HDR_BYTES + w->dbytes;
    if (!out) return need;
    if (cap < need) return 0;
    ork_npu *c = w->ctx;
    if (orkh_d2h((uint8_t *)out + ORK_PACK_HDR_BYTES, w->dB, w->dbytes, c->stream) || orkh_sync(c->stream)) {
        orki_hip_fail("ork_w_dump");
        return 0;
    }
    pack_stamp(out, dt, w->K, w->N);
    return need;
}

/* ---- loads ---- */
static ork_w *load_common(const char *who, ork_npu *c, int K, int N, int dtype, int rkind, const void *blob, size_t n) {
    if (!c || K <= 0 || N <= 0 || K % 32) return NULL;
    if (pack_check(blob, n, dtype, K, N)) return NULL;
    int KB;
    const size_t body = orki_panel_bytes(rkind, K, N, &KB);
    if (n != ORK_PACK_HDR_BYTES + body) {
        orki_err("%s: payload is %zu bytes, a %dx%d weight needs %zu", who, n - ORK_PACK_HDR_BYTES, K, N, body);
        return NULL;
    }
    const uint8_t *pan = (const uint8_t *)blob + ORK_PACK_HDR_BYTES;
    if (c->offline) {
        if (rkind == ORKH_F16) {
            orki_err("%s: offline context has no device (fp16 weights live only in HBM here)", who);
            return NULL;
        }
        ork_w *w = orki_w_new(c, K, N, dtype, -1);
        if (!w) return NULL;
        w->codes = malloc((size_t)K * N);
        if (!w->codes) { free(w); return NULL; }
        if (rkind == ORKH_I8) untile_i8(pan, K, N, KB, w->codes);
        else untile_nib(pan, K, N, KB, w->codes);
        return w;
    }
    ork_w *w = orki_w_new(c, K, N, dtype, rkind);
    if (!w) return NULL;
    if (orki_w_upload(w, pan)) { free(w); return NULL; }
    return w;
}

ork_w *ork_i8_mm_load(ork_npu *c, int K, int N, const void *blob, size_t n) {
    if (N % 32) return NULL;
    return load_common("ork_i8_mm_load", c, K, N, DT_I8, ORKH_I8, blob, n);
}

ork_w *ork_i4_mm_load(ork_npu *c, int K, int N, const void *blob, size_t n) {
    if (N % 64) return NULL;
    return load_common("ork_i4_mm_load", c, K, N, DT_I4, ORKH_I4U, blob, n);
}

ork_w *ork_f16_mm_load(ork_npu *c, int K, int N, const void *blob, size_t n) {
    if (N % 16) return NULL;
    return load_common("ork_f16_mm_load", c, K, N, DT_F16, ORKH_F16, blob, n);
}

ork_w *ork_i8_mm_load_import(ork_npu *c, int K, int N, const void *blob, size_t n) {
    (void)c, (void)K, (void)N, (void)blob, (void)n;
    return NULL; /* no dma-buf import here: callers fall back to ork_i8_mm_load */
}

ork_w *ork_f16_mm_load_import(ork_npu *c, int K, int N, const void *blob, size_t n) {
    (void)c, (void)K, (void)N, (void)blob, (void)n;
    return NULL; /* no dma-buf import here: callers fall back to ork_f16_mm_load */
}

/* reference include/ork/weights.h:231-235: a W4A4 pack (the tiled int4 blob ork_w_dump writes) loaded as
 * an int8-computed weight: its int4 values are the codes ork_i8_mm_run multiplies with, and G (0: none)
 * is the group size for ork_i8_mm_run_grouped. Scales come from the caller. */
ork_w *ork_i4a8_mm_load_tiled(ork_npu *c, int K, int N, const void *blob, size_t n, int G) {
    if (N % 64 || G < 0 || (G > 0 && K % G)) return NULL;
    ork_w *w = load_common("ork_i4a8_mm_load_tiled", c, K, N, DT_I4, ORKH_I4U, blob, n);
    if (!w) return NULL;
    w->dtype = DT_I8; /* runs through the int8 entry points */
    w->gsize = G;
    return w;
}
