/* weights.c -- pack / load / dump / free of resident weights.
 *
 * Reference entry points and the behaviour kept from each:
 *   ork_i8_mm_pack        src/npu/i8/pack.c:47-57   K%32, N%32; B[K][N] int8 codes copied as-is
 *   ork_i8_mm_pack_f32    src/npu/i8/pack.c:475-494 per-channel int8 quant of f32[N][K], bscale_out
 *   ork_f16_mm_pack       src/npu.c:732-734         K%32, N%16; fp16 B[K][N] bit copy
 *   ork_i4a8_mm_pack(_im) src/npu/i4/pack.c:26-87   $ORK_NF4 / $ORK_SR, imatrix clip search, Bi4 + bscale kept
 *   ork_i4a8_w_dump       src/npu/i4/pack.c:91-103  O4N1 = hdr(20 B) + bscale[N] + Bi4[N][K/2]
 *   ork_i4a8_mm_load      src/npu/i4/pack.c:115-193 size/magic/version/K/N/kind validation
 *   ork_i4a8_pack_cpu_blob(_qerr) src/npu/i4/pack.c:794-863
 *   ork_i4_mm_pack        src/npu/i4/pack.c:435-470 K%32, N%64; int4 values [-8,7] (low nibble kept)
 *   ork_w_free / ork_mm_free / accessors  src/npu.c:1140-1212, src/npu/core/buf.c:525, :571-574
 * What changes: the resident form is the gfx950 panel layout in one hipMalloc allocation (no Bb/Bf
 * K-slices, no IOVA), and i4a8 weights stay as nibbles in HBM instead of inflating to int8 tiles. */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "internal.h"

#define O4N1_MAGIC 0x4F344E31u /* 'O','4','N','1' -- src/npu/internal.h:584 */
#define O4N1_HDR 20            /* {u32 magic, u32 version, i32 K, i32 N, u32 quant_kind} */

ork_w *orki_w_new(ork_npu *c, int K, int N, int dtype, int rkind) {
    ork_w *w = calloc(1, sizeof *w);
    if (!w) return NULL;
    w->K = K;
    w->N = N;
    w->dtype = dtype;
    w->rkind = rkind;
    w->ctx = c;
    return w;
}

/* Allocate the weight's device panels and copy `panels` (host, orki_panel_bytes) into them. */
int orki_w_upload(ork_w *w, const void *panels) {
    ork_npu *c = w->ctx;
    const size_t bytes = orki_panel_bytes(w->rkind, w->K, w->N, &w->KB);
    w->dB = orkh_malloc(bytes);
    if (!w->dB) { orki_hip_fail("weight alloc"); return -1; }
    w->dbytes = bytes;
    if (orkh_h2d(w->dB, panels, bytes, c->stream) || orkh_sync(c->stream)) {
        orki_hip_fail("weight upload");
        orkh_free(w->dB);
        w->dB = NULL;
        return -1;
    }
    return 0;
}

static void w_destroy_host(ork_w *w) {
    free(w->Bi4);
    free(w->bscale);
    free(w->codes);
    free(w);
}

void ork_w_free(ork_w *w) {
    if (!w) return;
    if (w->dB) orki_orphan(w->ctx, w->dB); /* device memory goes at ork_npu_free */
    w_destroy_host(w);
}

void ork_mm_free(ork_npu *c, ork_w *w) {
    if (!w) return;
    if (w->dB) {
        ork_npu *o = c ? c : w->ctx;
        if (o && o->stream) (void)orkh_sync(o->stream);
        if (orkh_free(w->dB)) orki_hip_fail("ork_mm_free");
    }
    w_destroy_host(w);
}

size_t ork_w_bytes(const ork_w *w) {
    if (!w) return 0;
    if (w->codes) return (size_t)w->K * w->N;
    return w->dbytes;
}

int ork_w_device_panels(const ork_w *w, const void **panels, int *KB, int *kind, uint32_t lut[4]) {
    if (!w || !w->dB) return -1;
    if (panels) *panels = w->dB;
    if (KB) *KB = w->KB;
    if (kind) *kind = w->rkind;
    if (lut) memcpy(lut, w->lut, sizeof w->lut);
    return 0;
}

void ork_w_dims(const ork_w *w, int *K, int *N) {
    if (K) *K = w ? w->K : 0;
    if (N) *N = w ? w->N : 0;
}
int ork_w_quant_kind(const ork_w *w) { return w ? w->quant_kind : -1; }
const float *ork_w_bscale(const ork_w *w) { return w ? w->bscale : NULL; }
const int8_t *ork_w_codes(const ork_w *w) { return w ? w->codes : NULL; }

/* Offline weights keep their codes [K][N] on the host for inspection (ork_w_codes); nothing runs them. */
static ork_w *offline_codes(ork_npu *c, int K, int N, int dtype, const int8_t *codes_kn, const int8_t *codes_nk) {
    ork_w *w = orki_w_new(c, K, N, dtype, -1);
    if (!w) return NULL;
    w->codes = malloc((size_t)K * N);
    if (!w->codes) { free(w); return NULL; }
    if (codes_kn) memcpy(w->codes, codes_kn, (size_t)K * N);
    else
        for (int n = 0; n < N; n++)
            for (int k = 0; k < K; k++) w->codes[(size_t)k * N + n] = codes_nk[(size_t)n * K + k];
    return w;
}

/* ---- int8 ------------------------------------------------------------------------------------------ */
ork_w *ork_i8_mm_pack(ork_npu *c, int K, int N, const int8_t *B) {
    if (!c || !B || K <= 0 || N <= 0 || K % 32 || N % 32) return NULL;
    if (c->offline) return offline_codes(c, K, N, DT_I8, B, NULL);
    ork_w *w = orki_w_new(c, K, N, DT_I8, ORKH_I8);
    if (!w) return NULL;
    int KB;
    uint8_t *pan = malloc(orki_panel_bytes(ORKH_I8, K, N, &KB));
    if (!pan) { free(w); return NULL; }
    orki_tile_i8_kn(B, K, N, KB, pan);
    const int rc = orki_w_upload(w, pan);
    free(pan);
    if (rc) { free(w); return NULL; }
    return w;
}

ork_w *ork_i8_mm_pack_f32(ork_npu *c, int K, int N, const float *f32, float *bscale_out) {
    if (!c || !f32 || K <= 0 || N <= 0 || K % 32 || N % 32) return NULL;
    int8_t *codes = malloc((size_t)K * N);
    float *bs = malloc((size_t)N * sizeof(float));
    if (!codes || !bs) { free(codes); free(bs); return NULL; }
    orki_i8_quant_chans(f32, K, N, bs, codes);
    if (bscale_out) memcpy(bscale_out, bs, (size_t)N * sizeof(float));
    free(bs);
    ork_w *w = NULL;
    if (c->offline) {
        w = offline_codes(c, K, N, DT_I8, NULL, codes);
    } else if ((w = orki_w_new(c, K, N, DT_I8, ORKH_I8))) {
        int KB;
        uint8_t *pan = malloc(orki_panel_bytes(ORKH_I8, K, N, &KB));
        if (pan) orki_tile_i8_nk(codes, K, N, KB, pan);
        if (!pan || orki_w_upload(w, pan)) { free(w); w = NULL; }
        free(pan);
    }
    free(codes);
    return w;
}

/* ---- fp16 ------------------------------------------------------------------------------------------ */
ork_w *ork_f16_mm_pack(ork_npu *c, int K, int N, const ork_f16 *B) {
    if (!c || !B || K <= 0 || N <= 0 || K % 32 || N % 16) return NULL;
    if (orki_need_device(c, "ork_f16_mm_pack")) return NULL;
    ork_w *w = orki_w_new(c, K, N, DT_F16, ORKH_F16);
    if (!w) return NULL;
    int KB;
    uint8_t *pan = malloc(orki_panel_bytes(ORKH_F16, K, N, &KB));
    if (!pan) { free(w); return NULL; }
    orki_tile_f16_kn((const uint16_t *)B, K, N, KB, pan);
    const int rc = orki_w_upload(w, pan);
    free(pan);
    if (rc) { free(w); return NULL; }
    return w;
}

/* ---- int4 store (i4a8) --------------------------------------------------------------------------- */
static void nf4_lut_words(uint32_t out[4]) {
    int8_t lut[16];
    orki_nf4_lut(lut);
    for (int i = 0; i < 4; i++)
        out[i] = (uint32_t)(uint8_t)lut[4 * i] | (uint32_t)(uint8_t)lut[4 * i + 1] << 8 |
                 (uint32_t)(uint8_t)lut[4 * i + 2] << 16 | (uint32_t)(uint8_t)lut[4 * i + 3] << 24;
}

/* int8 codes [K][N] of a compact store (uniform: sign-extended nibble; NF4: codebook value). */
static void inflate_store(int K, int N, int kind, const uint8_t *nib, int8_t *codes_kn) {
    int8_t lut[16];
    orki_nf4_lut(lut);
    for (int n = 0; n < N; n++) {
        const uint8_t *nb = nib + (size_t)n * (K / 2);
        for (int k = 0; k < K; k++) {
            const unsigned ix = (k & 1) ? (nb[k >> 1] >> 4) : (nb[k >> 1] & 0xf);
            codes_kn[(size_t)k * N + n] = kind == ORK_QK_CODEBOOK_NF4 ? lut[ix] : (int8_t)(ix >= 8 ? (int)ix - 16 : (int)ix);
        }
    }
}

/* Build a weight around an already-quantised compact store (takes ownership of nib and bscale). */
static ork_w *i4a8_from_store(ork_npu *c, int K, int N, int kind, uint8_t *nib, float *bscale) {
    ork_w *w = NULL;
    if (c->offline) {
        int8_t *codes = malloc((size_t)K * N);
        if (codes) {
            inflate_store(K, N, kind, nib, codes);
            w = offline_codes(c, K, N, DT_I8, codes, NULL);
        }
        free(codes);
    } else {
        const int rk = kind == ORK_QK_CODEBOOK_NF4 ? ORKH_NF4 : ORKH_I4U;
        w = orki_w_new(c, K, N, DT_I8, rk);
        if (w) {
            int KB;
            uint8_t *pan = malloc(orki_panel_bytes(rk, K, N, &KB));
            /* pad k >= K with the code that inflates to 0: nibble 0 (uniform) / index 7 (NF4 level 0.0) */
            if (pan) orki_tile_nib_nk(nib, K, N, KB, rk == ORKH_NF4 ? 7 : 0, pan);
            if (!pan || orki_w_upload(w, pan)) { free(w); w = NULL; }
            free(pan);
            if (w && rk == ORKH_NF4) nf4_lut_words(w->lut);
        }
    }
    if (!w) { free(nib); free(bscale); return NULL; }
    w->quant_kind = kind;
    w->Bi4 = nib;
    w->bscale = bscale;
    return w;
}

ork_w *ork_i4a8_mm_pack_im(ork_npu *c, int K, int N, const float *f32, const float *imatrix, float *bscale_out) {
    if (!c || !f32 || K <= 0 || N <= 0 || K % 32 || N % 32) return NULL;
    const int sr = getenv("ORK_SR") != NULL;
    const int nf4 = getenv("ORK_NF4") != NULL;
    uint8_t *nib = malloc((size_t)N * (K / 2));
    float *bs = malloc((size_t)N * sizeof(float));
    if (!nib || !bs || orki_i4a8_quant(K, N, f32, imatrix, nf4, sr, bs, nib, NULL)) {
        free(nib);
        free(bs);
        return NULL;
    }
    if (bscale_out) memcpy(bscale_out, bs, (size_t)N * sizeof(float));
    return i4a8_from_store(c, K, N, nf4 ? ORK_QK_CODEBOOK_NF4 : ORK_QK_UNIFORM, nib, bs);
}

ork_w *ork_i4a8_mm_pack(ork_npu *c, int K, int N, const float *f32, float *bscale_out) {
    return ork_i4a8_mm_pack_im(c, K, N, f32, NULL, bscale_out);
}

size_t ork_i4a8_w_dump(const ork_w *w, void *out, size_t cap) {
    if (!w || !w->Bi4 || !w->bscale) return 0;
    const size_t sc = (size_t)w->N * sizeof(float), nib = (size_t)w->K * w->N / 2;
    const size_t need = O4N1_HDR + sc + nib;
    if (!out) return need;
    if (cap < need) return 0;
    const uint32_t h[5] = {O4N1_MAGIC, ork_pack_format_version(), (uint32_t)w->K, (uint32_t)w->N, (uint32_t)w->quant_kind};
    uint8_t *p = out;
    memcpy(p, h, O4N1_HDR);
    memcpy(p + O4N1_HDR, w->bscale, sc);
    memcpy(p + O4N1_HDR + sc, w->Bi4, nib);
    return need;
}

ork_w *ork_i4a8_mm_load(ork_npu *c, int K, int N, const void *blob, size_t n) {
    if (!c || !blob || K <= 0 || N <= 0 || K % 32 || N % 32) return NULL;
    const size_t sc = (size_t)N * sizeof(float), nibsz = (size_t)K * N / 2;
    if (n != O4N1_HDR + sc + nibsz) return NULL;
    uint32_t h[5];
    memcpy(h, blob, O4N1_HDR);
    if (h[0] != O4N1_MAGIC || h[1] != ork_pack_format_version() || (int32_t)h[2] != K || (int32_t)h[3] != N) return NULL;
    if (h[4] != ORK_QK_UNIFORM && h[4] != ORK_QK_CODEBOOK_NF4) return NULL;
    float *bs = malloc(sc);
    uint8_t *nib = malloc(nibsz);
    if (!bs || !nib) { free(bs); free(nib); return NULL; }
    memcpy(bs, (const uint8_t *)blob + O4N1_HDR, sc);
    memcpy(nib, (const uint8_t *)blob + O4N1_HDR + sc, nibsz);
    return i4a8_from_store(c, K, N, (int)h[4], nib, bs);
}

size_t ork_i4a8_pack_cpu_blob_qerr(ork_npu *c, int K, int N, const float *f32, const float *imatrix, int nf4,
                                   void *out, size_t cap, float *qerr_out) {
    (void)c;
    if (K <= 0 || N <= 0 || K % 32 || N % 32 || !f32) return 0;
    const size_t sc = (size_t)N * sizeof(float), nibsz = (size_t)K * N / 2, need = O4N1_HDR + sc + nibsz;
    if (!out) return need;
    if (cap < need) return 0;
    nf4 = nf4 ? 1 : 0;
    const int sr = getenv("ORK_SR") != NULL;
    uint8_t *p = out;
    float *bs = malloc(sc);
    int8_t *codes = qerr_out ? malloc((size_t)K * N) : NULL;
    if (!bs || (qerr_out && !codes)) { free(bs); free(codes); return 0; }
    if (orki_i4a8_quant(K, N, f32, imatrix, nf4, sr, bs, p + O4N1_HDR + sc, codes)) { free(bs); free(codes); return 0; }
    if (qerr_out) {
        /* qerr = sqrt(sum imp*(w - code*bscale)^2 / sum imp*w^2) in double, channel then k order
         * (src/npu/i4/pack.c:840-856) */
        double qnum = 0.0, qden = 0.0;
        for (int nn = 0; nn < N; nn++) {
            const float *fr = f32 + (size_t)nn * K;
            const float b = bs[nn];
            for (int k = 0; k < K; k++) {
                const double w = fr[k], q = (double)(float)codes[(size_t)nn * K + k] * b, d = w - q;
                const double imp = imatrix ? imatrix[k] : 1.0;
                qnum += imp * d * d;
                qden += imp * w * w;
            }
        }
        *qerr_out = qden > 0.0 ? (float)sqrt(qnum / qden) : 0.0f;
    }
    const uint32_t h[5] = {O4N1_MAGIC, ork_pack_format_version(), (uint32_t)K, (uint32_t)N,
                           (uint32_t)(nf4 ? ORK_QK_CODEBOOK_NF4 : ORK_QK_UNIFORM)};
    memcpy(p + O4N1_HDR, bs, sc);
    memcpy(p, h, O4N1_HDR);
    free(bs);
    free(codes);
    return need;
}

size_t ork_i4a8_pack_cpu_blob(ork_npu *c, int K, int N, const float *f32, const float *imatrix, int nf4, void *out, size_t cap) {
    return ork_i4a8_pack_cpu_blob_qerr(c, K, N, f32, imatrix, nf4, out, cap, NULL);
}

/* ---- W4A4 ------------------------------------------------------------------------------------------ */
ork_w *ork_i4_mm_pack(ork_npu *c, int K, int N, const int8_t *B) {
    if (!c || !B || K <= 0 || N <= 0 || K % 32 || N % 64) return NULL;
    if (c->offline) return offline_codes(c, K, N, DT_I4, B, NULL);
    ork_w *w = orki_w_new(c, K, N, DT_I4, ORKH_I4U);
    if (!w) return NULL;
    int KB;
    uint8_t *pan = malloc(orki_panel_bytes(ORKH_I4U, K, N, &KB));
    if (!pan) { free(w); return NULL; }
    orki_tile_nib_kn(B, K, N, KB, pan);
    const int rc = orki_w_upload(w, pan);
    free(pan);
    if (rc) { free(w); return NULL; }
    return w;
}

/* ---- grouped scales ---------------------------------------------------------------------------------
 * ork_i4_mm_pack_grouped (src/npu/i4/pack.c:686-700): the W4A4 pack plus a K-group size (K%32, N%64, G%32,
 * K%G, G <= 10752). ork_w_set_group (src/npu.c:1191-1200): int4 or int8 weights, K%G. The group size
 * only selects the scale layout of the grouped runs; the resident panels are the same as ungrouped. */
ork_w *ork_i4_mm_pack_grouped(ork_npu *c, int K, int N, const int8_t *B, int G) {
    if (!c || !B || K <= 0 || N <= 0 || K % 32 || N % 64 || G <= 0 || G % 32 || K % G || G > 10752) return NULL;
    ork_w *w = ork_i4_mm_pack(c, K, N, B);
    if (w) w->gsize = G;
    return w;
}

int ork_w_set_group(ork_w *w, int G) {
    if (!w || (w->dtype != DT_I4 && w->dtype != DT_I8)) return -1;
    if (G > 0 && w->K % G) return -1;
    w->gsize = G > 0 ? G : 0;
    return 0;
}
