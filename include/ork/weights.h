/* ork/weights.h -- resident weights: pack, load, dump, free, accessors (MI355X build).
 * Part of <ork_npu.h>. Packs copy B; the resident form lives in HBM in this build's panel layout
 * (not the reference's NPU tiles). Packs return NULL on bad dims or allocation failure. */
#ifndef ORK_WEIGHTS_H
#define ORK_WEIGHTS_H

/* reference include/ork/weights.h:39. B[K][N] row-major fp16. K%32, N%16. */
ork_w       *ork_f16_mm_pack(ork_npu *ctx, int K, int N, const ork_f16 *B);
/* reference include/ork/weights.h:47. B[K][N] row-major int8. K%32, N%32. */
ork_w       *ork_i8_mm_pack(ork_npu *ctx, int K, int N, const int8_t *B);
/* reference include/ork/weights.h:92. f32[N][K] (n-major); per-output-channel symmetric int8:
 * mx = max(1e-9, max|w|), q = clamp(rint(w * (127/mx)), -127, 127), bscale_out[n] = mx/127 (nullable). */
ork_w       *ork_i8_mm_pack_f32(ork_npu *ctx, int K, int N, const float *f32, float *bscale_out);

/* reference include/ork/weights.h:115 */
enum { ORK_QK_UNIFORM = 0, ORK_QK_CODEBOOK_NF4 = 1 };
/* reference include/ork/weights.h:116 and :124. "Effective w4a8": int4 codes per output channel
 * (uniform: scale = mx/7, q in [-7,7]; NF4 codebook with $ORK_NF4, bscale = mx/127), optional imatrix
 * clip-grid scale search, stochastic rounding with $ORK_SR. The nibbles stay resident (K*N/2 bytes of
 * HBM) and are inflated to int8 inside the kernels. Runs via ork_i8_mm_run. K%32, N%32. */
ork_w       *ork_i4a8_mm_pack(ork_npu *ctx, int K, int N, const float *f32, float *bscale_out);
ork_w       *ork_i4a8_mm_pack_im(ork_npu *ctx, int K, int N, const float *f32, const float *imatrix, float *bscale_out);
/* reference include/ork/weights.h:125. W4A4: B[K][N] int4 values [-8,7] in int8 containers. K%32, N%64. */
ork_w       *ork_i4_mm_pack(ork_npu *ctx, int K, int N, const int8_t *B);

/* Grouped scales. reference include/ork/weights.h:126-128: int4 weights whose scales are per (K-group of
 * G, channel), for ork_i4_mm_run_grouped. K%32, N%64, G%32, K%G, G <= 10752. */
ork_w       *ork_i4_mm_pack_grouped(ork_npu *ctx, int K, int N, const int8_t *B, int G);
/* reference include/ork/weights.h:129-132: set the group size of an int4 or int8 weight (K%G; G <= 0 clears
 * it). 0, or -1 if w is neither. */
int          ork_w_set_group(ork_w *w, int G);
/* reference include/ork/weights.h:231-235: a W4A4 pack (ork_w_dump / ork_i4_w_dump_cpu of an int4 weight)
 * loaded as an int8-computed weight with group size G (0: none); scales come from the caller. */
ork_w       *ork_i4a8_mm_load_tiled(ork_npu *c, int K, int N, const void *blob, size_t n, int G);
/* reference include/ork/weights.h:250-253: C f32[M][N] from int8 A, per-(row, group) aScale[m*(K/G)+g] and
 * per-(group, channel) bScale[g*N+n]; the int32 partial of each K-group is scaled and summed in ascending g,
 * bit-identical to the reference's CPU accumulate. G % 32 on the device (else -3). */
int          ork_i8_mm_run_grouped(ork_npu *c, ork_w *w, int M, const int8_t *A, const float *aScale,
                                   const float *bScale, float *C);

/* reference include/ork/weights.h:141. Frees the handle; its device memory is reclaimed at
 * ork_npu_free (as in the reference, where device buffers go at context teardown). */
void         ork_w_free(ork_w *w);
/* reference include/ork/weights.h:149. Frees the handle and its device memory now. */
void         ork_mm_free(ork_npu *ctx, ork_w *w);
/* reference include/ork/weights.h:150. Resident device bytes. */
size_t       ork_w_bytes(const ork_w *w);
/* reference include/ork/weights.h:154-158 */
void         ork_w_dims(const ork_w *w, int *K, int *N);
int          ork_w_quant_kind(const ork_w *w);
const float *ork_w_bscale(const ork_w *w);
/* reference include/ork/weights.h:240. Host codes [K][N] of an OFFLINE weight; NULL when resident. */
const int8_t *ork_w_codes(const ork_w *w);

/* Persisted weights (.orkpack). Reference include/ork/weights.h:159-193: every ork_w_dump /
 * ork_*_w_dump_cpu blob starts with this one-page header and every ork_*_mm_load refuses a blob that
 * lacks it or whose stamp disagrees with this build. The payload after it is this build's resident
 * panel layout, so capid names gfx950 and that geometry: packs tiled for another chip are refused. */
#define ORK_PACK_MAGIC      0x4b50414fu /* "OAPK" */
#define ORK_PACK_HDR_BYTES  4096u
typedef struct {
    uint32_t magic;     /* ORK_PACK_MAGIC */
    uint32_t fmt;       /* ork_pack_format_version() at dump time */
    uint32_t capid;     /* identity of the layout's caps: SoC + panel geometry + rule */
    uint32_t dtype;     /* ORK_DT_* of the packed weight */
    int32_t  K, N;
    uint32_t hdr_bytes; /* == ORK_PACK_HDR_BYTES */
    uint32_t flags;     /* reserved, 0 */
    char     soc[16];   /* SoC id at dump time, for the diagnostic */
} ork_pack_hdr;         /* zero-padded to ORK_PACK_HDR_BYTES */
/* Load refusal causes, reference include/ork/weights.h:189-193 (loaders return NULL and log the cause). */
#define ORK_PACKERR_SHORT     (-1) /* blob smaller than the header */
#define ORK_PACKERR_UNSTAMPED (-2) /* no magic */
#define ORK_PACKERR_FORMAT    (-3) /* different pack format */
#define ORK_PACKERR_CAPS      (-4) /* built for other caps (another chip's tile layout) */
#define ORK_PACKERR_SHAPE     (-5) /* header disagrees with the requested dtype/K/N */
/* reference include/ork/weights.h:194 */
size_t       ork_pack_hdr_bytes(void);
/* reference include/ork/weights.h:198. Header + the resident panels (int8 / fp16 / W4A4 nibbles; an i4a8
 * weight dumps the int8 codes it multiplies with, dtype I8). out=NULL -> size; 0 if cap is too small. */
size_t       ork_w_dump(const ork_w *w, void *out, size_t cap);
/* reference include/ork/weights.h:203. The bytes of ork_i8_mm_pack + ork_w_dump, tiled on the host. K%32, N%32. */
size_t       ork_i8_w_dump_cpu(ork_npu *ctx, int K, int N, const int8_t *B, void *out, size_t cap);
/* reference include/ork/weights.h:206. 0: the panel layout has no separate full-K copy to persist. */
size_t       ork_i8_w_dump_bf_cpu(ork_npu *ctx, int K, int N, const int8_t *B, void *out, size_t cap);
/* reference include/ork/weights.h:212. W4A4 twin of ork_i8_w_dump_cpu. K%32, N%64. */
size_t       ork_i4_w_dump_cpu(ork_npu *ctx, int K, int N, const int8_t *B, void *out, size_t cap);
/* reference include/ork/weights.h:219, :222, :265. NULL on a refused
 * header or a payload of the wrong size. On an offline context the int8 / W4A4 loaders recover the codes
 * (ork_w_codes); fp16 needs a device. */
ork_w       *ork_f16_mm_load(ork_npu *ctx, int K, int N, const void *blob, size_t n);
ork_w       *ork_i8_mm_load(ork_npu *ctx, int K, int N, const void *blob, size_t n);
ork_w       *ork_i4_mm_load(ork_npu *ctx, int K, int N, const void *blob, size_t n);
/* reference include/ork/weights.h:220, :17. NULL: no dma-buf import in this build
 * (the reference's "import unavailable"; callers fall back to the plain loader). */
ork_w       *ork_f16_mm_load_import(ork_npu *ctx, int K, int N, const void *blob, size_t n);
ork_w       *ork_i8_mm_load_import(ork_npu *ctx, int K, int N, const void *blob, size_t n);

/* reference include/ork/weights.h:230. O4N1 blob: {u32 'O4N1', u32 version, i32 K, i32 N,
 * u32 quant_kind} + f32 bscale[N] + nibbles[N][K/2] (low nibble = even k). out=NULL -> size;
 * 0 if cap is too small or w has no int4 store. */
size_t       ork_i4a8_w_dump(const ork_w *w, void *out, size_t cap);
/* reference include/ork/weights.h:255. NULL on a malformed blob or shape mismatch. */
ork_w       *ork_i4a8_mm_load(ork_npu *ctx, int K, int N, const void *blob, size_t n);
/* reference include/ork/weights.h:288 and :294. CPU-only pack straight to an O4N1 blob, byte-identical
 * to ork_i4a8_mm_pack_im + ork_i4a8_w_dump (nf4 explicit, $ORK_SR honoured). qerr =
 * sqrt(sum imp*(w-q)^2 / sum imp*w^2). Works on an offline context. */
size_t       ork_i4a8_pack_cpu_blob(ork_npu *ctx, int K, int N, const float *f32, const float *imatrix, int nf4, void *out, size_t cap);
size_t       ork_i4a8_pack_cpu_blob_qerr(ork_npu *ctx, int K, int N, const float *f32, const float *imatrix, int nf4, void *out, size_t cap, float *qerr_out);

/* reference include/ork/weights.h:345. A[M][K] fp16, C[M][N] fp32 (caller-allocated). 0 / negative. */
int          ork_f16_mm_run(ork_npu *ctx, ork_w *w, int M, const ork_f16 *A, float *C);
#endif
