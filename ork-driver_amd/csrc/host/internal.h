/* internal.h -- private state of the MI355X host library (context, weight handle, helpers).
 *
 * Mirrors the roles of the reference's struct ork_npu / struct ork_w (src/npu/internal.h:40-159) for the
 * matmul path only: a context owns one HIP stream, staging buffers and the buffer registries; a weight
 * owns one device allocation holding its panels (layout: ../hip/orkh.h). */
#ifndef ORK_INTERNAL_H
#define ORK_INTERNAL_H
#include <pthread.h>
#include <stddef.h>
#include <stdint.h>

#include "ork_npu.h"
#include "../hip/orkh.h"

/* Public dtypes (include/ork/run.h ork_dtype; reference DT_* values, src/npu/internal.h). */
enum { DT_F16 = 0, DT_I8 = 1, DT_I4 = 2 };

/* Largest K an int4-resident weight (uniform or NF4 panels) runs at. The uniform kernels widen a nibble v to
 * 16*v in an int8 lane, so the int32 sum is 16x the true one: |16*v*a| <= 16384 per product, and at
 * K = 131072 (the next multiple of 32) the worst case reaches 2^31 and wraps before the >>4. */
#define ORKI_I4_K_MAX 131040

#define ORK_DMA_MAX 64 /* zero-copy table size, as the reference (src/npu/internal.h:94-96) */

struct ork_buf { void *p; size_t n; };
struct orki_prof;

struct ork_npu {
    int offline;           /* ork_npu_init_offline: caps only, no device */
    char soc[32];
    int cores, core_budget;
    orkh_dev dev;
    void *stream;
    int async;
    /* ORK_PLAN_DEBUG set when the context was made: the planner then honours its test overrides (ORK_PLAN,
     * ORK_TILE, ORK_KSPLIT, ORK_ALINE, ORK_STREAM_NP, ORK_WPG), read at each plan so a test can switch them
     * between runs. Without it the planner reads no environment at all. */
    int plan_knobs;
    /* ORK_WS_GUARD set as well (tests): split-K partials get ORKI_WS_GUARD bytes of a fixed pattern on each side,
     * checked after the run's sync (which async mode then does not skip), so a kernel that writes past them fails
     * the run with -1 */
    int ws_guard;
    /* device staging for host-side A / C, split-K / grouped partials and grouped-run scales, grown on demand */
    struct ork_buf sA, sC, sW, sS;
    /* pinned, device-mapped host staging for host-side A (filled by the CPU, uploaded by one DMA copy) and
     * small host-side C (written by the kernels across PCIe, copied out by the CPU after the sync) */
    struct ork_buf hA, hC;
    /* ork_dma_alloc (pinned host) and ork_dev_alloc (HBM) registries */
    struct ork_buf dma[ORK_DMA_MAX];
    int dma_n;
    struct ork_buf *devb;
    int devb_n, devb_cap;
    /* ORK_PROFILE set when the context was made: per-call timing, printed at ork_npu_free (prof.c); else NULL */
    struct orki_prof *prof;
    /* device memory of weights whose handles were released with ork_w_free */
    void **orphan;
    int orphan_n, orphan_cap;
    pthread_mutex_t mu;
};

struct ork_w {
    int K, N;
    int dtype;             /* DT_F16 / DT_I8 / DT_I4: which run entry point accepts it */
    int rkind;             /* resident panel kind, ORKH_I8 / ORKH_I4U / ORKH_NF4 / ORKH_F16 */
    int KB;                /* K-blocks per panel */
    void *dB;              /* device panels (NULL for an offline weight) */
    size_t dbytes;
    int quant_kind;        /* ORK_QK_* of the int4 store (i4a8); 0 otherwise */
    uint8_t *Bi4;          /* i4a8: compact nibble store [N][K/2], kept for ork_i4a8_w_dump */
    float *bscale;         /* i4a8: per-channel scale [N] (NULL for other weights) */
    int8_t *codes;         /* offline weights only: codes [K][N] for ork_w_codes */
    uint32_t lut[4];       /* NF4 int8 codebook, packed 4 entries per word */
    int gsize;             /* K-group size for the grouped runs (0: per-channel weight) */
    ork_npu *ctx;
};

/* ---- diagnostics ---- */
void orki_err(const char *fmt, ...) __attribute__((format(printf, 1, 2)));
void orki_hip_fail(const char *what); /* counts an unexpected HIP failure and reports it */

/* ---- host worker pool: fn(lo, hi, arg) over [0, n) split into contiguous chunks ---- */
void orki_parallel_for(int n, void (*fn)(int lo, int hi, void *arg), void *arg);

/* ---- quantizers (quant.c) ---- */
extern const float ORKI_NF4_LEVELS[16];
void     orki_nf4_lut(int8_t lut[16]);
uint32_t orki_xs32(uint32_t *s);
float    orki_chan_absmax(const float *fr, int K);
void     orki_i8_quant_chans(const float *f32, int K, int N, float *bscale, int8_t *codes_nk);
float    orki_wq_best_absmax(const float *fr, int K, float rawabsmax, int nf4, const float *im, float *dq);
void     orki_i4_quant_chan(const float *fr, int K, float scale, int sr, uint32_t *seed, uint8_t *nib, int8_t *codes);
void     orki_nf4_quant_chan(const float *fr, int K, float absmax, int sr, uint32_t *seed, uint8_t *nib, uint8_t *idx);
/* Per-channel int4 quant of a whole weight, as ork_i4a8_mm_pack_im (pack.c:63-80): writes bscale[N]
 * and nib[N][K/2]; codes_nk (nullable) receives the int8 codes the weight multiplies with. */
int      orki_i4a8_quant(int K, int N, const float *f32, const float *imatrix, int nf4, int sr,
                         float *bscale, uint8_t *nib, int8_t *codes_nk);

/* ---- panels (panel.c): host tilers into the device layout of ../hip/orkh.h ---- */
size_t orki_panel_bytes(int rkind, int K, int N, int *KB_out);
void   orki_tile_i8_nk(const int8_t *codes_nk, int K, int N, int KB, uint8_t *out);
void   orki_tile_i8_kn(const int8_t *B_kn, int K, int N, int KB, uint8_t *out);
void   orki_tile_f16_kn(const uint16_t *B_kn, int K, int N, int KB, uint8_t *out);
void   orki_tile_nib_nk(const uint8_t *nib_nk, int K, int N, int KB, uint8_t pad, uint8_t *out);
void   orki_tile_nib_kn(const int8_t *B_kn, int K, int N, int KB, uint8_t *out);

/* ---- planner (plan.c) ---- */
int orki_plan(const ork_npu *c, int rkind, int M, int K, int N, int KB, orkh_plan *q, size_t *ws_bytes);
/* Waves per workgroup of the whole-panel GEMV for this weight (the grouped M = 1 launch of the multi-matmul submit). */
int orki_gemv_panel_wpg(const ork_npu *c, int rkind, int KB, int NB);
/* Kernel for a grouped-scale run (never K-split). */
void orki_plan_grouped(const ork_npu *c, int rkind, int M, int K, int N, int KB, int G, orkh_plan *q);

/* ---- context helpers (context.c) ---- */
int   orki_need_device(const ork_npu *c, const char *who);
void *orki_stage(ork_npu *c, struct ork_buf *b, size_t n);
void *orki_hstage(ork_npu *c, struct ork_buf *b, size_t n); /* pinned, device-mapped host memory */
int   orki_dev_find(ork_npu *c, const void *p, size_t n);   /* 1 if [p,p+n) lies in an ork_dev_alloc buffer */
int   orki_dma_find(ork_npu *c, const void *p);             /* 1 if p lies in an ork_dma_alloc buffer */
/* Host operands of a run. orki_host_a: device copy of a host A (async upload on the stream; NULL on failure).
 * orki_host_c: the device-visible pointer the kernels write a host C through, and how it reaches C (*mode);
 * orki_host_c_post: after the launches (queues the D2H copy where one is needed);
 * orki_host_c_done: after the stream sync (the CPU copy-out where one is needed). */
enum { ORKI_C_INPLACE = 0, ORKI_C_PINNED = 1, ORKI_C_HBM = 2 };
#define ORKI_HOST_C_DIRECT (1u << 20) /* host C up to this size is written straight into pinned memory */
const void *orki_host_a(ork_npu *c, const void *A, size_t n);
void *orki_host_c(ork_npu *c, void *C, size_t n, int *mode);
int   orki_host_c_post(ork_npu *c, void *C, const void *dC, size_t n, int mode);
void  orki_host_c_done(ork_npu *c, void *C, size_t n, int mode);
void  orki_orphan(ork_npu *c, void *dptr);
ork_w *orki_w_new(ork_npu *c, int K, int N, int dtype, int rkind);
int   orki_w_upload(ork_w *w, const void *panels);

/* ---- split-K workspace guard bands (ork_npu.ws_guard) ---- */
#define ORKI_WS_GUARD 4096
/* Stage a split-K workspace of ws bytes for one run or chain: the context's grown buffer (or `fixed`, holding at
 * least ws + 2 * ORKI_WS_GUARD bytes when guarded, for the no-allocation run), with the guard bands filled on the
 * stream when the context guards. NULL on failure. */
void *orki_ws_stage(ork_npu *c, size_t ws, void *fixed);
/* After the stream sync: 0 if the guard bands around the workspace orki_ws_stage returned are intact (or the
 * context does not guard), -1 with a message naming `who` if a kernel wrote into them. */
int   orki_ws_check(ork_npu *c, const void *ws_base, size_t ws, const char *who);

/* ---- ORK_PROFILE (prof.c): around each successful run call, begin (device: 1 to time its launches with events
 * on the stream), launched (after its last launch), end (on return; host wall time). No-ops without ORK_PROFILE. */
typedef struct { double t0; int pair; } orki_ptok;
void orki_prof_init(ork_npu *c);
void orki_prof_begin(ork_npu *c, orki_ptok *t, int device);
void orki_prof_launched(ork_npu *c, orki_ptok *t);
void orki_prof_end(ork_npu *c, orki_ptok *t, const char *who, const char *plan);
void orki_prof_settle(ork_npu *c); /* after a stream sync: read back the pending event pairs */
void orki_prof_dump(ork_npu *c);   /* print the rows, release the profile */

/* ---- host GEMMs of an offline context (cpu_gemm.c): exact int32, and the grouped float accumulate ---- */
int orki_cpu_gemm_grouped(int M, int K, int N, int G, const int8_t *A, const int8_t *B_kn, const float *aS,
                          const float *bS, float *C);

/* ---- overlap guard (run.c), reference src/npu/core/submit.c:532-539 ---- */
int orki_check_overlap(const char *name, uintptr_t a0, uintptr_t a1, uintptr_t c0, uintptr_t c1);

#endif
