/* orkh.h -- the thin C-ABI between the C host library and HIP (gfx950 / MI355X).
 *
 * Plain C: no HIP types cross this boundary. Streams are opaque `void *` (a hipStream_t underneath),
 * device memory is `void *`. Every call returns 0 on success and a negative value on a HIP error,
 * with the HIP error string available from orkh_last_error().
 *
 * Resident weight layout ("panels") shared by every kernel
 * -------------------------------------------------------
 * B[K][N] is stored as 1 KiB blocks, block (nb, kb) at byte offset (nb * KB + kb) * 1024, where
 * nb = n / 16 indexes a 16-column output panel and kb indexes a K-block; KB = Kp / KPB blocks per panel.
 * Inside a block, lane l (0..63) of a wave owns the 16 bytes at l*16: column n = nb*16 + (l % 16) and
 * the K-chunk selected by g = l / 16:
 *   ORKH_I8   int8,   KPB = 64:  bytes i = 0..15 hold k = kb*64 + g*16 + i
 *   ORKH_F16  fp16,   KPB = 32:  halves i = 0..7 hold k = kb*32 + g*8 + i
 *   ORKH_I4U / ORKH_NF4 nibbles, KPB = 128: dword d (0..3), byte b (0..3) holds
 *             k = kb*128 + g*32 + d*8 + b in its low nibble and k + 4 in its high nibble.
 *             ORKH_I4U nibbles are two's-complement int4 codes; ORKH_NF4 nibbles index a 16-entry
 *             int8 codebook (lut).
 * Padding k >= K is zero (code 0; for NF4 the index of the 0 level). One wave-wide 16-byte load per
 * lane fetches one whole block: the GEMV streams B with perfectly coalesced 1 KiB reads and the same
 * bytes are already an MFMA B-fragment (v_mfma_*_16x16x{64 i8, 32 f16}: lane%16 = column,
 * lane/16 = K-group). A and B fragments use the same lane/byte -> k assignment, so the MFMA's
 * internal k order never matters for the (exact, integer) result.
 */
#ifndef ORKH_H
#define ORKH_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORKH_I8 = 0, ORKH_I4U = 1, ORKH_NF4 = 2, ORKH_F16 = 3 };

typedef struct orkh_dev {
    int ordinal;
    int cu_count;         /* multiProcessorCount */
    int clock_khz;        /* peak shader clock */
    int mem_clock_khz;
    int mem_bus_bits;
    size_t lds_per_block; /* sharedMemPerBlock */
    size_t hbm_bytes;     /* totalGlobalMem */
    int l2_bytes;
    char arch[64];        /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
    char name[256];
    void *scratch;        /* this device's copy of the library's static scratch array (ORKH_SCRATCH_BYTES) */
    int wall_khz;         /* rate of the device's constant wall clock (orkh_mark) */
} orkh_dev;

/* Device scratch of fixed size that needs no allocation: a file-scope __device__ array in orkh_runtime.hip, one
 * copy per GPU, held until the process ends. orkh_init resolves this device's address of it (orkh_dev.scratch).
 * Calls that use it on one GPU share it, so overlapping calls race; nothing in it starts at zero. */
#define ORKH_SCRATCH_BYTES (8u << 20)

/* ---- runtime ---- */
int         orkh_device_count(void);
int         orkh_init(int ordinal, orkh_dev *out, void **stream_out);
void        orkh_stream_destroy(void *stream);
const char *orkh_last_error(void);
/* Why the last orkh_mm_launch* call on this thread refused its plan ("" when it did not). */
const char *orkh_launch_error(void);
void       *orkh_malloc(size_t n);                 /* device memory (HBM); NULL on failure */
int         orkh_free(void *p);
void       *orkh_host_alloc(size_t n);             /* pinned, device-mapped host memory */
int         orkh_host_free(void *p);
void       *orkh_host_devptr(void *p);             /* device address of pinned, device-mapped host memory */
int         orkh_h2d(void *dst, const void *src, size_t n, void *stream);   /* async; direction inferred */
int         orkh_d2h(void *dst, const void *src, size_t n, void *stream);   /* async */
int         orkh_d2d(void *dst, const void *src, size_t n, void *stream);   /* async */
/* async strided copy: rows x width bytes, row pitches dpitch / spitch */
int         orkh_d2h_2d(void *dst, size_t dpitch, const void *src, size_t spitch, size_t width, size_t rows, void *stream);
int         orkh_sync(void *stream);
/* Enqueue on the stream one 1-thread kernel that writes the device wall clock (a 64-bit counter at
 * orkh_dev.wall_khz) to dev_u64: a timestamp taken where the stream reaches it, also inside a captured graph. */
int         orkh_mark(void *dev_u64, void *stream);
/* streaming read of `bytes` device bytes, one XOR word per workgroup into sink; the workgroup count, or -1 */
long long   orkh_read_probe(const void *dev, size_t bytes, unsigned *sink, void *stream);
int         orkh_device_sync(void);
/* Timing events: a HIP event (NULL on failure), recorded in stream order; orkh_event_ms waits for e1 and gives the
 * milliseconds between the two recordings (-1 on a HIP error). */
void       *orkh_event_new(void);
void        orkh_event_free(void *ev);
int         orkh_event_record(void *ev, void *stream);
float       orkh_event_ms(void *e0, void *e1);
/* 1 if the stream is being captured into a HIP graph, 0 if not, -1 on a HIP error. */
int         orkh_stream_capturing(void *stream);
/* 1 if p is device (or device-mapped) memory known to the HIP runtime, 0 if plain host memory. */
int         orkh_ptr_is_device(const void *p);

/* ---- matmul launch ---- */
enum { ORKH_ALGO_STREAM = 0, ORKH_ALGO_TILED = 1, ORKH_ALGO_GEMV = 2, ORKH_ALGO_TILED2 = 3 };

/* One C[M][N] = A[M][K] x B[K][N] launch on resident panels. A is row-major with row stride lda
 * elements (int8 for the integer kinds, fp16 for ORKH_F16); C is row-major int32 (integer kinds) or
 * fp32 (ORKH_F16) with row stride ldc elements. All pointers are device pointers; A and B must be
 * 16-byte aligned and lda*elem a multiple of 16 bytes. A (M*lda*elem bytes) and the panels are read
 * through 32-bit buffer offsets, so each must stay below ORKH_MAX_OPERAND_BYTES. */
#define ORKH_MAX_OPERAND_BYTES 0x80000000u
typedef struct orkh_mm {
    int kind;
    int M, K, N;
    int KB;               /* K-blocks per panel (Kp / KPB) */
    const void *A;
    int lda;
    const void *B;
    void *C;
    int ldc;
    uint32_t lut[4];      /* ORKH_NF4 codebook, entry e in byte e%4 of lut[e/4] */
    int c_wt;             /* k_tiled2: 1 = store C with write-through stores (set by the launcher from plan.cwt) */
} orkh_mm;

/* Launch plan chosen by the host planner (ork-driver_amd/csrc/host/plan.c). */
typedef struct orkh_plan {
    int algo;             /* ORKH_ALGO_STREAM | ORKH_ALGO_TILED | ORKH_ALGO_GEMV | ORKH_ALGO_TILED2 */
    /* GEMV (M = 1 only): the STREAM grid and fields below, VALU dot products instead of MFMA.
     * STREAM: grid (N/16, ksplit), wpg waves per workgroup, each wave kbw K-blocks of one panel,
     * mt = ceil(M/16) row tiles (1..4). ksplit > 1 writes partials to ws and adds a reduce pass. */
    int mt, wpg, kbw, kbs, ksplit;
    /* TILED: bm x bn output tile per 256-thread workgroup, K staged through LDS. */
    int bm, bn;
    /* TILED2: 1 = load A stages as whole 128-byte row lines into a swizzled LDS image where the stage's rows
     * are one line each (else, and with 0, in MFMA fragment order) */
    int aline;
    /* TILED2: 2 = a two-slot ring (two workgroups per CU on the tiles whose 4-slot ring fills one), else 0 */
    int ring;
    /* TILED2: 1 = write-through C stores, else write-back */
    int cwt;
    /* STREAM: np = 2 pairs panels: npg workgroups, the first N/16 - npg owning two adjacent panels each */
    int np, npg;
    /* GEMV and STREAM: 1 = half a panel (8 columns) per workgroup, grid (N/8, ksplit) (k_gemv_half, k_stream's
     * half mode), else one panel (or two: np) */
    int half;
    void *ws;             /* split-K partials, >= ksplit*M*N*4 bytes (device) */
} orkh_plan;

int orkh_mm_launch(const orkh_mm *p, const orkh_plan *plan, void *stream);

/* Grouped tiled launch (multi-matmul submit, M > 1): n (2..ORKH_TGROUP_MAX) matmuls of one kind, one M and one K in
 * a single k_tiled2 launch under one plan (algo ORKH_ALGO_TILED2, ksplit 1: the tile the planner picks for their
 * columns together); each matmul keeps its own A, B, C, N and ldc. 0 / -2 inconsistent tasks or plan / -1 HIP. */
#define ORKH_TGROUP_MAX 8
int orkh_mm_launch_tgroup(const orkh_mm *p, int n, const orkh_plan *plan, void *stream);

/* Grouped M = 1 launch (multi-matmul submit): n independent GEMVs of one kind (p.kind equal, p.M == 1)
 * in one launch. Task i covers workgroups [t[i].wg0, t[i].wg0 + p.N/16), wg0 ascending from 0 with no
 * gaps; each workgroup runs wpg waves over the whole K of one panel, kbw K-blocks per wave
 * (kbw * wpg >= p.KB). */
#define ORKH_GROUP_MAX 16
typedef struct orkh_gtask {
    orkh_mm p;
    int kbw;
    int wg0;
} orkh_gtask;
typedef struct orkh_group {
    int n;
    orkh_gtask t[ORKH_GROUP_MAX];
} orkh_group;
/* Grouped run: C[m][n] = sum over K-groups g ascending of ((float)P_g[m][n] * aS[m*(K/G)+g]) * bS[g*N+n],
 * P_g the exact int32 partial of group g. Integer kinds only; G % 32 == 0, K % G == 0. plan->algo selects
 * the panel-streaming k_grouped (ORKH_ALGO_STREAM) or the LDS-ring tile k_tiled2g (ORKH_ALGO_TILED2, bm x bn;
 * int8 and uniform int4). 0 / -2 bad arguments / -1 HIP error. */
int orkh_mm_launch_grouped(const orkh_mm *p, const orkh_plan *plan, int G, const float *aS, const float *bS, float *C,
                           int ldc, void *stream);
int orkh_mm_launch_group(const orkh_group *g, int wpg, void *stream);
/* One-row run with a fused row prologue and column epilogue (k_gemv_row, orkh_rowrun.hip): every workgroup builds the
 * int8 row in LDS from a float row (pro: ORKH_ROW_RMSNORM = RMSNorm with weight nw, then the per-row quant;
 * ORKH_ROW_QUANT = the per-row quant), runs the M = 1 GEMV on its panel or half panel, and applies epi to its
 * columns' int32 sums: ORKH_COL_STORE C[t][n] = c; ORKH_COL_RESID x[n] += (c * s) * ws0[n]; ORKH_COL_SWIGLU
 * y[n] = silu((c_gate * s) * ws0[n]) * ((c_up * s) * ws1[n]), s the row's scale (written to *as_out by workgroup 0
 * when non-NULL). Built: RMSNORM + STORE (ORKH_I8), QUANT + RESID and RMSNORM + SWIGLU (ORKH_I8 / I4U / NF4). */
enum { ORKH_ROW_RMSNORM = 0, ORKH_ROW_QUANT = 1 };
enum { ORKH_COL_STORE = 0, ORKH_COL_RESID = 1, ORKH_COL_SWIGLU = 2 };
#define ORKH_ROW_KMAX 8192 /* bytes of the int8 row in LDS: KB * (64 or 128) <= this */
typedef struct orkh_row {
    int kind, K, KB;      /* panel kind (ORKH_I8 / ORKH_I4U / ORKH_NF4), row length, K-blocks per panel */
    uint32_t lut[4];      /* ORKH_NF4 codebook */
    int pro, epi;
    int nt;               /* STORE: 1..3 weights, their workgroups back to back; RESID 1; SWIGLU 2 (gate, up) */
    const void *B[3];     /* panels of each weight */
    int nb[3];            /* 16-column panels (N / 16) of each weight */
    int32_t *C[3];        /* STORE */
    const float *row;     /* the float row, K elements */
    const float *nw;      /* RMSNORM weight, K elements */
    float eps;
    float *as_out;        /* nullable */
    const float *ws0, *ws1;
    float *x;             /* RESID: updated in place (must not overlap row) */
    float *y;             /* SWIGLU: output (must not overlap row) */
    int half;             /* 1: half a panel (8 columns) per workgroup */
} orkh_row;
/* 0 / -2 an unbuilt combination or bad fields / -1 HIP error */
int orkh_row_launch(const orkh_row *p, void *stream);
/* Bytes of LDS the stage ring of k_tiled2 takes for (kind, bm x bn); -1 for a tile that is not built. */
int orkh_tiled2_ring_lds(int kind, int bm, int bn);
/* 1 where the LDS-ring kernel has a two-slot ring for the tile (plan.ring = 2): tiles whose ring of up to 4 slots
 * leaves room for one workgroup per CU, and two with 2 slots; never NF4 */
int orkh_tiled2_ring2_ok(int kind, int bm, int bn);
/* Names of the compiled kernel variants, for diagnostics ("stream_i8_mt1_w4", ...). */
const char *orkh_mm_variant(const orkh_mm *p, const orkh_plan *plan);

#ifdef __cplusplus
}
#endif
#endif
