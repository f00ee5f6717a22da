/* ork/hip.h -- MI355X-specific extensions (no reference counterpart). Part of <ork_npu.h>.
 *
 * The reference API takes host pointers and returns when C is on the host. A decode loop on a
 * discrete GPU wants A and C to stay in HBM: allocate them here and pass them to the ordinary run
 * entry points, which then launch in place (no copies). With async mode on, a run whose A and C are
 * both device buffers returns right after the launch; ork_npu_sync() waits. */
#ifndef ORK_HIP_H
#define ORK_HIP_H

/* Device (HBM) buffer owned by the context, usable in place as A or C. NULL on failure/offline. */
void        *ork_dev_alloc(ork_npu *ctx, size_t size);
void         ork_dev_free(ork_npu *ctx, void *ptr);
/* Synchronous copies between host memory and a device buffer. 0 / -1. */
int          ork_dev_upload(ork_npu *ctx, void *dst_dev, const void *src, size_t n);
int          ork_dev_download(ork_npu *ctx, void *dst, const void *src_dev, size_t n);
/* Async mode for device-resident runs (default 0 = every run synchronizes). */
void         ork_npu_set_async(ork_npu *ctx, int on);
/* Wait for every launch on the context's stream. 0 / -1. */
int          ork_npu_sync(ork_npu *ctx);
/* The context's hipStream_t, for callers that order their own work after a run (or time it). */
void        *ork_npu_stream(ork_npu *ctx);
/* No counterpart in the reference: ork_i8_mm_run (include/ork/run.h:21) for callers that cannot allocate --
 * code under HIP graph capture, serving loops and harnesses that forbid hipMalloc. A and C must be device memory
 * (ork_dev_alloc or any hipMalloc) and A 16-byte aligned (ork_i8_mm_run stages a misaligned A; this call refuses
 * it, -1); a split-K plan keeps its partials in a static 8 MiB per-GPU scratch array instead of a grown
 * workspace, and a plan needing more is refused (-1). No call allocates. Under HIP graph capture async mode is
 * required (ork_npu_set_async(ctx, 1)): outside it the call ends with a stream synchronisation, so on a capturing
 * stream it is refused (-1) before anything is enqueued. Calls that overlap on one GPU share that array and race.
 * Same results and return codes as ork_i8_mm_run otherwise. */
int          ork_i8_mm_run_noalloc(ork_npu *ctx, ork_w *w, int M, const int8_t *A, int32_t *C);
/* No counterpart in the reference, whose harness prepares each activation row on the host, runs ork_i8_mm_run and
 * uses the output columns on the host (examples/bench.c:83-90 quantise / dequantise, :105-113 mm(), :128-145 the
 * layer's norm, residual add and SwiGLU): ork_i8_mm_run for ONE activation row with the row's preparation and each
 * output column's use fused into the matmul launch, for decode loops on device-resident rows. S weights from
 * ork_i8_mm_pack(_f32) or ork_i4a8_mm_pack(_im) / ork_i4a8_mm_load (int8, uniform int4 or NF4 resident), one K
 * (K <= ORK_ROW_KMAX).
 *   prologue  ORK_ROW_RMSNORM  y = (row * (1 / sqrt(ss / K + eps))) * norm_w, ss = sum of row^2 (taken as a
 *                              512-thread workgroup takes it: thread t sums elements t, t + 512, ... in order, then
 *                              the waves' partials by a fixed tree)
 *             ORK_ROW_QUANT    y = row
 *             then the int8 row a = clamp(rint(y / s), -127, 127), s = max|y| / 127 (1 for a zero row), the
 *             per-row quantisation of examples/quant.c:34-37; s is written to *row_scale when non-NULL.
 *   epilogue  on each output column's exact int32 sum c[n] = sum_k a[k] * B[k][n]:
 *             ORK_COL_STORE    C[i][n] = c (S = 1..3 weights, e.g. q / k / v, each into its own C[i])
 *             ORK_COL_RESID    out[n] += (c * s) * w_scale[0][n]                            (S = 1: a residual add)
 *             ORK_COL_SWIGLU   out[n] = silu(g) * u, g = (c_gate * s) * w_scale[0][n], u = (c_up * s) * w_scale[1][n],
 *                              silu(g) = g / (1 + exp(-g))         (S = 2: gate and up weights of one shape and kind)
 * Built combinations: RMSNORM + STORE (int8 weights), QUANT + RESID and RMSNORM + SWIGLU (every kind); others -2.
 * Every pointer is device memory (ork_dev_alloc or hipMalloc); `out` and the C[i] must not overlap the row. Products
 * and sums round as written (no fused multiply-add), so a caller that prepares the row by these operations in this
 * order and runs ork_i8_mm_run gets the same results bit for bit. Returns 0 after the launch in async mode, else
 * after the stream sync; -2 for bad arguments or an unbuilt combination; -1 on a device failure. */
#define ORK_ROW_KMAX 8192
enum { ORK_ROW_RMSNORM = 0, ORK_ROW_QUANT = 1 };
enum { ORK_COL_STORE = 0, ORK_COL_RESID = 1, ORK_COL_SWIGLU = 2 };
typedef struct ork_row_op {
    int prologue;              /* ORK_ROW_* */
    const float *row;          /* f32[K] */
    const float *norm_w;       /* f32[K], ORK_ROW_RMSNORM */
    float eps;                 /* ORK_ROW_RMSNORM */
    float *row_scale;          /* nullable: s */
    int epilogue;              /* ORK_COL_* */
    int32_t *C[3];             /* ORK_COL_STORE: int32[N] of weight i */
    const float *w_scale[2];   /* per-output-channel weight scales f32[N]: RESID [0]; SWIGLU gate [0], up [1] */
    float *out;                /* RESID: f32[N] updated in place; SWIGLU: f32[N] written */
} ork_row_op;
int          ork_i8_mm_run_row(ork_npu *ctx, int S, ork_w *const *w, const ork_row_op *op);
/* Profiling: enqueue on the context's stream a timestamp of the device wall clock, written to 8-byte aligned
 * device memory dev_u64 when the stream reaches it (a tiny kernel, so it also works inside a captured HIP graph,
 * where event timestamps are not available). ork_npu_wallclock_khz gives the clock's constant rate. 0 / -1. */
int          ork_npu_mark(ork_npu *ctx, void *dev_u64);
int          ork_npu_wallclock_khz(const ork_npu *ctx);
/* Profiling: enqueue on the context's stream a plain streaming read of `bytes` (a multiple of 16) of 16-byte
 * aligned device memory -- the M = 1 GEMV's loads without its arithmetic, which prices a weight's bytes in the
 * same launch harness. Workgroup i stores the XOR of the 32-bit words it read into dev_sink[i]; the XOR of all
 * of them is the XOR of every word of the bytes. Returns the workgroup count (ceil(bytes / 8192) words of
 * dev_sink), or -1. Synchronises unless async mode is on. */
long long    ork_npu_read_probe(ork_npu *ctx, const void *dev, size_t bytes, uint32_t *dev_sink);
/* The resident form of a device weight, for callers that run their own kernels on it (the decoder harness fuses
 * its per-row operators into M = 1 matmul launches): the device address of its panels, the K-blocks per panel and
 * the panel kind (0 int8, 1 uniform int4, 2 NF4, 3 fp16), laid out as ork-driver_amd/csrc/hip/orkh.h documents,
 * and the NF4 codebook words (entry e in byte e % 4 of lut[e / 4]). 0, or -1 for NULL or an offline weight. */
int          ork_w_device_panels(const ork_w *w, const void **panels, int *KB, int *kind, uint32_t lut[4]);
/* Name of the kernel variant the planner picks for (kind of w, M); for diagnostics and profiling. */
const char  *ork_w_plan_name(ork_npu *ctx, const ork_w *w, int M);
/* The same for a grouped-scale run (ork_i8_mm_run_grouped / ork_i4_mm_run_grouped) of w at M rows:
 * "grouped_<kind>_mt<n>" (panel streaming) or "tiled2g_<kind>_<BM>x<BN>"; "none" without a group size. */
const char  *ork_w_grouped_plan_name(ork_npu *ctx, const ork_w *w, int M);
#endif
