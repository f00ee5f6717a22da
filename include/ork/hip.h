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
 * (ork_dev_alloc or any hipMalloc); a split-K plan keeps its partials in a static 8 MiB per-GPU scratch array
 * instead of a grown workspace, and a plan needing more is refused (-1). No call allocates. Calls that overlap
 * on one GPU share that array and race. Same results and return codes as ork_i8_mm_run otherwise. */
int          ork_i8_mm_run_noalloc(ork_npu *ctx, ork_w *w, int M, const int8_t *A, int32_t *C);
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
