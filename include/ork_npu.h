/* ork_npu.h -- resident-weight matmul engine, MI355X (gfx950) build.
 *
 * Drop-in for the GEMM path of ork-driver's public C API (reference: include/ork_npu.h): the same
 * typedefs, version macros and function signatures, implemented on one AMD Instinct MI355X through
 * HIP. Pack a weight B[K,N] once (resident in HBM), then run C = A x B many times:
 *
 *   C[M,N] (int32) = A[M,K] (int8)  x B[K,N] (int8 / int4 / NF4 codes)   ork_i8_mm_run, ork_i4_mm_run
 *   C[M,N] (fp32)  = A[M,K] (fp16)  x B[K,N] (fp16)                      ork_f16_mm_run
 *
 * Only the resident-weight matmul subset is provided (context, DMA buffers, pack/load/dump, run, and
 * the multi-matmul submit of ork/chain.h); ork/hip.h adds device-resident operands for callers that
 * keep A and C in HBM.
 */
#ifndef ORK_NPU_H
#define ORK_NPU_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef _Float16 ork_f16;           /* reference include/ork_npu.h:19 */
typedef struct ork_npu ork_npu;     /* device context (one per process)       -- include/ork_npu.h:20 */
typedef struct ork_w ork_w;         /* resident packed weights for one B[K,N]  -- include/ork_npu.h:21 */

/* Library API version (reference include/ork_npu.h:30); ork_npu_version() appends "+mi355x". */
#define ORK_NPU_VERSION "1.0.190"
/* On-disk pack format version (reference include/ork_npu.h:37). The O4N1 int4 blob is byte-compatible. */
#define ORK_PACK_FORMAT_VERSION 1u

#include "ork/context.h"
#include "ork/dma.h"
#include "ork/weights.h"
#include "ork/run.h"
#include "ork/chain.h"
#include "ork/hip.h"

#ifdef __cplusplus
}
#endif
#endif
