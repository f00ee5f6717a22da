/* ork/chain.h -- multi-matmul submit: S independent matmuls in one call (MI355X build). Part of
 * <ork_npu.h>.
 *
 * The reference chains (PC-chained NPU programs) and streams (round-robin across NPU cores) S
 * independent matmuls; results are identical to S single runs. Here every M = 1 task of one weight
 * kind shares a single grouped kernel launch (up to 16 tasks per launch) and the other tasks launch
 * back to back on the context's stream, so a decode step pays one launch, not S.
 * Returns 0 on success; -2 on bad arguments (NULL context/tasks/weight, S outside 1..1024, M < 1,
 * dtype mismatch, a bad cstride); -1 on A/C overlap or a device failure. On an offline context the int8
 * chain and the int4 chain / stream run every task exactly on the CPU from its host codes (C rows packed at
 * stride N, as the reference's CPU chain), -1 if a weight is not an offline one; the int8 and fp16 streams
 * have no offline path (-1), as in the reference.
 * A and C may be host memory, ork_dma_alloc buffers or ork_dev_alloc buffers, per task. */
#ifndef ORK_CHAIN_H
#define ORK_CHAIN_H

/* reference include/ork/dynamic.h:15-21. cstride: row stride of C in elements (0 = N). */
typedef struct {
    ork_w *w;
    int M;
    const int8_t *A;
    int32_t *C;
    int cstride;
} ork_mm_task_i8;

/* reference include/ork/dynamic.h:23-28 */
typedef struct {
    ork_w *w;
    int M;
    const int8_t *A;
    int32_t *C;
} ork_mm_task_i4;

/* reference include/ork/bmm.h:117 */
typedef struct {
    ork_w *w;
    int M;
    const ork_f16 *A;
    float *C;
} ork_mm_task_f16;

/* reference include/ork/dynamic.h:30 (int8 and i4a8 weights, packed as DT_I8) */
int ork_i8_mm_run_chain(ork_npu *ctx, int S, const ork_mm_task_i8 *tasks);
/* reference include/ork/chain.h:116 */
int ork_i8_mm_run_stream(ork_npu *ctx, int S, const ork_mm_task_i8 *tasks);
/* reference include/ork/chain.h:110 (W4A4 weights from ork_i4_mm_pack) */
int ork_i4_mm_run_chain(ork_npu *ctx, int S, const ork_mm_task_i4 *tasks);
/* reference include/ork/chain.h:123 */
int ork_i4_mm_run_stream(ork_npu *ctx, int S, const ork_mm_task_i4 *tasks);
/* reference include/ork/bmm.h:118 */
int ork_f16_mm_run_stream(ork_npu *ctx, int S, const ork_mm_task_f16 *tasks);
#endif
