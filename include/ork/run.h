/* ork/run.h -- matmul entry points (MI355X build). Part of <ork_npu.h>.
 * Runs are synchronous: C is valid on return (see ork/hip.h for the device-resident async mode).
 * Errors: -1 on bad arguments, dtype mismatch (run dtype must match the pack dtype), A/C overlap,
 * an offline context, or a device failure. */
#ifndef ORK_RUN_H
#define ORK_RUN_H

/* reference include/ork/run.h:21. C[M][N] int32 = A[M][K] int8 x packed B (int8 or an i4a8 weight).
 * Exact int32. */
int          ork_i8_mm_run(ork_npu *ctx, ork_w *w, int M, const int8_t *A, int32_t *C);
/* reference include/ork/run.h:27 (never returned by this build; every shape has a path). */
#define ORK_RC_WEDGE_PRONE (-501)
/* reference include/ork/run.h:36 */
typedef enum { ORK_DT_F16 = 0, ORK_DT_I8 = 1, ORK_DT_I4 = 2 } ork_dtype;
/* reference include/ork/run.h:111. W4A4: A int4 values in int8 containers; exact int32 C. */
int          ork_i4_mm_run(ork_npu *ctx, ork_w *w, int M, const int8_t *A, int32_t *C);
/* reference include/ork/run.h:121-125. Grouped W4A4: A int4 values in int8 containers, aScale[M*(K/G)],
 * bScale[(K/G)*N], C f32[M][N]; weight from ork_i4_mm_pack_grouped (or ork_w_set_group). Bit-identical to
 * the reference's CPU accumulate. -1 / -3 as ork_i8_mm_run_grouped. */
int          ork_i4_mm_run_grouped(ork_npu *ctx, ork_w *w, int M, const int8_t *A, const float *aScale,
                                   const float *bScale, float *C);
/* reference include/ork/run.h:132. The CPU int8 GEMM (B [K][N] raw codes), exact int32; no device,
 * no context. Exposed so a caller can time the CPU side of a routing decision. */
void         ork_i8_mm_run_cpu(int M, int K, int N, const int8_t *A, const int8_t *B, int32_t *C);
#endif
