/* oracle/ref_driver.c -- entry points into the reference's OWN CPU code, compiled from the reference
 * sources in place (see ref.mk). TEST INFRASTRUCTURE ONLY: loaded by tests/ and by bench.py's
 * cpu_baseline leg, never by the product.
 *
 * Only reference functions whose translation units compile on x86 as they are, and that link with
 * nothing outside those units once unreferenced sections are discarded, are reachable here:
 *   orki_cpu_gemm_i32   src/npu/core/buf.c:428-477   (the CPU MAC / offline oracle)
 *   orki_i4_quant_chan  src/npu/i4/quant.c:28-40     (uniform int4 channel quant, RN and SR)
 *   orki_i4_expand_chan_to_i8 src/npu/i4/quant.c:110-128 (nibble sign-extend)
 *   orki_cpu_gemm_grouped src/npu/core/buf.c:501-520 (per-group scaled accumulate, the grouped-run oracle)
 * Built twice by ref.mk: plain (-O2, as the reference library is built: single-threaded) and with -fopenmp
 * (the row-parallel pragma of orki_cpu_gemm_i32 live, for the all-cores baseline); ref_threads reports which.
 * Everything else on the path reaches ORKI_NF4_LEVELS or the scales in src/npu.c, which does not
 * compile on x86 (three unguarded NEON intrinsics at src/npu.c:1813, :1816, :1880), so it is not
 * buildable here. */
#include <stdint.h>
#ifdef _OPENMP
#include <omp.h>
#endif
void orki_cpu_gemm_i32(int M, int K, int N, const int8_t *A, const int8_t *B, int32_t *C);
void orki_i4_quant_chan(const float *fr, int K, float scale, int sr, uint32_t *seed, uint8_t *nib, float *qf32);
void orki_i4_expand_chan_to_i8(const uint8_t *nib, int K, int8_t *i8);
int orki_cpu_gemm_grouped(int M, int K, int N, int G, const int8_t *A, const int8_t *codes, const float *aScale,
                          const float *bScale, float *C);

void ref_gemm_i32(int M, int K, int N, const int8_t *A, const int8_t *B, int32_t *C) {
    orki_cpu_gemm_i32(M, K, N, A, B, C);
}
void ref_i4_quant_chan(const float *fr, int K, float scale, int sr, uint32_t *seed, uint8_t *nib, float *qf32) {
    orki_i4_quant_chan(fr, K, scale, sr, seed, nib, qf32);
}
void ref_i4_expand_chan_to_i8(const uint8_t *nib, int K, int8_t *i8) {
    orki_i4_expand_chan_to_i8(nib, K, i8);
}
int ref_gemm_grouped(int M, int K, int N, int G, const int8_t *A, const int8_t *codes, const float *aScale,
                     const float *bScale, float *C) {
    return orki_cpu_gemm_grouped(M, K, N, G, A, codes, aScale, bScale, C);
}

/* Threads the OpenMP build's row loop uses (1 in the plain build, where the pragma is inert). */
int ref_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
