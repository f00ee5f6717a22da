// The bench's host-side call sequences (pack, dump, load, run, chain, grouped, free; device and host operands)
// at reduced sizes, against the HIP-layer stand-ins of orkh_host_stubs.c, for AddressSanitizer
// (tests/test_host_asan.py). Prints "done" when every call returned success.
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "ork_npu.h"

static uint64_t rs = 88172645463325252ull;
static double urand(void) {
    rs ^= rs << 13;
    rs ^= rs >> 7;
    rs ^= rs << 17;
    return (double)(rs >> 11) / 9007199254740992.0;
}
static float nrand(void) { return (float)(sqrt(-2 * log(urand() + 1e-12)) * cos(6.283185307 * urand())); }
#define REQ(x)                                                                                                 \
    do {                                                                                                       \
        if (!(x)) {                                                                                            \
            printf("FAILED: %s (line %d)\n", #x, __LINE__);                                                    \
            return 1;                                                                                          \
        }                                                                                                      \
    } while (0)

int main(void) {
    ork_npu *c = ork_npu_init();
    REQ(c);
    const int K = 1024, N = 768;
    float *W = malloc((size_t)K * N * 4), *im = malloc(K * 4), *bs = malloc(N * 4);
    for (size_t i = 0; i < (size_t)K * N; i++) W[i] = 0.02f * nrand();
    for (int i = 0; i < K; i++) im[i] = (float)(0.5 + 1.5 * urand());
    int8_t *dA = ork_dev_alloc(c, 512 * K);
    int32_t *dC = ork_dev_alloc(c, (size_t)512 * N * 4);
    REQ(dA && dC);
    ork_npu_set_async(c, 1);
    for (int nf4 = 0; nf4 < 2; nf4++) { /* config 3: w4a8 with an importance vector, uniform and NF4 */
        if (nf4) setenv("ORK_NF4", "1", 1);
        ork_w *w0 = ork_i4a8_mm_pack_im(c, K, N, W, im, bs);
        unsetenv("ORK_NF4");
        REQ(w0);
        const size_t need = ork_i4a8_w_dump(w0, NULL, 0);
        uint8_t *blob = malloc(need);
        REQ(ork_i4a8_w_dump(w0, blob, need) == need);
        ork_w *ws[4] = {w0};
        for (int i = 1; i < 4; i++) REQ((ws[i] = ork_i4a8_mm_load(c, K, N, blob, need)) != NULL);
        for (int M = 1; M <= 64; M += 63)
            for (int i = 0; i < 4; i++) REQ(ork_i8_mm_run(c, ws[i], M, dA, dC) == 0);
        ork_npu_set_async(c, 0);
        int8_t *A3 = malloc(2 * K);
        int32_t *C3 = malloc((size_t)2 * N * 4);
        REQ(ork_dev_download(c, A3, dA, 2 * K) == 0 && ork_i8_mm_run(c, ws[3], 2, dA, dC) == 0 &&
            ork_dev_download(c, C3, dC, (size_t)2 * N * 4) == 0);
        ork_npu_set_async(c, 1);
        for (int i = 0; i < 4; i++) ork_mm_free(c, ws[i]);
        free(blob);
        free(A3);
        free(C3);
    }
    { /* config 1 and the chain, host operands, config 2 fp16, config 4 W4A4, grouped W4A4 */
        ork_w *w8[3];
        for (int i = 0; i < 3; i++) REQ((w8[i] = ork_i8_mm_pack_f32(c, K, N, W, bs)) != NULL);
        for (int M = 1; M <= 512; M *= 8)
            for (int i = 0; i < 3; i++) REQ(ork_i8_mm_run(c, w8[i], M, dA, dC) == 0);
        ork_mm_task_i8 t[3];
        for (int i = 0; i < 3; i++) {
            t[i].w = w8[i];
            t[i].M = 1;
            t[i].A = dA;
            t[i].C = dC + (size_t)i * N;
            t[i].cstride = 0;
        }
        REQ(ork_i8_mm_run_chain(c, 3, t) == 0);
        int8_t *hA = calloc(16, K);
        int32_t *hC = malloc((size_t)16 * N * 4);
        ork_npu_set_async(c, 0);
        for (int M = 1; M <= 16; M += 15) REQ(ork_i8_mm_run(c, w8[0], M, hA, hC) == 0);
        ork_npu_set_async(c, 1);
        free(hA);
        free(hC);
        for (int i = 0; i < 3; i++) ork_mm_free(c, w8[i]);
        const int K2 = 512, N2 = 512;
        ork_f16 *B2 = malloc((size_t)K2 * N2 * 2);
        for (size_t i = 0; i < (size_t)K2 * N2; i++) B2[i] = (ork_f16)(0.02f * nrand());
        ork_w *wf = ork_f16_mm_pack(c, K2, N2, B2);
        ork_f16 *dA2 = ork_dev_alloc(c, (size_t)512 * K2 * 2);
        REQ(wf && dA2);
        for (int M = 1; M <= 512; M *= 2) REQ(ork_f16_mm_run(c, wf, M, dA2, (float *)dC) == 0);
        ork_mm_free(c, wf);
        ork_dev_free(c, dA2);
        free(B2);
        const int K4 = 1024, N4 = 512;
        int8_t *B4 = malloc((size_t)K4 * N4);
        for (size_t i = 0; i < (size_t)K4 * N4; i++) B4[i] = (int8_t)((int)(urand() * 16) - 8);
        ork_w *w4 = ork_i4_mm_pack(c, K4, N4, B4);
        int8_t *dA4 = ork_dev_alloc(c, (size_t)256 * K4);
        REQ(w4 && dA4 && ork_i4_mm_run(c, w4, 256, dA4, dC) == 0);
        ork_mm_free(c, w4);
        ork_w *wg = ork_i4_mm_pack_grouped(c, K4, N4, B4, 128);
        float *aS = ork_dev_alloc(c, (size_t)256 * (K4 / 128) * 4), *bS = ork_dev_alloc(c, (size_t)(K4 / 128) * N4 * 4);
        float *dCf = ork_dev_alloc(c, (size_t)256 * N4 * 4);
        REQ(wg && aS && bS && dCf);
        for (int M = 1; M <= 256; M *= 256) REQ(ork_i4_mm_run_grouped(c, wg, M, dA4, aS, bS, dCf) == 0);
        ork_mm_free(c, wg);
        ork_dev_free(c, dA4);
        ork_dev_free(c, aS);
        ork_dev_free(c, bS);
        ork_dev_free(c, dCf);
        free(B4);
    }
    ork_dev_free(c, dA);
    ork_dev_free(c, dC);
    ork_npu_free(c);
    free(W);
    free(im);
    free(bs);
    printf("done\n");
    return 0;
}
