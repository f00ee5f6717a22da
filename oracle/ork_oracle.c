/* oracle/ork_oracle.c -- CPU restatement of ork-driver's resident-weight matmul path.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker, never the product: only tests/, the smoke()
 * check in __graft_entry__.py and bench.py's cpu_baseline leg load it. The product library
 * (ork-driver_amd/) never links, loads or calls anything here, and has no CPU fallback onto it.
 *
 * Every function restates one reference function; the citation (path:line, relative to the
 * reference tree) is on each definition. Float semantics follow the reference as compiled for x86:
 * IEEE binary32, round-to-nearest-even (lrintf under the default rounding mode), multiply by the
 * reciprocal where the reference multiplies, divide where it divides, and no FMA contraction
 * (build with -ffp-contract=off). The NEON branches of the reference are bit-identical to its
 * scalar branches (the reference says so at each site and its own tests assert it), so only the
 * scalar semantics are restated.
 *
 * What pins each function (tests/test_oracle_golden.py, tests/test_oracle_pins.py):
 *   oracle_gemm_i32          the reference's FNV-64 goldens (examples/quant.c:72-81, test_matmul.c chains),
 *                            the reference's own compiled orki_cpu_gemm_i32 (oracle/_ref), brute force
 *   oracle_gemm_f16_*        test_matmul.c:611-612 goldens (integer-valued inputs: every sum exact)
 *   oracle_chan_scales_f32, oracle_quant_i8, oracle_pack_i8_f32
 *                            exact half-even ties, the 1e-9 floor, max|q| = 127, the half-step error
 *                            bound, the reference's 3% RMS gate (test_matmul.c:280-306)
 *   oracle_i4_quant_chan     the reference's own compiled orki_i4_quant_chan (oracle/_ref), RN and SR
 *   oracle_nf4_lut, oracle_nf4_quant_chan (RN)
 *                            the int8 codebook, nearest level by brute force, the exact float32 ties
 *                            t == 0.5f -> upper level (quant.c:84), the NF4 < uniform gate
 *                            (test_matmul.c:402-427)
 *   oracle_nf4_quant_chan (SR)  bracket, P(hi) = t, the xorshift32 stream (the same generator the
 *                            compiled reference's uniform SR draws, oracle/_ref) and which elements draw;
 *                            PARITY UNPINNED against a compiled reference for the NF4 draw coupling across
 *                            channels (src/npu.c, which holds the NF4 levels, does not compile on x86, so
 *                            no compiled reference NF4 exists here: that order is the source read as text)
 *   oracle_wq_err_chan, oracle_wq_best_absmax
 *                            grid membership and float64 argmin, every candidate's error equal to an
 *                            independent float32 sequential sum bit for bit, exact ties keep the first
 *                            candidate, NULL path = absmax/7, the importance gate (test_matmul.c:430-500);
 *                            PARITY UNPINNED against a reference build that contracts `e += im*d*d` into a
 *                            fused multiply-add (GCC's default on aarch64): its float32 near-ties may differ
 *   oracle_i4a8_blob, oracle_o4n1_decode
 *                            header bytes, offsets, size (test_matmul.c:528), round trip, rejections,
 *                            qerr recomputed in float64
 *   oracle_gemm_grouped      the reference's own compiled orki_cpu_gemm_grouped (oracle/_ref), bit for bit;
 *                            a numpy float32 restatement; G = K reduces to one scaled int32 GEMM
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORACLE_API __attribute__((visibility("default")))

/* ------------------------------------------------------------------------------------------ */
/* FNV-1a 64, over raw little-endian bytes: examples/quant.c:24-25, examples/test_matmul.c:16-18 */
ORACLE_API uint64_t oracle_fnv64(uint64_t h, const void *p, size_t n) {
    const uint8_t *b = (const uint8_t *)p;
    for (size_t i = 0; i < n; i++) { h ^= b[i]; h *= 1099511628211ULL; }
    return h;
}

/* ------------------------------------------------------------------------------------------ */
/* Exact int32 GEMM, k-outer AXPY with the zero-activation skip: src/npu/core/buf.c:428-477.
 * B is raw codes [K][N] (k-major). C is overwritten. */
ORACLE_API void oracle_gemm_i32(int M, int K, int N, const int8_t *A, const int8_t *B, int32_t *C) {
    for (int m = 0; m < M; m++) {
        const int8_t *arow = A + (size_t)m * K;
        int32_t *crow = C + (size_t)m * N;
        memset(crow, 0, (size_t)N * sizeof *crow);
        for (int k = 0; k < K; k++) {
            const int32_t a = arow[k];
            if (!a) continue;
            const int8_t *wrow = B + (size_t)k * N;
            for (int n = 0; n < N; n++) crow[n] += a * (int32_t)wrow[n];
        }
    }
}

/* The naive triple loop the reference uses as its own scalar reference: examples/test_cpu_gemm.c:26-32 */
ORACLE_API void oracle_gemm_i32_naive(int M, int K, int N, const int8_t *A, const int8_t *B, int32_t *C) {
    for (int m = 0; m < M; m++)
        for (int n = 0; n < N; n++) {
            int32_t s = 0;
            for (int k = 0; k < K; k++) s += (int32_t)A[(size_t)m * K + k] * (int32_t)B[(size_t)k * N + n];
            C[(size_t)m * N + n] = s;
        }
}

/* ------------------------------------------------------------------------------------------ */
/* Per-channel int8 scales: src/npu.c:854-865.  mx = max(1e-9, max|w|); inv = 127/mx; bscale = mx/127 */
/* src/npu/core/buf.c:501-520 orki_cpu_gemm_grouped: per K-group int32 partials (exact), each scaled as
 * ((float)acc * aScale[m*Sk+g]) * bScale[g*N+n] and added to C in ascending g, from 0.0f. */
ORACLE_API int oracle_gemm_grouped(int M, int K, int N, int G, const int8_t *A, const int8_t *codes_kn,
                                   const float *aScale, const float *bScale, float *C) {
    if (M < 1 || K < 1 || N < 1 || G < 1 || K % G) return -1;
    const int Sk = K / G;
    int32_t *acc = malloc((size_t)N * sizeof *acc);
    if (!acc) return -1;
    for (int m = 0; m < M; m++) {
        float *cr = C + (size_t)m * N;
        for (int n = 0; n < N; n++) cr[n] = 0.0f;
        for (int g = 0; g < Sk; g++) {
            const float as = aScale[(size_t)m * Sk + g];
            const float *bs = bScale + (size_t)g * N;
            oracle_gemm_i32(1, G, N, A + (size_t)m * K + (size_t)g * G, codes_kn + (size_t)g * G * N, acc);
            for (int n = 0; n < N; n++) cr[n] += (float)acc[n] * as * bs[n];
        }
    }
    free(acc);
    return 0;
}

ORACLE_API void oracle_chan_scales_f32(const float *f32, int K, int N, float *inv, float *bscale) {
    for (int n = 0; n < N; n++) {
        const float *fr = f32 + (size_t)n * K;
        float mx = 1e-9f;
        for (int k = 0; k < K; k++) { float v = fabsf(fr[k]); if (v > mx) mx = v; }
        inv[n] = 127.0f / mx;
        if (bscale) bscale[n] = mx / 127.0f;
    }
}

/* quant32_f32_i8 (src/npu/i8/pack.c:442-453): q = clamp(lrintf(f*inv), -127, 127), applied to every
 * element of channel n exactly as orki_i8_tile_f32 (src/npu/i8/pack.c:455-473) does. The oracle emits
 * the LOGICAL codes in the reference's offline layout [K][N] (cpu_codes, src/npu/i8/pack.c:48-55);
 * tiling is a layout, not arithmetic. */
ORACLE_API void oracle_quant_i8(const float *f32, int K, int N, const float *inv, int8_t *codes_kn) {
    for (int n = 0; n < N; n++) {
        const float *fr = f32 + (size_t)n * K;
        const float iv = inv[n];
        for (int k = 0; k < K; k++) {
            int q = (int)lrintf(fr[k] * iv);
            codes_kn[(size_t)k * N + n] = (int8_t)(q > 127 ? 127 : q < -127 ? -127 : q);
        }
    }
}

/* ork_i8_mm_pack_f32 (src/npu/i8/pack.c:475-494): dims gate, scales, quant. Returns 0, or -1 on bad dims. */
ORACLE_API int oracle_pack_i8_f32(int K, int N, const float *f32, float *bscale, int8_t *codes_kn) {
    if (K % 32 || N % 32) return -1;
    float *inv = malloc((size_t)N * sizeof(float));
    if (!inv) return -1;
    oracle_chan_scales_f32(f32, K, N, inv, bscale);
    oracle_quant_i8(f32, K, N, inv, codes_kn);
    free(inv);
    return 0;
}

/* ------------------------------------------------------------------------------------------ */
/* NF4 levels: src/npu.c:888-892 (the 16 bitsandbytes NF4 normalised levels) */
ORACLE_API const float ORACLE_NF4_LEVELS[16] = {
    -1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f,
    -0.28444138169288635f, -0.18477343022823334f, -0.09105003625154495f, 0.0f,
    0.07958029955625534f, 0.16093020141124725f, 0.24611230194568634f, 0.33791524171829224f,
    0.44070982933044434f, 0.5626170039176941f, 0.7229568362236023f, 1.0f};

/* int8 LUT of the NF4 codebook: lut[i] = (int8_t)lrintf(level[i]*127) (src/npu/i4/pack.c:57) */
ORACLE_API void oracle_nf4_lut(int8_t lut[16]) {
    for (int i = 0; i < 16; i++) lut[i] = (int8_t)lrintf(ORACLE_NF4_LEVELS[i] * 127.0f);
}

/* xorshift32 for stochastic rounding: src/npu/internal.h:589 */
static inline uint32_t oracle_xs32(uint32_t *s) {
    uint32_t x = *s; x ^= x << 13; x ^= x >> 17; x ^= x << 5; *s = x; return x;
}

/* Uniform int4 channel quant: src/npu/i4/quant.c:28-40. codes[k] receives the int code in [-7,7]. */
ORACLE_API void oracle_i4_quant_chan(const float *fr, int K, float scale, int sr, uint32_t *seed,
                                     uint8_t *nib, int8_t *codes) {
    float inv = scale > 0 ? 1.0f / scale : 0.0f;
    for (int k = 0; k < K; k++) {
        int q;
        if (sr) {
            float u = (float)(oracle_xs32(seed) >> 8) * (1.0f / 16777216.0f);
            float t = fr[k] * inv;
            q = (int)floorf(t + u);
        } else {
            q = (int)lrintf(fr[k] * inv);
        }
        if (q > 7) q = 7; else if (q < -7) q = -7;
        codes[k] = (int8_t)q;
        uint8_t nb = (uint8_t)(q & 0xf);
        if (k & 1) nib[k >> 1] |= (uint8_t)(nb << 4); else nib[k >> 1] = nb;
    }
}

/* NF4 bracketing index for a normalised weight (src/npu/i4/quant.c:73-76, :78-84 with sr=0) */
static int oracle_nf4_bracket(float wn, int *lo_out, int *hi_out) {
    if (wn > 1.0f) wn = 1.0f; else if (wn < -1.0f) wn = -1.0f;
    int hi = 0;
    while (hi < 15 && ORACLE_NF4_LEVELS[hi] < wn) hi++;
    *lo_out = hi > 0 ? hi - 1 : 0;
    *hi_out = hi;
    return 0;
}

/* NF4 channel quant: src/npu/i4/quant.c:70-90. qidx[k] receives the 0..15 index. */
ORACLE_API void oracle_nf4_quant_chan(const float *fr, int K, float absmax, int sr, uint32_t *seed,
                                      uint8_t *nib, uint8_t *qidx) {
    float inv = absmax > 0 ? 1.0f / absmax : 0.0f;
    for (int k = 0; k < K; k++) {
        float wn = fr[k] * inv;
        if (wn > 1.0f) wn = 1.0f; else if (wn < -1.0f) wn = -1.0f;
        int lo, hi, idx;
        oracle_nf4_bracket(wn, &lo, &hi);
        if (lo == hi) idx = hi;
        else {
            float dlo = ORACLE_NF4_LEVELS[hi] - ORACLE_NF4_LEVELS[lo];
            float t = (wn - ORACLE_NF4_LEVELS[lo]) / dlo;
            if (sr) {
                float u = (float)(oracle_xs32(seed) >> 8) * (1.0f / 16777216.0f);
                idx = (t > u) ? hi : lo;
            } else idx = (t >= 0.5f) ? hi : lo;
        }
        qidx[k] = (uint8_t)idx;
        uint8_t nb = (uint8_t)(idx & 0xf);
        if (k & 1) nib[k >> 1] |= (uint8_t)(nb << 4); else nib[k >> 1] = nb;
    }
}

/* Importance-weighted reconstruction error of one channel at a candidate absmax:
 * src/npu/i4/quant.c:130-151 (float, sequential accumulation, no contraction). */
ORACLE_API float oracle_wq_err_chan(const float *fr, int K, float absmax, int nf4, const float *im, float *dq) {
    if (nf4) {
        float sc = absmax / 127.0f, inv = absmax > 0 ? 1.0f / absmax : 0.0f;
        for (int k = 0; k < K; k++) {
            float wn = fr[k] * inv;
            if (wn > 1.0f) wn = 1.0f; else if (wn < -1.0f) wn = -1.0f;
            int lo, hi, idx;
            oracle_nf4_bracket(wn, &lo, &hi);
            if (lo == hi) idx = hi;
            else {
                float t = (wn - ORACLE_NF4_LEVELS[lo]) / (ORACLE_NF4_LEVELS[hi] - ORACLE_NF4_LEVELS[lo]);
                idx = (t >= 0.5f) ? hi : lo;
            }
            dq[k] = (float)((int8_t)lrintf(ORACLE_NF4_LEVELS[idx] * 127.0f)) * sc;
        }
    } else {
        float scale = absmax / 7.0f, inv = scale > 0 ? 1.0f / scale : 0.0f;
        for (int k = 0; k < K; k++) {
            int q = (int)lrintf(fr[k] * inv);
            if (q > 7) q = 7; else if (q < -7) q = -7;
            dq[k] = (float)q * scale;
        }
    }
    float e = 0.0f;
    for (int k = 0; k < K; k++) {
        float d = fr[k] - dq[k];
        float w = (im ? im[k] : 1.0f) * d;
        w = w * d;
        e = e + w;
    }
    return e;
}

/* Clip-grid search: src/npu/i4/quant.c:26 (grid), :153-161 (first strict minimum wins) */
static const float ORACLE_IM_CLIP_GRID[7] = {1.0f, 0.92f, 0.85f, 0.78f, 0.70f, 0.62f, 0.55f};
ORACLE_API float oracle_wq_best_absmax(const float *fr, int K, float rawabsmax, int nf4, const float *im, float *dq) {
    float best_abs = rawabsmax, best_e = oracle_wq_err_chan(fr, K, rawabsmax, nf4, im, dq);
    for (int g = 1; g < 7; g++) {
        float cand = rawabsmax * ORACLE_IM_CLIP_GRID[g];
        float e = oracle_wq_err_chan(fr, K, cand, nf4, im, dq);
        if (e < best_e) { best_e = e; best_abs = cand; }
    }
    return best_abs;
}

/* Channel absmax with the 1e-9 floor (src/npu/i4/pack.c:64-70) */
static float oracle_chan_absmax(const float *fr, int K) {
    float mx = 1e-9f;
    for (int k = 0; k < K; k++) { float v = fabsf(fr[k]); if (v > mx) mx = v; }
    return mx;
}

/* ork_i4a8_mm_pack_im (src/npu/i4/pack.c:30-87) with ORK_SR / ORK_NF4 as explicit flags.
 * Outputs: bscale[N]; nib[N][K/2] (the compact store, low nibble = even k); codes_kn[K][N], the
 * int8 codes the packed weight multiplies with (uniform: sign-extended nibble, pack.c:83 + quant.c:42-68;
 * NF4: lut[idx], pack.c:82 + quant.c:92-108). Returns 0, or -1 on bad dims. */
ORACLE_API int oracle_pack_i4a8(int K, int N, const float *f32, const float *imatrix, int nf4, int sr,
                                float *bscale, uint8_t *nib, int8_t *codes_kn) {
    if (K % 32 || N % 32) return -1;
    uint32_t seed = 0x2545F491u;
    int8_t lut[16];
    oracle_nf4_lut(lut);
    int8_t *codes = malloc((size_t)K);
    uint8_t *qidx = malloc((size_t)K);
    float *imdq = malloc((size_t)K * sizeof(float));
    if (!codes || !qidx || !imdq) { free(codes); free(qidx); free(imdq); return -1; }
    for (int n = 0; n < N; n++) {
        const float *fr = f32 + (size_t)n * K;
        float mx = oracle_chan_absmax(fr, K);
        if (imatrix) mx = oracle_wq_best_absmax(fr, K, mx, nf4, imatrix, imdq);
        uint8_t *nb = nib + (size_t)n * (K / 2);
        if (nf4) {
            bscale[n] = mx / 127.0f;
            oracle_nf4_quant_chan(fr, K, mx, sr, &seed, nb, qidx);
            for (int k = 0; k < K; k++) codes[k] = lut[qidx[k]];
        } else {
            float scale = mx / 7.0f;
            bscale[n] = scale;
            oracle_i4_quant_chan(fr, K, scale, sr, &seed, nb, codes);
        }
        if (codes_kn)
            for (int k = 0; k < K; k++) codes_kn[(size_t)k * N + n] = codes[k];
    }
    free(codes); free(qidx); free(imdq);
    return 0;
}

/* O4N1 blob: header {u32 magic 'O4N1'=0x4F344E31, u32 version=1, i32 K, i32 N, u32 quant_kind} (20 B, LE)
 * + f32 bscale[N] + Bi4[K*N/2]: src/npu/internal.h:584,597; src/npu/i4/pack.c:91-103. */
#define ORACLE_O4N1_MAGIC 0x4F344E31u
#define ORACLE_PACK_FORMAT_VERSION 1u /* include/ork_npu.h:37; src/npu/core/device.c:385 */

/* ork_i4a8_pack_cpu_blob_qerr (src/npu/i4/pack.c:814-863). Returns the blob size (out==NULL: required
 * size), or 0 on bad dims / small cap. qerr_out may be NULL. */
ORACLE_API size_t oracle_i4a8_blob(int K, int N, const float *f32, const float *imatrix, int nf4, int sr,
                                   void *out, size_t cap, float *qerr_out) {
    if (K % 32 || N % 32 || !f32) return 0;
    size_t hdr = 20, sc = (size_t)N * sizeof(float), nibsz = (size_t)K * N / 2, need = hdr + sc + nibsz;
    if (!out) return need;
    if (cap < need) return 0;
    nf4 = nf4 ? 1 : 0;
    uint32_t seed = 0x2545F491u;
    uint8_t *p = (uint8_t *)out;
    float *bscale = malloc(sc);
    uint8_t *Bi4 = p + hdr + sc;
    int8_t *codes = malloc((size_t)K);
    uint8_t *qidx = malloc((size_t)K);
    float *imdq = malloc((size_t)K * sizeof(float));
    if (!bscale || !codes || !qidx || !imdq) { free(bscale); free(codes); free(qidx); free(imdq); return 0; }
    int8_t lut[16];
    oracle_nf4_lut(lut);
    double qnum = 0.0, qden = 0.0;
    for (int n = 0; n < N; n++) {
        const float *fr = f32 + (size_t)n * K;
        float mx = oracle_chan_absmax(fr, K);
        if (imatrix) mx = oracle_wq_best_absmax(fr, K, mx, nf4, imatrix, imdq);
        uint8_t *nib = Bi4 + (size_t)n * (K / 2);
        if (nf4) {
            bscale[n] = mx / 127.0f;
            oracle_nf4_quant_chan(fr, K, mx, sr, &seed, nib, qidx);
            for (int k = 0; k < K; k++) codes[k] = lut[qidx[k]];
        } else {
            float scale = mx / 7.0f;
            bscale[n] = scale;
            oracle_i4_quant_chan(fr, K, scale, sr, &seed, nib, codes);
        }
        if (qerr_out) {
            const float bs = bscale[n];
            for (int kk = 0; kk < K; kk++) {
                double w = fr[kk], q = (double)(float)codes[kk] * bs, d = w - q;
                double imp = imatrix ? imatrix[kk] : 1.0;
                qnum += imp * d * d;
                qden += imp * w * w;
            }
        }
    }
    if (qerr_out) *qerr_out = qden > 0.0 ? (float)sqrt(qnum / qden) : 0.0f;
    uint32_t h[5] = {ORACLE_O4N1_MAGIC, ORACLE_PACK_FORMAT_VERSION, (uint32_t)K, (uint32_t)N,
                     (uint32_t)(nf4 ? 1 : 0)};
    memcpy(p, h, hdr);
    memcpy(p + hdr, bscale, sc);
    free(bscale); free(codes); free(qidx); free(imdq);
    return need;
}

/* O4N1 validation + offline inflate: src/npu/i4/pack.c:115-150. Returns 0 and fills bscale[N] and
 * codes_kn[K][N]; -1 when the reference loader would return NULL. */
ORACLE_API int oracle_o4n1_decode(int K, int N, const void *blob, size_t n, float *bscale, int8_t *codes_kn) {
    if (K % 32 || N % 32) return -1;
    size_t hdr = 20, sc = (size_t)N * sizeof(float), nib = (size_t)K * N / 2;
    if (n != hdr + sc + nib) return -1;
    const uint8_t *p = (const uint8_t *)blob;
    uint32_t h[5];
    memcpy(h, p, hdr);
    if (h[0] != ORACLE_O4N1_MAGIC || h[1] != ORACLE_PACK_FORMAT_VERSION || (int32_t)h[2] != K || (int32_t)h[3] != N)
        return -1;
    if (h[4] != 0 && h[4] != 1) return -1;
    memcpy(bscale, p + hdr, sc);
    const uint8_t *nibs = p + hdr + sc;
    int8_t lut[16];
    oracle_nf4_lut(lut);
    for (int nn = 0; nn < N; nn++) {
        const uint8_t *nb = nibs + (size_t)nn * (K / 2);
        for (int k = 0; k < K; k++) {
            uint8_t ix = (k & 1) ? (nb[k >> 1] >> 4) : (nb[k >> 1] & 0xf);
            codes_kn[(size_t)k * N + nn] = (h[4] == 1) ? lut[ix] : (int8_t)(ix >= 8 ? (int)ix - 16 : (int)ix);
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------------------------ */
/* fp16 helpers. IEEE binary16 -> binary32 is exact; written from the format definition. */
ORACLE_API float oracle_h2f(uint16_t h) {
    uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 0x1f, m = h & 0x3ff, u;
    if (e == 0) {
        if (m == 0) u = s;
        else { /* subnormal: normalise */
            int sh = 0;
            while (!(m & 0x400)) { m <<= 1; sh++; }
            m &= 0x3ff;
            u = s | ((uint32_t)(127 - 15 - sh + 1) << 23) | (m << 13);
        }
    } else if (e == 31) u = s | 0x7f800000u | (m << 13);
    else u = s | ((e - 15 + 127) << 23) | (m << 13);
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* fp16 GEMM with fp32 accumulation in k order -- the reference's own check loop
 * (examples/test_matmul.c:37). A [M][K], B [K][N] row-major fp16 bits. */
ORACLE_API void oracle_gemm_f16_f32acc(int M, int K, int N, const uint16_t *A, const uint16_t *B, float *C) {
    for (int m = 0; m < M; m++)
        for (int n = 0; n < N; n++) {
            float ref = 0;
            for (int k = 0; k < K; k++) {
                float p = oracle_h2f(A[(size_t)m * K + k]) * oracle_h2f(B[(size_t)k * N + n]);
                ref = ref + p;
            }
            C[(size_t)m * N + n] = ref;
        }
}

/* fp16 GEMM with fp64 accumulation: the tolerance reference for the fp16 path. Products of two
 * binary16 values are exact in binary64, so only the sum order rounds (at 2^-53). */
ORACLE_API void oracle_gemm_f16_f64acc(int M, int K, int N, const uint16_t *A, const uint16_t *B, double *C) {
    float *bf = malloc((size_t)K * N * sizeof(float));
    if (!bf) return;
    for (size_t i = 0; i < (size_t)K * N; i++) bf[i] = oracle_h2f(B[i]);
    double *row = malloc((size_t)N * sizeof(double));
    for (int m = 0; m < M; m++) {
        for (int n = 0; n < N; n++) row[n] = 0.0;
        for (int k = 0; k < K; k++) {
            double a = oracle_h2f(A[(size_t)m * K + k]);
            if (a == 0.0) continue;
            const float *br = bf + (size_t)k * N;
            for (int n = 0; n < N; n++) row[n] += a * (double)br[n];
        }
        memcpy(C + (size_t)m * N, row, (size_t)N * sizeof(double));
    }
    free(row);
    free(bf);
}

/* ------------------------------------------------------------------------------------------ */
/* Input generators of the reference's own tests, so their embedded goldens can be replayed. */

/* examples/quant.c:18  frand(): sd=sd*1103515245+12345; ((int)((sd>>9)&0x3fff)-8192)/16384.0f */
ORACLE_API void oracle_gen_quant_frand(uint32_t *sd, float *out, size_t n) {
    uint32_t s = *sd;
    for (size_t i = 0; i < n; i++) {
        s = s * 1103515245u + 12345u;
        out[i] = ((int)((s >> 9) & 0x3fff) - 8192) / 16384.0f;
    }
    *sd = s;
}

/* examples/quant.c:19 q8() and :30-37 (the test's own quantisation: divide by the scale) */
static int8_t oracle_q8(float x) { int q = (int)lrintf(x); return (int8_t)(q < -127 ? -127 : q > 127 ? 127 : q); }
ORACLE_API void oracle_quant_test_weights(int K, int N, const float *B, float *ws, int8_t *Bq) {
    for (int n = 0; n < N; n++) {
        float mx = 0;
        for (int k = 0; k < K; k++) { float a = fabsf(B[(size_t)k * N + n]); if (a > mx) mx = a; }
        ws[n] = mx > 0 ? mx / 127.0f : 1.0f;
        for (int k = 0; k < K; k++) Bq[(size_t)k * N + n] = oracle_q8(B[(size_t)k * N + n] / ws[n]);
    }
}
ORACLE_API void oracle_quant_test_acts(int M, int K, const float *A, float *as, int8_t *Aq) {
    for (int m = 0; m < M; m++) {
        float mx = 0;
        for (int k = 0; k < K; k++) { float a = fabsf(A[(size_t)m * K + k]); if (a > mx) mx = a; }
        as[m] = mx > 0 ? mx / 127.0f : 1.0f;
        for (int k = 0; k < K; k++) Aq[(size_t)m * K + k] = oracle_q8(A[(size_t)m * K + k] / as[m]);
    }
}

/* examples/test_matmul.c:11  rnd(): sd=sd*1103515245+12345; (sd>>16)%4. Emits the raw 0..3 values. */
ORACLE_API void oracle_gen_tm_rnd(uint32_t *sd, uint8_t *out, size_t n) {
    uint32_t s = *sd;
    for (size_t i = 0; i < n; i++) {
        s = s * 1103515245u + 12345u;
        out[i] = (uint8_t)((s >> 16) % 4);
    }
    *sd = s;
}

/* Jump the 32-bit LCG x -> a*x + c by n steps (affine-map squaring). Used to skip the inputs of
 * tests whose goldens are not replayed but whose rnd() draws move the shared stream. */
ORACLE_API uint32_t oracle_lcg_skip(uint32_t x, uint64_t n) {
    uint32_t a = 1103515245u, c = 12345u, A = 1u, C = 0u;
    while (n) {
        if (n & 1) { A = A * a; C = C * a + c; }
        c = c * (a + 1u);
        a = a * a;
        n >>= 1;
    }
    return A * x + C;
}

/* examples/i4.c:16-18  W4A4 inputs: sd=99+M*7+K*13+N*17; v=(int8)((int)((sd>>17)%15)-7) for A then B */
ORACLE_API void oracle_gen_i4_test(int M, int K, int N, int8_t *A, int8_t *B) {
    uint32_t sd = 99u + (uint32_t)(M * 7 + K * 13 + N * 17);
    for (size_t i = 0; i < (size_t)M * K; i++) { sd = sd * 1103515245u + 12345u; A[i] = (int8_t)((int)((sd >> 17) % 15) - 7); }
    for (size_t i = 0; i < (size_t)K * N; i++) { sd = sd * 1103515245u + 12345u; B[i] = (int8_t)((int)((sd >> 17) % 15) - 7); }
}

/* examples/i4.c:37-46  the 0x7fff construction (one output cell is exactly 32767) */
ORACLE_API void oracle_gen_i4_sattest(int M, int K, int N, int8_t *A, int8_t *B) {
    memset(A, 0, (size_t)M * K);
    memset(B, 0, (size_t)K * N);
    uint32_t sd = 4242u + (uint32_t)(M * K * N);
    for (size_t i = 0; i < (size_t)M * K; i++) { sd = sd * 1103515245u + 12345u; A[i] = (int8_t)((int)((sd >> 17) % 15) - 7); }
    for (size_t i = 0; i < (size_t)K * N; i++) { sd = sd * 1103515245u + 12345u; B[i] = (int8_t)((int)((sd >> 17) % 15) - 7); }
    for (int k = 0; k < K; k++) { A[k] = 7; B[(size_t)k * N] = 0; }
    for (int k = 0; k < 668; k++) B[(size_t)k * N] = 7;
    B[(size_t)668 * N] = 5;
}

/* examples/test_cpu_gemm.c:22-23  xorshift rnd(lo,hi), state g=7777 carried across cases */
ORACLE_API void oracle_gen_cpu_gemm(uint32_t *g, int lo, int hi, int8_t *out, size_t n) {
    uint32_t s = *g;
    for (size_t i = 0; i < n; i++) {
        s ^= s << 13; s ^= s >> 17; s ^= s << 5;
        out[i] = (int8_t)(lo + (int)(s % (uint32_t)(hi - lo + 1)));
    }
    *g = s;
}

/* examples/test_matmul.c:339-340  Box-Muller gauss() with its own LCG gsd (initial 99173) */
ORACLE_API void oracle_gen_tm_gauss(uint32_t *gsd, float *out, size_t n) {
    uint32_t s = *gsd;
    for (size_t i = 0; i < n; i++) {
        s = s * 1103515245u + 12345u;
        double u1 = ((s >> 8) & 0xffffff) / 16777216.0 + 1e-9;
        s = s * 1103515245u + 12345u;
        double u2 = ((s >> 8) & 0xffffff) / 16777216.0 + 1e-9;
        out[i] = (float)(sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2));
    }
    *gsd = s;
}
