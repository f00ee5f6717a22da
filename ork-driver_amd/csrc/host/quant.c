/* quant.c -- host-side weight quantisation (pack time), bit-exact with the reference.
 *
 * Semantics (each function cites the reference code it must agree with bit for bit):
 *   per-channel int8     src/npu.c:854-865 (scales), src/npu/i8/pack.c:442-453 (quant32_f32_i8)
 *   uniform int4         src/npu/i4/quant.c:28-40, src/npu/i4/pack.c:64-80
 *   NF4 codebook         src/npu.c:888-892 (levels), src/npu/i4/quant.c:70-90, src/npu/i4/pack.c:57
 *   imatrix clip search  src/npu/i4/quant.c:26, :130-161
 *   stochastic rounding  src/npu/internal.h:589 (xorshift32), seed 0x2545F491 (src/npu/i4/pack.c:32)
 * Float rules that make the match exact: IEEE binary32 throughout, multiply by the reciprocal where
 * the reference does, lrintf (round half to even) for rounding, the 1e-9 absmax floor, first strict
 * minimum on the clip grid, and no FMA contraction (this file is built with -ffp-contract=off).
 * Channels are independent unless stochastic rounding couples them through the shared xorshift
 * stream, so the deterministic paths run channel-parallel on the host pool. */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "internal.h"

const float ORKI_NF4_LEVELS[16] = {
    -1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f,
    -0.28444138169288635f, -0.18477343022823334f, -0.09105003625154495f, 0.0f,
    0.07958029955625534f, 0.16093020141124725f, 0.24611230194568634f, 0.33791524171829224f,
    0.44070982933044434f, 0.5626170039176941f, 0.7229568362236023f, 1.0f};

static const float CLIP_GRID[7] = {1.0f, 0.92f, 0.85f, 0.78f, 0.70f, 0.62f, 0.55f};

void orki_nf4_lut(int8_t lut[16]) {
    for (int i = 0; i < 16; i++) lut[i] = (int8_t)lrintf(ORKI_NF4_LEVELS[i] * 127.0f);
}

uint32_t orki_xs32(uint32_t *s) {
    uint32_t x = *s;
    x ^= x << 13;
    x ^= x >> 17;
    x ^= x << 5;
    *s = x;
    return x;
}

float orki_chan_absmax(const float *fr, int K) {
    float mx = 1e-9f;
    for (int k = 0; k < K; k++) {
        const float v = fabsf(fr[k]);
        mx = v > mx ? v : mx;
    }
    return mx;
}

/* ---- per-channel int8 --------------------------------------------------------------------------- */
struct i8q { const float *f32; int K; float *bscale; int8_t *codes; };
static void i8q_range(int lo, int hi, void *a) {
    struct i8q *q = a;
    for (int n = lo; n < hi; n++) {
        const float *fr = q->f32 + (size_t)n * q->K;
        const float mx = orki_chan_absmax(fr, q->K);
        const float inv = 127.0f / mx;
        q->bscale[n] = mx / 127.0f;
        int8_t *dst = q->codes + (size_t)n * q->K;
        for (int k = 0; k < q->K; k++) {
            const long v = lrintf(fr[k] * inv);
            dst[k] = (int8_t)(v > 127 ? 127 : v < -127 ? -127 : v);
        }
    }
}

void orki_i8_quant_chans(const float *f32, int K, int N, float *bscale, int8_t *codes_nk) {
    struct i8q q = {f32, K, bscale, codes_nk};
    orki_parallel_for(N, i8q_range, &q);
}

/* ---- int4 / NF4 --------------------------------------------------------------------------------- */
static inline void put_nib(uint8_t *nib, int k, unsigned v) {
    if (k & 1) nib[k >> 1] |= (uint8_t)((v & 0xf) << 4);
    else nib[k >> 1] = (uint8_t)(v & 0xf);
}

void orki_i4_quant_chan(const float *fr, int K, float scale, int sr, uint32_t *seed, uint8_t *nib, int8_t *codes) {
    const float inv = scale > 0 ? 1.0f / scale : 0.0f;
    for (int k = 0; k < K; k++) {
        int q;
        if (sr) {
            const float u = (float)(orki_xs32(seed) >> 8) * (1.0f / 16777216.0f);
            const float t = fr[k] * inv;
            q = (int)floorf(t + u);
        } else {
            q = (int)lrintf(fr[k] * inv);
        }
        q = q > 7 ? 7 : q < -7 ? -7 : q;
        if (codes) codes[k] = (int8_t)q;
        put_nib(nib, k, (unsigned)q);
    }
}

/* Index of the nearest NF4 level (ties to the upper level), or the stochastic pick, for wn in [-1,1]. */
static inline int nf4_index(float wn, int sr, uint32_t *seed) {
    int hi = 0;
    while (hi < 15 && ORKI_NF4_LEVELS[hi] < wn) hi++;
    if (hi == 0) return 0;
    const int lo = hi - 1;
    const float t = (wn - ORKI_NF4_LEVELS[lo]) / (ORKI_NF4_LEVELS[hi] - ORKI_NF4_LEVELS[lo]);
    if (sr) {
        const float u = (float)(orki_xs32(seed) >> 8) * (1.0f / 16777216.0f);
        return t > u ? hi : lo;
    }
    return t >= 0.5f ? hi : lo;
}

void orki_nf4_quant_chan(const float *fr, int K, float absmax, int sr, uint32_t *seed, uint8_t *nib, uint8_t *idx) {
    const float inv = absmax > 0 ? 1.0f / absmax : 0.0f;
    for (int k = 0; k < K; k++) {
        float wn = fr[k] * inv;
        wn = wn > 1.0f ? 1.0f : wn < -1.0f ? -1.0f : wn;
        const int i = nf4_index(wn, sr, seed);
        if (idx) idx[k] = (uint8_t)i;
        put_nib(nib, k, (unsigned)i);
    }
}

/* Importance-weighted squared reconstruction error at one candidate absmax (float, k order). */
static float wq_err(const float *fr, int K, float absmax, int nf4, const float *im, const int8_t lut[16]) {
    float e = 0.0f;
    if (nf4) {
        const float sc = absmax / 127.0f, inv = absmax > 0 ? 1.0f / absmax : 0.0f;
        for (int k = 0; k < K; k++) {
            float wn = fr[k] * inv;
            wn = wn > 1.0f ? 1.0f : wn < -1.0f ? -1.0f : wn;
            const float dq = (float)lut[nf4_index(wn, 0, NULL)] * sc;
            const float d = fr[k] - dq;
            const float wd = (im ? im[k] : 1.0f) * d;
            e = e + wd * d;
        }
    } else {
        const float scale = absmax / 7.0f, inv = scale > 0 ? 1.0f / scale : 0.0f;
        for (int k = 0; k < K; k++) {
            int q = (int)lrintf(fr[k] * inv);
            q = q > 7 ? 7 : q < -7 ? -7 : q;
            const float dq = (float)q * scale;
            const float d = fr[k] - dq;
            const float wd = (im ? im[k] : 1.0f) * d;
            e = e + wd * d;
        }
    }
    return e;
}

float orki_wq_best_absmax(const float *fr, int K, float rawabsmax, int nf4, const float *im, float *dq) {
    (void)dq;
    int8_t lut[16];
    orki_nf4_lut(lut);
    float best_abs = rawabsmax, best_e = wq_err(fr, K, rawabsmax, nf4, im, lut);
    for (int g = 1; g < 7; g++) {
        const float cand = rawabsmax * CLIP_GRID[g];
        const float e = wq_err(fr, K, cand, nf4, im, lut);
        if (e < best_e) { best_e = e; best_abs = cand; }
    }
    return best_abs;
}

struct i4q {
    int K, nf4;
    _Atomic int fail;  /* set by a worker that could not allocate its scratch: the whole quant fails */
    const float *f32, *im;
    float *bscale;
    uint8_t *nib;
    int8_t *codes;
    int8_t lut[16];
};

/* One channel, deterministic (sr = 0) or with the caller's shared seed. */
static void i4q_chan(struct i4q *q, int n, int sr, uint32_t *seed, int8_t *tmp, uint8_t *idx) {
    const int K = q->K;
    const float *fr = q->f32 + (size_t)n * K;
    float mx = orki_chan_absmax(fr, K);
    if (q->im) mx = orki_wq_best_absmax(fr, K, mx, q->nf4, q->im, NULL);
    uint8_t *nb = q->nib + (size_t)n * (K / 2);
    if (q->nf4) {
        q->bscale[n] = mx / 127.0f;
        orki_nf4_quant_chan(fr, K, mx, sr, seed, nb, idx);
        if (q->codes)
            for (int k = 0; k < K; k++) q->codes[(size_t)n * K + k] = q->lut[idx[k]];
    } else {
        const float scale = mx / 7.0f;
        q->bscale[n] = scale;
        orki_i4_quant_chan(fr, K, scale, sr, seed, nb, tmp);
        if (q->codes) memcpy(q->codes + (size_t)n * K, tmp, (size_t)K);
    }
}

static void i4q_range(int lo, int hi, void *a) {
    struct i4q *q = a;
    int8_t *tmp = malloc((size_t)q->K);
    uint8_t *idx = malloc((size_t)q->K);
    if (!tmp || !idx) {
        free(tmp);
        free(idx);
        q->fail = 1; /* its channels stay unquantised: the caller must not use the store */
        return;
    }
    for (int n = lo; n < hi; n++) i4q_chan(q, n, 0, NULL, tmp, idx);
    free(tmp);
    free(idx);
}

int orki_i4a8_quant(int K, int N, const float *f32, const float *imatrix, int nf4, int sr,
                    float *bscale, uint8_t *nib, int8_t *codes_nk) {
    struct i4q q = {K, nf4 ? 1 : 0, 0, f32, imatrix, bscale, nib, codes_nk, {0}};
    orki_nf4_lut(q.lut);
    if (!sr) {
        orki_parallel_for(N, i4q_range, &q);
        return q.fail ? -1 : 0;
    }
    /* Stochastic rounding draws one xorshift value per element from a stream that runs across
     * channels in order (src/npu/i4/pack.c:32, :74, :77), so the channels run in sequence. */
    uint32_t seed = 0x2545F491u;
    int8_t *tmp = malloc((size_t)K);
    uint8_t *idx = malloc((size_t)K);
    if (!tmp || !idx) { free(tmp); free(idx); return -1; }
    for (int n = 0; n < N; n++) i4q_chan(&q, n, 1, &seed, tmp, idx);
    free(tmp);
    free(idx);
    return 0;
}
