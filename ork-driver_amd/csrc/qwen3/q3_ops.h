/* q3_ops.h -- C-ABI of the decoder harness's fused non-matmul kernels (q3_ops.hip).
 *
 * Plain structs of device pointers and sizes, one per kernel; each launcher enqueues on the given
 * hipStream_t and returns 0, -2 for arguments the kernel's grid cannot cover, -1 on a HIP error.
 * Activations: fp32 rows; matmul results: int32 rows with the row scale of their int8 A and the
 * per-output-channel scale of their weight, dequantised as (c * a_scale) * w_scale. */
#ifndef Q3_OPS_H
#define Q3_OPS_H
#include <stdint.h>

#ifdef __cplusplus
#include <hip/hip_fp16.h>
typedef __half q3_half;
extern "C" {
#else
typedef uint16_t q3_half;
#endif

#define Q3_CHUNK 32   /* keys per attention workgroup (32 or 64) */
#define Q3_MAX_HD 256 /* head_dim bound of k_qkv_post / k_attn_part */
#define Q3_MAX_S 32   /* key chunks per row: max_ctx <= 1024 */

/* st[] decode state: st[0] position of row 0 of the current pass, st[1] next free position.
 * best: greedy-sampling key, (order-preserving bits of the logit << 32) | (0xFFFFFFFF - token). */

typedef struct q3_nq { /* [embed | x += acc] -> RMSNorm -> int8 rows */
    int M, H, V;
    float *x;                 /* [M][H] residual stream, updated in place */
    const int32_t *acc;       /* nullable: [M][H] projection result added to x */
    const float *acc_as;      /* [M] row scales of that projection's A */
    const float *acc_ws;      /* [H] its column scales */
    const q3_half *emb;       /* nullable: [V][H] embedding rows; x = emb[token] */
    const int *tok;           /* prefill: [M] tokens; NULL in decode (token = best) */
    unsigned long long *best; /* decode: read then cleared; prefill: cleared when non-NULL */
    int *st;                  /* decode state (see above) */
    int *toks;                /* [max_ctx] token log, written at each row's position */
    const float *nw;          /* [H] RMSNorm weight */
    float eps;
    int8_t *a8;               /* [M][H] out */
    float *as;                /* [M] out: row scales */
} q3_nq;

typedef struct q3_qkv { /* q/k/v dequant -> per-head RMSNorm -> RoPE -> q rows, KV-cache append */
    int M, NH, NKV, HD, max_ctx;
    const int32_t *cq, *ck, *cv; /* [M][NH*HD], [M][NKV*HD], [M][NKV*HD] */
    const float *as;             /* [M] */
    const float *wsq, *wsk, *wsv;
    const float *qn, *kn; /* [HD] */
    float eps;
    const float *rcos, *rsin; /* [max_ctx][HD/2] */
    const int *st;
    float *q;       /* [M][NH*HD] out */
    float *kc, *vc; /* [max_ctx][NKV*HD] this layer's cache */
} q3_qkv;

typedef struct q3_att { /* grid (NKV * query-head sub-groups, S, M): Q3_CHUNK-key chunk partials */
    int M, NH, NKV, HD, S, max_ctx;
    const float *q; /* [M][NH*HD] rotated queries (unfused) */
    float *kc, *vc; /* this layer's cache; the fused form appends the new row */
    const int *st;
    float scale;
    float *part; /* [M][NH][S][HD + 2]: P.V, then max and sum */
    int rows;    /* unfused form: 1 = one workgroup per block of rows (k_attn_rows), 0 = per row; same partials */
    /* fused form (M = 1, cq != NULL): the q/k/v matmul results and what k_qkv_post takes */
    const int32_t *cq, *ck, *cv;
    const float *as, *wsq, *wsk, *wsv, *qn, *kn;
    float eps;
    const float *rcos, *rsin;
} q3_att;

typedef struct q3_aq { /* chunk combine -> int8 rows */
    int M, NH, HD, S;
    const float *part;
    int8_t *a8; /* [M][NH*HD] */
    float *as;
} q3_aq;

typedef struct q3_glu { /* silu(gate) * up -> int8 rows */
    int M, F;
    const int32_t *cg, *cu; /* [M][F] */
    const float *as_in;     /* [M] */
    const float *wsg, *wsu; /* [F] */
    int8_t *a8;
    float *as_out;
} q3_glu;

typedef struct q3_amax { /* greedy sampling over one row of logits */
    int V;
    const int32_t *c; /* [V] */
    const float *as;  /* the row's scale (one float) */
    const float *ws;  /* [V] */
    unsigned long long *best;
} q3_amax;

typedef struct q3_comb { /* grid NH: one head's chunks combined into an fp32 row */
    int NH, HD, S;
    const float *part; /* [NH][S][HD + 2] */
    float *out;        /* [NH * HD] */
} q3_comb;

int q3k_attn_combine(const q3_comb *p, void *stream);

/* LDS bytes of k_attn_part for a workgroup of G query heads (launches above 64 KiB are refused). */
#define Q3_ATT_LDS(G, HD) ((size_t)(Q3_CHUNK * ((HD) + 4) + 2 * (G) * (HD) + (G) * Q3_CHUNK + 2 * (G) + 2 * (HD)) * 4)

int q3k_norm_quant(const q3_nq *p, void *stream);
int q3k_copy_f32(float *dst, const float *src, long long n, void *stream); /* n floats, device to device */
int q3k_qkv_post(const q3_qkv *p, void *stream);
int q3k_attn_part(const q3_att *p, void *stream);
int q3k_attn_quant(const q3_aq *p, void *stream);
int q3k_swiglu_quant(const q3_glu *p, void *stream);
int q3k_argmax(const q3_amax *p, void *stream);

int q3g_begin(void *stream);
int q3g_end(void *stream, void **exec);
int q3g_launch(void *exec, void *stream);
void q3g_destroy(void *exec);
int q3g_sync(void *stream);
int q3t_begin(void *stream, void **ev);
double q3t_end(void *stream, void **ev);

#ifdef __cplusplus
}
#endif
#endif
