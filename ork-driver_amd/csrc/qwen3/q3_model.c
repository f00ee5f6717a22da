/* q3_model.c -- host side of the Qwen3-shaped decoder harness (qwen3.h).
 *
 * Follows the reference's end-to-end benchmark (examples/bench.c:80-81 weight construction, :105-113
 * the quantise -> ork_i8_mm_run -> dequantise round trip, :128-145 one decoder layer, :147-188
 * decode / prefill loops) with the MI355X-native differences:
 *   - weights are f32 N(0, std) packed per output channel by ork_i8_mm_pack_f32 (NF4 FFNs through
 *     ork_i4a8_mm_pack), not small integer patterns;
 *   - activations stay in HBM (ork_dev_alloc buffers, async runs); q/k/v and gate/up are one
 *     ork_i8_mm_run_chain each; the non-matmul operators are the fused kernels of q3_ops.hip;
 *   - the activation scale is per row (examples/quant.c:34-37), not the benchmark's dummy constant;
 *   - Qwen3 details the reference benchmark omits: q/k head RMSNorm, tied embedding, final norm,
 *     greedy sampling of the next token (which the benchmark replaces by re-feeding x).
 * One decode step can be captured once as a HIP graph: every kernel reads the position and the input
 * token from device memory, so the graph replays unchanged step after step. */
#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include "q3_ops.h"
#include "qwen3.h"

struct q3_lin {
    ork_w *w;
    float *ws; /* device: per-output-channel scales */
    int K, N;
};

struct q3_layer {
    struct q3_lin l[Q3_NLIN];
    float *n1, *n2, *qn, *kn; /* device norm weights */
    float *kc, *vc;           /* device KV cache [max_ctx][kv_heads * head_dim] */
};

struct q3_model {
    ork_npu *ctx;
    q3_cfg c;
    void *stream;
    struct q3_layer *L;
    struct q3_lin lm;
    float *lm_ws_host;
    q3_half *emb;
    float *nf;
    float *x, *q, *part, *rcos, *rsin;
    float *att, *yffn; /* fused decode: the attention row [heads * head_dim] and silu(g) * u [ffn] */
    int8_t *a8x, *a8att, *a8ffn;
    float *asx, *asatt, *asffn;
    int32_t *cq, *ck, *cv, *co, *cg, *cu, *cd, *clog;
    int *st, *tok_in, *toks;
    unsigned long long *best;
    int S;        /* key chunks per attention row */
    int pos;      /* positions filled */
    int sampled;  /* a next token is waiting in best */
    int last_row; /* row of the last LM-head input in asx */
    int fused;    /* decode with the fused M = 1 kernels where the weights allow (default 1) */
    void *graph;  /* captured decode step */
    float *trace; /* q3_set_trace: [layers + 1][max_rows][hidden] layer-input rows of the last pass */
    int trace_on, trace_rows;
    void **dev;   /* every device buffer of the model */
    int ndev, capdev;
};

#define CK(call)                                                                                          \
    do {                                                                                                  \
        const int rc_ = (call);                                                                           \
        if (rc_) {                                                                                        \
            fprintf(stderr, "[q3] %s failed (%d) at %s:%d\n", #call, rc_, __FILE__, __LINE__);            \
            return rc_ == -2 ? -2 : -1;                                                                   \
        }                                                                                                 \
    } while (0)

static void *dalloc(q3_model *m, size_t bytes) {
    if (m->ndev == m->capdev) {
        const int nc = m->capdev ? 2 * m->capdev : 64;
        void **nd = realloc(m->dev, (size_t)nc * sizeof *nd);
        if (!nd) return NULL;
        m->dev = nd;
        m->capdev = nc;
    }
    void *p = ork_dev_alloc(m->ctx, bytes ? bytes : 16);
    if (p) m->dev[m->ndev++] = p;
    return p;
}

static int upload(q3_model *m, void *dst, const void *src, size_t n) { return ork_dev_upload(m->ctx, dst, src, n); }

/* ---- seeded N(0, std) generator (Box-Muller over splitmix64 counters), threaded ------------------------ */
static uint64_t mix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

struct gen_job {
    float *out;
    size_t lo, hi; /* pair indices */
    size_t n;
    uint64_t base;
    double std, mean;
};

static void *gen_worker(void *arg) {
    const struct gen_job *j = arg;
    for (size_t i = j->lo; i < j->hi; i++) {
        const uint64_t h1 = mix64(j->base + 2 * i), h2 = mix64(j->base + 2 * i + 1);
        const double u1 = ((double)(h1 >> 11) + 1.0) * 0x1.0p-53; /* (0, 1] */
        const double u2 = (double)(h2 >> 11) * 0x1.0p-53;         /* [0, 1) */
        const double r = sqrt(-2.0 * log(u1)), a = 6.283185307179586 * u2;
        j->out[2 * i] = (float)(j->mean + j->std * r * cos(a));
        if (2 * i + 1 < j->n) j->out[2 * i + 1] = (float)(j->mean + j->std * r * sin(a));
    }
    return NULL;
}

static int gen_threads(void) {
    const char *e = getenv("ORK_PACK_THREADS");
    int n = e ? atoi(e) : (int)sysconf(_SC_NPROCESSORS_ONLN);
    if (n < 1) n = 1;
    return n > 16 ? 16 : n;
}

/* stream id: (layer + 2) << 8 | slot; slot < 0x80 linears, 0x80 + which for norms */
static void gen_normal(float *out, size_t n, uint64_t seed, uint64_t id, double mean, double std) {
    const uint64_t base = mix64(seed * 0x100000001B3ull ^ mix64(id));
    const size_t pairs = (n + 1) / 2;
    int nt = gen_threads();
    if ((size_t)nt > pairs / 4096 + 1) nt = (int)(pairs / 4096 + 1);
    pthread_t th[16];
    struct gen_job jobs[16];
    int started = 0;
    for (int t = 0; t < nt; t++) {
        jobs[t] = (struct gen_job){out, pairs * t / nt, pairs * (t + 1) / nt, n, base, std, mean};
        if (t > 0 && pthread_create(&th[t], NULL, gen_worker, &jobs[t]) == 0) started |= 1 << t;
        else if (t > 0) gen_worker(&jobs[t]);
    }
    gen_worker(&jobs[0]);
    for (int t = 1; t < nt; t++)
        if (started & (1 << t)) pthread_join(th[t], NULL);
}

/* ---- shapes ------------------------------------------------------------------------------------------------ */
static int lin_dims(const q3_cfg *c, int layer, int which, int *K, int *N) {
    const int H = c->hidden, QD = c->heads * c->head_dim, KVD = c->kv_heads * c->head_dim;
    if (layer == -1) {
        *K = H;
        *N = c->vocab;
        return 0;
    }
    if (layer < 0 || layer >= c->layers) return -2;
    switch (which) {
    case Q3_WQ: *K = H; *N = QD; return 0;
    case Q3_WK:
    case Q3_WV: *K = H; *N = KVD; return 0;
    case Q3_WO: *K = QD; *N = H; return 0;
    case Q3_WG:
    case Q3_WU: *K = H; *N = c->ffn; return 0;
    case Q3_WD: *K = c->ffn; *N = H; return 0;
    default: return -2;
    }
}

static int cfg_ok(const q3_cfg *c) {
    if (!c || c->layers < 1 || c->hidden < 64 || c->heads < 1 || c->kv_heads < 1 || c->heads % c->kv_heads ||
        c->head_dim < Q3_CHUNK || c->head_dim > Q3_MAX_HD || c->head_dim % 64 || c->ffn < 32 || c->vocab < 32 ||
        c->max_ctx < 1 || c->max_ctx > Q3_MAX_S * Q3_CHUNK || c->max_rows < 1 || c->max_rows > c->max_ctx ||
        c->ffn_nf4 < 0 || c->ffn_nf4 > 2)
        return 0;
    if (Q3_ATT_LDS(256 / c->head_dim, c->head_dim) > 65536) return 0;
    /* the matmul API's dimension rules: K % 32, N % 32 */
    if (c->hidden % 32 || c->ffn % 32 || c->vocab % 32 || (c->kv_heads * c->head_dim) % 32) return 0;
    /* LDS rows of the fused kernels */
    if (c->hidden + 16 > 16384 || c->ffn + 16 > 16384 || c->heads * c->head_dim + 16 > 16384) return 0;
    return 1;
}

int q3_gen_linear(const q3_cfg *c, uint64_t seed, float std, int layer, int which, float *out) {
    int K, N;
    if (!c || !out || lin_dims(c, layer, layer == -1 ? 0 : which, &K, &N)) return -2;
    const uint64_t id = ((uint64_t)(layer + 2) << 8) | (uint64_t)(layer == -1 ? 0 : which);
    gen_normal(out, (size_t)K * N, seed, id, 0.0, std);
    return 0;
}

/* ---- create / free ----------------------------------------------------------------------------------------- */
void q3_free(q3_model *m) {
    if (!m) return;
    if (m->ctx) (void)ork_npu_sync(m->ctx);
    q3g_destroy(m->graph);
    for (int l = 0; m->L && l < m->c.layers; l++)
        for (int i = 0; i < Q3_NLIN; i++)
            if (m->L[l].l[i].w) ork_mm_free(m->ctx, m->L[l].l[i].w);
    if (m->lm.w) ork_mm_free(m->ctx, m->lm.w);
    for (int i = 0; i < m->ndev; i++) ork_dev_free(m->ctx, m->dev[i]);
    if (m->ctx) ork_npu_set_async(m->ctx, 0);
    free(m->dev);
    free(m->L);
    free(m->lm_ws_host);
    free(m);
}

q3_model *q3_create(ork_npu *ctx, const q3_cfg *cfg) {
    if (!ctx || !cfg_ok(cfg) || !ork_npu_stream(ctx)) {
        fprintf(stderr, "[q3] q3_create: bad configuration or no device context\n");
        return NULL;
    }
    q3_model *m = calloc(1, sizeof *m);
    if (!m) return NULL;
    m->ctx = ctx;
    m->c = *cfg;
    m->stream = ork_npu_stream(ctx);
    m->L = calloc((size_t)cfg->layers, sizeof *m->L);
    m->lm_ws_host = calloc((size_t)cfg->vocab, sizeof(float));
    if (!m->L || !m->lm_ws_host) goto fail;
    const q3_cfg *c = cfg;
    const size_t R = (size_t)c->max_rows, H = c->hidden, QD = (size_t)c->heads * c->head_dim,
                 KVD = (size_t)c->kv_heads * c->head_dim, F = c->ffn, HD = c->head_dim;
    m->S = (c->max_ctx + Q3_CHUNK - 1) / Q3_CHUNK;
#define DA(ptr, bytes)                                                                                      \
    do {                                                                                                    \
        if (!((ptr) = dalloc(m, (bytes)))) goto fail;                                                       \
    } while (0)
    for (int l = 0; l < c->layers; l++) {
        struct q3_layer *Ly = &m->L[l];
        DA(Ly->n1, H * 4);
        DA(Ly->n2, H * 4);
        DA(Ly->qn, HD * 4);
        DA(Ly->kn, HD * 4);
        DA(Ly->kc, (size_t)c->max_ctx * KVD * 4);
        DA(Ly->vc, (size_t)c->max_ctx * KVD * 4);
        for (int i = 0; i < Q3_NLIN; i++) {
            int K, N;
            lin_dims(c, l, i, &K, &N);
            Ly->l[i].K = K;
            Ly->l[i].N = N;
            DA(Ly->l[i].ws, (size_t)N * 4);
        }
    }
    m->lm.K = c->hidden;
    m->lm.N = c->vocab;
    DA(m->lm.ws, (size_t)c->vocab * 4);
    DA(m->emb, (size_t)c->vocab * H * 2);
    DA(m->nf, H * 4);
    DA(m->x, R * H * 4);
    DA(m->q, R * QD * 4);
    DA(m->part, R * c->heads * m->S * (HD + 2) * 4);
    DA(m->att, QD * 4);
    DA(m->yffn, F * 4);
    DA(m->rcos, (size_t)c->max_ctx * (HD / 2) * 4);
    DA(m->rsin, (size_t)c->max_ctx * (HD / 2) * 4);
    DA(m->a8x, R * H);
    DA(m->a8att, R * QD);
    DA(m->a8ffn, R * F);
    DA(m->asx, R * 4);
    DA(m->asatt, R * 4);
    DA(m->asffn, R * 4);
    DA(m->cq, R * QD * 4);
    DA(m->ck, R * KVD * 4);
    DA(m->cv, R * KVD * 4);
    DA(m->co, R * H * 4);
    DA(m->cg, R * F * 4);
    DA(m->cu, R * F * 4);
    DA(m->cd, R * H * 4);
    DA(m->clog, (size_t)c->vocab * 4);
    DA(m->st, 16);
    DA(m->tok_in, R * 4);
    DA(m->toks, (size_t)c->max_ctx * 4);
    DA(m->best, 8);
#undef DA
    { /* RoPE tables (examples/bench.c:76): angle = pos * theta^(-2i/HD), in double, rounded once */
        const size_t half = HD / 2, n = (size_t)c->max_ctx * half;
        float *cs = malloc(n * 4), *sn = malloc(n * 4);
        int rc = (cs && sn) ? 0 : -1;
        for (size_t p = 0; !rc && p < (size_t)c->max_ctx; p++)
            for (size_t i = 0; i < half; i++) {
                const double a = (double)p * pow((double)c->rope_theta, -2.0 * (double)i / (double)HD);
                cs[p * half + i] = (float)cos(a);
                sn[p * half + i] = (float)sin(a);
            }
        if (!rc) rc = upload(m, m->rcos, cs, n * 4) || upload(m, m->rsin, sn, n * 4);
        free(cs);
        free(sn);
        if (rc) goto fail;
    }
    {
        const int st0[4] = {0, 0, 0, 0};
        const unsigned long long b0 = 0;
        if (upload(m, m->st, st0, sizeof st0) || upload(m, m->best, &b0, 8)) goto fail;
    }
    m->fused = 1;
    ork_npu_set_async(ctx, 1);
    return m;
fail:
    fprintf(stderr, "[q3] q3_create: device allocation failed\n");
    q3_free(m);
    return NULL;
}

/* ---- weights ----------------------------------------------------------------------------------------------- */
int q3_set_linear(q3_model *m, int layer, int which, const float *w) {
    if (!m || !w) return -2;
    int K, N;
    if (lin_dims(&m->c, layer, layer == -1 ? 0 : which, &K, &N)) return -2;
    struct q3_lin *L = layer == -1 ? &m->lm : &m->L[layer].l[which];
    float *bs = malloc((size_t)N * 4);
    if (!bs) return -1;
    const int w4 = layer >= 0 && m->c.ffn_nf4 && (which == Q3_WG || which == Q3_WU || which == Q3_WD);
    ork_w *pw;
    if (w4) { /* ork_i4a8_mm_pack selects the NF4 codebook when ORK_NF4 is present, uniform int4 otherwise */
        const char *prev = getenv("ORK_NF4");
        char *saved = prev ? strdup(prev) : NULL;
        if (m->c.ffn_nf4 == 2) unsetenv("ORK_NF4");
        else setenv("ORK_NF4", "1", 1);
        pw = ork_i4a8_mm_pack(m->ctx, K, N, w, bs);
        if (saved) {
            setenv("ORK_NF4", saved, 1);
            free(saved);
        } else {
            unsetenv("ORK_NF4");
        }
    } else {
        pw = ork_i8_mm_pack_f32(m->ctx, K, N, w, bs);
    }
    int rc = pw ? upload(m, L->ws, bs, (size_t)N * 4) : -1;
    if (!rc && layer == -1) {
        memcpy(m->lm_ws_host, bs, (size_t)N * 4);
        /* tied embedding: row t of the LM head, in fp16 */
        const size_t n = (size_t)N * K;
        ork_f16 *e = malloc(n * 2);
        if (!e) rc = -1;
        for (size_t i = 0; !rc && i < n; i++) e[i] = (ork_f16)w[i];
        if (!rc) rc = upload(m, m->emb, e, n * 2);
        free(e);
    }
    free(bs);
    if (rc) {
        if (pw) ork_mm_free(m->ctx, pw);
        return -1;
    }
    if (L->w) ork_mm_free(m->ctx, L->w);
    L->w = pw;
    /* a captured decode step holds the old weight's addresses */
    if (m->graph) {
        (void)ork_npu_sync(m->ctx);
        q3g_destroy(m->graph);
        m->graph = NULL;
    }
    return 0;
}

int q3_set_norm(q3_model *m, int layer, int which, const float *w) {
    if (!m || !w || layer < -1 || layer >= m->c.layers) return -2;
    float *dst;
    size_t n = (size_t)m->c.hidden;
    if (layer == -1) {
        if (which != Q3_N_ATTN) return -2;
        dst = m->nf;
    } else {
        struct q3_layer *Ly = &m->L[layer];
        switch (which) {
        case Q3_N_ATTN: dst = Ly->n1; break;
        case Q3_N_FFN: dst = Ly->n2; break;
        case Q3_N_Q: dst = Ly->qn; n = (size_t)m->c.head_dim; break;
        case Q3_N_K: dst = Ly->kn; n = (size_t)m->c.head_dim; break;
        default: return -2;
        }
    }
    return upload(m, dst, w, n * 4) ? -1 : 0;
}

int q3_init_random(q3_model *m, uint64_t seed, float std) {
    if (!m || !(std > 0.f)) return -2;
    const q3_cfg *c = &m->c;
    size_t maxn = (size_t)c->vocab * c->hidden;
    for (int i = 0; i < Q3_NLIN; i++) {
        int K, N;
        lin_dims(c, 0, i, &K, &N);
        if ((size_t)K * N > maxn) maxn = (size_t)K * N;
    }
    float *buf = malloc(maxn * 4);
    if (!buf) return -1;
    int rc = 0;
    for (int l = -1; !rc && l < c->layers; l++) {
        const int nl = l == -1 ? 1 : Q3_NLIN;
        for (int i = 0; !rc && i < nl; i++) {
            rc = q3_gen_linear(c, seed, std, l, i, buf);
            if (!rc) rc = q3_set_linear(m, l, i, buf);
        }
        const int nn = l == -1 ? 1 : 4;
        for (int i = 0; !rc && i < nn; i++) {
            const size_t n = (i == Q3_N_Q || i == Q3_N_K) ? (size_t)c->head_dim : (size_t)c->hidden;
            gen_normal(buf, n, seed, ((uint64_t)(l + 2) << 8) | (uint64_t)(0x80 + i), 1.0, 0.02);
            rc = q3_set_norm(m, l, i, buf);
        }
    }
    free(buf);
    return rc;
}

/* ---- layer-input trace (q3_set_trace) ---------------------------------------------------------------------- */
static int trace_x(q3_model *m, int l, int M) {
    if (!m->trace_on) return 0;
    const size_t H = (size_t)m->c.hidden;
    return q3k_copy_f32(m->trace + (size_t)l * m->c.max_rows * H, m->x, (long long)M * (long long)H, m->stream);
}

int q3_set_trace(q3_model *m, int on) {
    if (!m) return -2;
    if (on && !m->trace) {
        m->trace = dalloc(m, (size_t)(m->c.layers + 1) * m->c.max_rows * m->c.hidden * 4);
        if (!m->trace) return -1;
    }
    if ((on != 0) != m->trace_on) { /* a captured step holds the other form */
        if (ork_npu_sync(m->ctx)) return -1;
        q3g_destroy(m->graph);
        m->graph = NULL;
    }
    m->trace_on = on != 0;
    m->trace_rows = 0;
    return 0;
}

int q3_layer_rows(q3_model *m, int l, float *out, int rows) {
    if (!m || !out || !m->trace || l < 0 || l > m->c.layers || rows < 1 || rows > m->trace_rows) return -2;
    if (ork_npu_sync(m->ctx)) return -1;
    const size_t H = (size_t)m->c.hidden;
    return ork_dev_download(m->ctx, out, m->trace + (size_t)l * m->c.max_rows * H, (size_t)rows * H * 4) ? -1 : 0;
}

/* ---- one pass of the decoder over M rows ------------------------------------------------------------------- */
static int pass(q3_model *m, int M, int decode) {
    const q3_cfg *c = &m->c;
    void *s = m->stream;
    const int H = c->hidden, NH = c->heads, NKV = c->kv_heads, HD = c->head_dim;
    for (int l = 0; l < c->layers; l++) {
        struct q3_layer *Ly = &m->L[l];
        q3_nq nq = {0};
        nq.M = M;
        nq.H = H;
        nq.V = c->vocab;
        nq.x = m->x;
        nq.st = m->st;
        nq.toks = m->toks;
        nq.nw = Ly->n1;
        nq.eps = c->eps;
        nq.a8 = m->a8x;
        nq.as = m->asx;
        if (l == 0) {
            nq.emb = m->emb;
            nq.tok = decode ? NULL : m->tok_in;
            nq.best = m->best;
        } else {
            nq.acc = m->cd;
            nq.acc_as = m->asffn;
            nq.acc_ws = m->L[l - 1].l[Q3_WD].ws;
        }
        CK(q3k_norm_quant(&nq, s));
        CK(trace_x(m, l, M));
        ork_mm_task_i8 qkv[3] = {{Ly->l[Q3_WQ].w, M, m->a8x, m->cq, 0},
                                 {Ly->l[Q3_WK].w, M, m->a8x, m->ck, 0},
                                 {Ly->l[Q3_WV].w, M, m->a8x, m->cv, 0}};
        CK(ork_i8_mm_run_chain(m->ctx, 3, qkv));
        /* A prefill starts at position 0, so its rows see at most M keys: its attention covers the first
         * ceil(M / Q3_CHUNK) chunks only. The chunks past them would hold empty partials (max -inf, sum 0,
         * P.V 0), which add exact zeros to the combine's sums, so the rows are the same bit for bit. */
        const int Sa = decode ? m->S : (M + Q3_CHUNK - 1) / Q3_CHUNK;
        q3_att at = {.M = M, .NH = NH, .NKV = NKV, .HD = HD, .S = Sa, .max_ctx = decode ? c->max_ctx : M,
                     .q = m->q, .kc = Ly->kc, .vc = Ly->vc, .st = m->st, .scale = 1.0f / sqrtf((float)HD),
                     .part = m->part, .rows = m->fused};
        if (M == 1) { /* one row: attention does the q/k/v post-processing itself */
            at.cq = m->cq;
            at.ck = m->ck;
            at.cv = m->cv;
            at.as = m->asx;
            at.wsq = Ly->l[Q3_WQ].ws;
            at.wsk = Ly->l[Q3_WK].ws;
            at.wsv = Ly->l[Q3_WV].ws;
            at.qn = Ly->qn;
            at.kn = Ly->kn;
            at.eps = c->eps;
            at.rcos = m->rcos;
            at.rsin = m->rsin;
        } else {
            const q3_qkv qp = {M, NH, NKV, HD, c->max_ctx, m->cq, m->ck, m->cv, m->asx,
                               Ly->l[Q3_WQ].ws, Ly->l[Q3_WK].ws, Ly->l[Q3_WV].ws, Ly->qn, Ly->kn, c->eps,
                               m->rcos, m->rsin, m->st, m->q, Ly->kc, Ly->vc};
            CK(q3k_qkv_post(&qp, s));
        }
        CK(q3k_attn_part(&at, s));
        const q3_aq aq = {M, NH, HD, Sa, m->part, m->a8att, m->asatt};
        CK(q3k_attn_quant(&aq, s));
        CK(ork_i8_mm_run(m->ctx, Ly->l[Q3_WO].w, M, m->a8att, m->co));
        q3_nq n2 = nq;
        n2.emb = NULL;
        n2.tok = NULL;
        n2.best = NULL;
        n2.acc = m->co;
        n2.acc_as = m->asatt;
        n2.acc_ws = Ly->l[Q3_WO].ws;
        n2.nw = Ly->n2;
        CK(q3k_norm_quant(&n2, s));
        ork_mm_task_i8 gu[2] = {{Ly->l[Q3_WG].w, M, m->a8x, m->cg, 0}, {Ly->l[Q3_WU].w, M, m->a8x, m->cu, 0}};
        CK(ork_i8_mm_run_chain(m->ctx, 2, gu));
        const q3_glu gl = {M, c->ffn, m->cg, m->cu, m->asx, Ly->l[Q3_WG].ws, Ly->l[Q3_WU].ws, m->a8ffn, m->asffn};
        CK(q3k_swiglu_quant(&gl, s));
        CK(ork_i8_mm_run(m->ctx, Ly->l[Q3_WD].w, M, m->a8ffn, m->cd));
    }
    q3_nq fn = {0};
    fn.M = M;
    fn.H = H;
    fn.V = c->vocab;
    fn.x = m->x;
    fn.st = m->st;
    fn.toks = m->toks;
    fn.acc = m->cd;
    fn.acc_as = m->asffn;
    fn.acc_ws = m->L[c->layers - 1].l[Q3_WD].ws;
    fn.nw = m->nf;
    fn.eps = c->eps;
    fn.a8 = m->a8x;
    fn.as = m->asx;
    CK(q3k_norm_quant(&fn, s));
    CK(trace_x(m, c->layers, M));
    CK(ork_i8_mm_run(m->ctx, m->lm.w, 1, m->a8x + (size_t)(M - 1) * H, m->clog));
    const q3_amax am = {c->vocab, m->clog, m->asx + (M - 1), m->lm.ws, m->best};
    CK(q3k_argmax(&am, s));
    m->last_row = M - 1;
    m->trace_rows = m->trace_on ? M : 0;
    return 0;
}

/* ---- the fused decode step (M = 1) --------------------------------------------------------------------------- *
 * Per layer: q/k/v as one ork_i8_mm_run_row (the library's one-row run: RMSNorm + int8 row in its prologue, the
 * three int32 results stored; layer 0: the embedding kernel and the q/k/v chain, as in pass()); attention partials;
 * the chunk combine into an fp32 row; o (the row's quant in the prologue, the residual add in the epilogue);
 * gate/up (the FFN RMSNorm prologue, the silu(g) * u epilogue); down (quant prologue, residual add). 6 launches per
 * layer instead of 9, with the same float operations in the same order (orkh_rowops.h), so logits and tokens equal
 * those of pass(). */
static int fused_ok(const q3_model *m) {
    const q3_cfg *c = &m->c;
    if (!m->fused) return 0;
    /* the row bound of the fused run; q/k/v / o are int8, the FFN weights int8, uniform int4 or NF4 */
    return c->hidden <= ORK_ROW_KMAX && c->ffn <= ORK_ROW_KMAX && c->heads * c->head_dim <= ORK_ROW_KMAX;
}

static int pass_fused(q3_model *m) {
    const q3_cfg *c = &m->c;
    void *s = m->stream;
    const int H = c->hidden, NH = c->heads, NKV = c->kv_heads, HD = c->head_dim;
    for (int l = 0; l < c->layers; l++) {
        struct q3_layer *Ly = &m->L[l];
        const struct q3_lin *Lq = &Ly->l[Q3_WQ], *Lk = &Ly->l[Q3_WK], *Lv = &Ly->l[Q3_WV], *Lo = &Ly->l[Q3_WO],
                            *Lg = &Ly->l[Q3_WG], *Lu = &Ly->l[Q3_WU], *Ld = &Ly->l[Q3_WD];
        if (l == 0) {
            q3_nq nq = {0};
            nq.M = 1;
            nq.H = H;
            nq.V = c->vocab;
            nq.x = m->x;
            nq.st = m->st;
            nq.toks = m->toks;
            nq.nw = Ly->n1;
            nq.eps = c->eps;
            nq.a8 = m->a8x;
            nq.as = m->asx;
            nq.emb = m->emb;
            nq.best = m->best;
            CK(q3k_norm_quant(&nq, s));
            CK(trace_x(m, 0, 1));
            ork_mm_task_i8 qkv[3] = {{Lq->w, 1, m->a8x, m->cq, 0}, {Lk->w, 1, m->a8x, m->ck, 0},
                                     {Lv->w, 1, m->a8x, m->cv, 0}};
            CK(ork_i8_mm_run_chain(m->ctx, 3, qkv));
        } else {
            CK(trace_x(m, l, 1)); /* the previous layer's down epilogue completed the residual row */
            ork_w *const wq[3] = {Lq->w, Lk->w, Lv->w};
            ork_row_op f = {0};
            f.prologue = ORK_ROW_RMSNORM;
            f.row = m->x;
            f.norm_w = Ly->n1;
            f.eps = c->eps;
            f.row_scale = m->asx;
            f.epilogue = ORK_COL_STORE;
            f.C[0] = m->cq;
            f.C[1] = m->ck;
            f.C[2] = m->cv;
            CK(ork_i8_mm_run_row(m->ctx, 3, wq, &f));
        }
        q3_att at = {.M = 1, .NH = NH, .NKV = NKV, .HD = HD, .S = m->S, .max_ctx = c->max_ctx, .q = m->q,
                     .kc = Ly->kc, .vc = Ly->vc, .st = m->st, .scale = 1.0f / sqrtf((float)HD), .part = m->part,
                     .cq = m->cq, .ck = m->ck, .cv = m->cv, .as = m->asx, .wsq = Lq->ws, .wsk = Lk->ws,
                     .wsv = Lv->ws, .qn = Ly->qn, .kn = Ly->kn, .eps = c->eps, .rcos = m->rcos, .rsin = m->rsin};
        CK(q3k_attn_part(&at, s));
        const q3_comb cb = {NH, HD, m->S, m->part, m->att};
        CK(q3k_attn_combine(&cb, s));
        ork_row_op fo = {0};
        fo.prologue = ORK_ROW_QUANT;
        fo.row = m->att;
        fo.epilogue = ORK_COL_RESID;
        fo.w_scale[0] = Lo->ws;
        fo.out = m->x;
        CK(ork_i8_mm_run_row(m->ctx, 1, &Lo->w, &fo));
        ork_w *const wgu[2] = {Lg->w, Lu->w};
        ork_row_op fg = {0};
        fg.prologue = ORK_ROW_RMSNORM;
        fg.row = m->x;
        fg.norm_w = Ly->n2;
        fg.eps = c->eps;
        fg.epilogue = ORK_COL_SWIGLU;
        fg.w_scale[0] = Lg->ws;
        fg.w_scale[1] = Lu->ws;
        fg.out = m->yffn;
        CK(ork_i8_mm_run_row(m->ctx, 2, wgu, &fg));
        ork_row_op fd = {0};
        fd.prologue = ORK_ROW_QUANT;
        fd.row = m->yffn;
        fd.epilogue = ORK_COL_RESID;
        fd.w_scale[0] = Ld->ws;
        fd.out = m->x;
        CK(ork_i8_mm_run_row(m->ctx, 1, &Ld->w, &fd));
    }
    CK(trace_x(m, c->layers, 1));
    q3_nq fn = {0}; /* the residual add is done: plain final norm */
    fn.M = 1;
    fn.H = H;
    fn.V = c->vocab;
    fn.x = m->x;
    fn.st = m->st;
    fn.toks = m->toks;
    fn.nw = m->nf;
    fn.eps = c->eps;
    fn.a8 = m->a8x;
    fn.as = m->asx;
    CK(q3k_norm_quant(&fn, s));
    CK(ork_i8_mm_run(m->ctx, m->lm.w, 1, m->a8x, m->clog));
    const q3_amax am = {c->vocab, m->clog, m->asx, m->lm.ws, m->best};
    CK(q3k_argmax(&am, s));
    m->last_row = 0;
    m->trace_rows = m->trace_on ? 1 : 0;
    return 0;
}

static int decode_pass(q3_model *m) { return fused_ok(m) ? pass_fused(m) : pass(m, 1, 1); }

int q3_set_fused(q3_model *m, int on) {
    if (!m) return -2;
    if ((on != 0) != m->fused) {
        if (ork_npu_sync(m->ctx)) return -1;
        q3g_destroy(m->graph);
        m->graph = NULL;
    }
    m->fused = on != 0;
    return 0;
}

int q3_decode_fused(const q3_model *m) { return m ? fused_ok(m) : 0; }

static int weights_ready(const q3_model *m) {
    if (!m->lm.w) return 0;
    for (int l = 0; l < m->c.layers; l++)
        for (int i = 0; i < Q3_NLIN; i++)
            if (!m->L[l].l[i].w) return 0;
    return 1;
}

int q3_prefill(q3_model *m, const int *tokens, int n) {
    if (!m || !tokens || n < 1 || n > m->c.max_rows || n > m->c.max_ctx) return -2;
    if (!weights_ready(m)) {
        fprintf(stderr, "[q3] q3_prefill: weights are not all set\n");
        return -2;
    }
    for (int i = 0; i < n; i++)
        if (tokens[i] < 0 || tokens[i] >= m->c.vocab) return -2;
    const int st0[4] = {0, n, 0, 0};
    if (upload(m, m->tok_in, tokens, (size_t)n * 4) || upload(m, m->st, st0, sizeof st0)) return -1;
    CK(pass(m, n, 0));
    if (ork_npu_sync(m->ctx)) return -1;
    m->pos = n;
    m->sampled = 1;
    return 0;
}

int q3_decode(q3_model *m, int steps, int graph) {
    if (!m || steps < 0) return -2;
    if (!m->sampled) {
        fprintf(stderr, "[q3] q3_decode: no sampled token (run q3_prefill first)\n");
        return -2;
    }
    if (m->pos + steps > m->c.max_ctx) {
        fprintf(stderr, "[q3] q3_decode: %d + %d positions exceed max_ctx %d\n", m->pos, steps, m->c.max_ctx);
        return -2;
    }
    for (int i = 0; i < steps; i++) {
        if (graph && !m->graph) {
            if (q3g_begin(m->stream)) return -1;
            const int rc = decode_pass(m);
            void *g = NULL;
            const int rc2 = q3g_end(m->stream, &g);
            if (rc || rc2) {
                q3g_destroy(g);
                fprintf(stderr, "[q3] q3_decode: graph capture failed (%d, %d)\n", rc, rc2);
                return -1;
            }
            m->graph = g;
        }
        if (graph) {
            if (q3g_launch(m->graph, m->stream)) return -1;
        } else {
            CK(decode_pass(m));
        }
        m->pos++;
    }
    return ork_npu_sync(m->ctx) ? -1 : 0;
}

int q3_positions(const q3_model *m) { return m ? m->pos : 0; }

int q3_tokens(q3_model *m, int *out, int n) {
    if (!m || !out || n < 0) return -2;
    if (ork_npu_sync(m->ctx)) return -1;
    const int have = n < m->pos ? n : m->pos;
    if (have > 0 && ork_dev_download(m->ctx, out, m->toks, (size_t)have * 4)) return -1;
    if (n > m->pos && m->sampled) {
        unsigned long long b = 0;
        if (ork_dev_download(m->ctx, &b, m->best, 8)) return -1;
        out[m->pos] = (int)(0xFFFFFFFFu - (unsigned)(b & 0xFFFFFFFFull));
    }
    return 0;
}

int q3_last_logits(q3_model *m, float *out) {
    if (!m || !out || !m->sampled) return -2;
    if (ork_npu_sync(m->ctx)) return -1;
    const int V = m->c.vocab;
    int32_t *c = malloc((size_t)V * 4);
    float as = 0.f;
    int rc = c ? 0 : -1;
    if (!rc) rc = ork_dev_download(m->ctx, c, m->clog, (size_t)V * 4);
    if (!rc) rc = ork_dev_download(m->ctx, &as, m->asx + m->last_row, 4);
    for (int n = 0; !rc && n < V; n++) out[n] = ((float)c[n] * as) * m->lm_ws_host[n];
    free(c);
    return rc ? -1 : 0;
}

double q3_weight_bytes(const q3_model *m) {
    if (!m) return 0;
    double b = 0;
    for (int l = 0; l < m->c.layers; l++)
        for (int i = 0; i < Q3_NLIN; i++)
            if (m->L[l].l[i].w) b += (double)ork_w_bytes(m->L[l].l[i].w) + 4.0 * m->L[l].l[i].N;
    if (m->lm.w) b += (double)ork_w_bytes(m->lm.w) + 4.0 * m->lm.N;
    return b;
}
