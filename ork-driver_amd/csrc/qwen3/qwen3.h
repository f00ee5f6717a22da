/* qwen3.h -- a Qwen3-shaped decoder harness over the resident-weight matmul API (libork_qwen3.so).
 *
 * The MI355X counterpart of the reference's end-to-end benchmark and model examples
 * (examples/bench.c:19-28 shapes, :105-190 layer / decode / prefill; examples/layer.c, decode.c,
 * model.c): every projection and the LM head go through the public ork_* matmul API (int8 w8a8 weights
 * from ork_i8_mm_pack_f32, optionally NF4 w4a8 FFN weights from ork_i4a8_mm_pack), q/k/v and gate/up
 * as multi-matmul chains; the non-matmul operators are fused HIP kernels on the context's stream.
 * Activations are quantised per row to int8 before each matmul (examples/quant.c:34-37), as a real
 * w8a8 engine does (the reference benchmark uses a dummy per-tensor scale, examples/bench.c:100-104).
 * Architecture: RMSNorm, GQA attention with Qwen3's per-head q/k RMSNorm, NeoX RoPE, SwiGLU FFN, final
 * norm, LM head whose rows double as the (tied) embedding table, greedy sampling.
 *
 * All functions return 0 on success, -2 on bad arguments, -1 on a device or library error. */
#ifndef ORK_QWEN3_H
#define ORK_QWEN3_H
#include <stdint.h>

#include "ork_npu.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct q3_cfg {
    int layers, hidden, heads, kv_heads, head_dim, ffn, vocab;
    int max_ctx;       /* KV-cache positions (prefill + decode) */
    int max_rows;      /* largest prefill batch */
    int ffn_nf4;       /* 1: gate/up/down packed as NF4 w4a8 (ork_i4a8_mm_pack with ORK_NF4); 2: uniform int4 w4a8 */
    float rope_theta;  /* Qwen3: 1e6 */
    float eps;         /* Qwen3: 1e-6 */
} q3_cfg;

typedef struct q3_model q3_model;

/* Linear weights, f32[N][K] (out x in), as ork_i8_mm_pack_f32 takes them. */
enum { Q3_WQ = 0, Q3_WK, Q3_WV, Q3_WO, Q3_WG, Q3_WU, Q3_WD, Q3_NLIN };
/* Norm weights: per layer attention / FFN input norms (hidden), q / k head norms (head_dim); the final
 * norm is layer -1, Q3_N_ATTN. */
enum { Q3_N_ATTN = 0, Q3_N_FFN, Q3_N_Q, Q3_N_K };

q3_model *q3_create(ork_npu *ctx, const q3_cfg *cfg);
void      q3_free(q3_model *m);
/* layer -1: the LM head / tied embedding, f32[vocab][hidden]. */
int       q3_set_linear(q3_model *m, int layer, int which, const float *w_nk);
int       q3_set_norm(q3_model *m, int layer, int which, const float *w);
/* Every weight from a seeded N(0, std) generator (norm weights 1 + N(0, 0.02)), on host threads. */
int       q3_init_random(q3_model *m, uint64_t seed, float std);
/* The same generator's values for one linear (tests): (layer, which) as in q3_set_linear. */
int       q3_gen_linear(const q3_cfg *cfg, uint64_t seed, float std, int layer, int which, float *out_nk);

/* Prefill n tokens at positions 0..n-1 (clears the cache), then greedy-sample the next token. */
int       q3_prefill(q3_model *m, const int *tokens, int n);
/* Greedy decode: feed the last sampled token, sample the next; `steps` times. graph = 1 replays one
 * captured HIP graph per step. Returns after the last step has finished. */
int       q3_decode(q3_model *m, int steps, int graph);
/* Decode through the fused M = 1 kernels and prefill attention by blocks of rows (on = 1, the default), or the
 * unfused operator sequence and row-by-row prefill attention (0); both give identical logits and tokens. The fused form needs every weight resident on the device with K-blocks that fit
 * its LDS row (8 KiB); q3_decode_fused says whether the current weights take it. */
int       q3_set_fused(q3_model *m, int on);
int       q3_decode_fused(const q3_model *m);
/* Tokens at positions 0..n-1 and the one sampled last (out[n] when n == the position count). */
int       q3_tokens(q3_model *m, int *out, int n);
/* Number of positions filled (prefill + decode inputs). */
int       q3_positions(const q3_model *m);
/* Dequantised logits of the last sampled row, f32[vocab]. */
int       q3_last_logits(q3_model *m, float *out);
/* Test aid: the residual rows entering each layer. With on = 1, every later prefill and decode step also copies x,
 * the fp32 rows entering layer l (l = 0 .. layers - 1) and leaving the last layer (l = layers, before the final
 * norm), into a device trace (kernels of the step, so captured decode graphs hold them too). q3_layer_rows reads
 * `rows` rows of layer l from the last pass (a prefill's n rows, a decode step's one) into out f32[rows][hidden]. */
int       q3_set_trace(q3_model *m, int on);
int       q3_layer_rows(q3_model *m, int l, float *out, int rows);
/* Resident weight bytes read per decode token (projections + LM head, scales included). */
double    q3_weight_bytes(const q3_model *m);

#ifdef __cplusplus
}
#endif
#endif
