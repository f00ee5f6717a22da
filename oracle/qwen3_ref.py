"""CPU restatement (numpy, float32) of the Qwen3-shaped decoder that libork_qwen3.so runs on the GPU.

TEST INFRASTRUCTURE ONLY: imported by tests/ and bench.py's checker, never by the product.

It follows the reference's model examples operator by operator:
  rmsnorm        examples/bench.c:75, examples/layer.c:21-24 (o = x * (1/sqrt(mean(x^2) + eps)) * w)
  rope           examples/bench.c:76, examples/layer.c:25-28 (NeoX rotate-halves, theta^(-2i/HD))
  attention      examples/layer.c:50-56 (GQA: query head h reads kv head h // (NH/NKV); causal softmax of
                 q.k * 1/sqrt(HD), then the weighted sum of v)
  swiglu         examples/bench.c:77, :140 (silu(g) * u, silu(x) = x / (1 + exp(-x)))
  layer          examples/bench.c:128-145 (norm -> q,k,v -> rope -> cache -> attention -> o -> residual ->
                 norm -> gate,up -> swiglu -> down -> residual)
  w8a8 matmul    examples/quant.c:5-6, :30-37 (per-output-channel weight codes from ork_i8_mm_pack_f32's
                 rule, per-row activation quantisation), int32 products exact (oracle.gemm_i32)
plus what a Qwen3 checkpoint adds and the reference benchmark leaves out: per-head q/k RMSNorm before
RoPE, an embedding table tied to the LM head (its fp16 rows), a final norm and greedy sampling.

The GPU kernels compute the same formulas in float32 with different summation orders (tree reductions,
chunked online softmax), so results agree to a tolerance, not bit for bit; the integer matmuls inside
are exact on both sides. Pins (tests/test_qwen3_ref.py): closed forms of each operator (RMSNorm of a
constant row, RoPE at position 0 and its norm and relative-position invariance, attention with one
key / equal scores, silu(0), argmax ties) and a brute-force float64 evaluation of one small layer.
"""
import numpy as np

import oracle as O

F32 = np.float32


def rmsnorm(x, w, eps):
    x = np.asarray(x, F32)
    ss = np.sum(x * x, axis=-1, dtype=F32, keepdims=True)
    r = F32(1.0) / np.sqrt(ss / F32(x.shape[-1]) + F32(eps))
    return (x * r) * np.asarray(w, F32)


def rope_tables(max_ctx, head_dim, theta):
    """cos, sin [max_ctx][head_dim/2] of angle pos * theta^(-2i/HD), evaluated in double, rounded once."""
    half = head_dim // 2
    i = np.arange(half, dtype=np.float64)
    fr = np.power(np.float64(theta), -2.0 * i / head_dim)
    ang = np.arange(max_ctx, dtype=np.float64)[:, None] * fr[None, :]
    return np.cos(ang).astype(F32), np.sin(ang).astype(F32)


def rope(v, cos, sin):
    """v [..., HD] rotated with one position's cos/sin [HD/2] (rotate halves)."""
    half = v.shape[-1] // 2
    a, b = v[..., :half], v[..., half:]
    return np.concatenate([a * cos - b * sin, a * sin + b * cos], axis=-1).astype(F32)


def silu_mul(g, u):
    g = np.asarray(g, F32)
    return (g / (F32(1.0) + np.exp(-g))) * np.asarray(u, F32)


def attend(q, K, V, scale):
    """One query row q [HD] over keys K [L][HD] / values V [L][HD]: softmax(q.K * scale) . V."""
    s = (K @ q).astype(F32) * F32(scale)
    p = np.exp(s - s.max())
    return ((p / p.sum(dtype=F32)) @ V).astype(F32)


def quant_rows(x):
    """Per-row int8 (examples/quant.c:34-37): (row scales [M], codes [M][K])."""
    a_s, q = O.quant_test_acts(np.ascontiguousarray(x, F32))
    return a_s, q


def dequant(c, a_s, ws):
    return (c.astype(F32) * np.asarray(a_s, F32)[:, None]) * np.asarray(ws, F32)[None, :]


class Linear:
    """A packed linear as the library stores it: codes [K][N] and per-channel scales [N]."""

    def __init__(self, w_nk, nf4=False):
        """nf4: False (int8, ork_i8_mm_pack_f32), True or 1 (NF4 w4a8) or 2 (uniform int4 w4a8), as the harness's
        ffn_nf4 (both w4a8 kinds through ork_i4a8_mm_pack, src/npu/i4/pack.c)."""
        if nf4:
            bs, _, codes = O.pack_i4a8(w_nk, nf4=(nf4 != 2))
        else:
            codes, bs = O.pack_i8_f32(w_nk)
        self.codes, self.ws = codes, bs

    def __call__(self, x):
        a_s, q = quant_rows(x)
        return dequant(O.gemm_i32(q, self.codes), a_s, self.ws)


class Qwen3Ref:
    """weights: {(layer, which): f32[N][K]} for which in 0..6 (q k v o gate up down) and (-1, 0) for the
    LM head; norms: {(layer, which): f32[...]} for which in 0..3 (attn, ffn, q, k) and (-1, 0) final."""

    def __init__(self, cfg, weights, norms, ffn_nf4=False):
        self.c = cfg
        self.lin = {k: Linear(w, nf4=ffn_nf4 if (k[0] >= 0 and k[1] in (4, 5, 6)) else False) for k, w in weights.items()}
        self.emb = weights[(-1, 0)].astype(np.float16).astype(F32)
        self.norms = {k: np.asarray(v, F32) for k, v in norms.items()}
        self.cos, self.sin = rope_tables(cfg.max_ctx, cfg.head_dim, cfg.rope_theta)
        kvd = cfg.kv_heads * cfg.head_dim
        self.kc = np.zeros((cfg.layers, cfg.max_ctx, kvd), F32)
        self.vc = np.zeros((cfg.layers, cfg.max_ctx, kvd), F32)

    def forward(self, tokens, pos0):
        """Rows `tokens` at positions pos0.. (the cache holds 0..pos0-1); returns the last row's logits."""
        x = self.emb[np.asarray(tokens)]
        for l in range(self.c.layers):
            x = self.layer(l, x, pos0)
        return self.head(x)

    def layer(self, l, x, pos0):
        """Decoder layer l (examples/bench.c:128-145) on the residual rows x [M][H] at positions pos0..: appends
        their keys and values to layer l's cache (which holds positions 0..pos0-1) and returns the rows leaving the
        layer. Fed another engine's rows, it checks one layer on that engine's input (teacher forcing)."""
        c = self.c
        NH, NKV, HD, eps = c.heads, c.kv_heads, c.head_dim, c.eps
        G = NH // NKV
        scale = F32(1.0) / np.sqrt(F32(HD))
        x = np.asarray(x, F32)
        M = x.shape[0]
        h = rmsnorm(x, self.norms[(l, 0)], eps)
        q, k, v = self.lin[(l, 0)](h), self.lin[(l, 1)](h), self.lin[(l, 2)](h)
        att = np.zeros_like(q)
        for t in range(M):
            pos = pos0 + t
            cs, sn = self.cos[pos], self.sin[pos]
            kh = rope(rmsnorm(k[t].reshape(NKV, HD), self.norms[(l, 3)], eps), cs, sn)
            self.kc[l, pos] = kh.reshape(-1)
            self.vc[l, pos] = v[t]
        for t in range(M):
            L = pos0 + t + 1
            cs, sn = self.cos[pos0 + t], self.sin[pos0 + t]
            qh = rope(rmsnorm(q[t].reshape(NH, HD), self.norms[(l, 2)], eps), cs, sn)
            for hh in range(NH):
                g = hh // G
                K = self.kc[l, :L, g * HD:(g + 1) * HD]
                V = self.vc[l, :L, g * HD:(g + 1) * HD]
                att[t, hh * HD:(hh + 1) * HD] = attend(qh[hh], K, V, scale)
        x = x + self.lin[(l, 3)](att)
        h2 = rmsnorm(x, self.norms[(l, 1)], eps)
        a = silu_mul(self.lin[(l, 4)](h2), self.lin[(l, 5)](h2))
        return x + self.lin[(l, 6)](a)

    def head(self, x):
        """Final norm and LM head of the last row of x [M][H]: its logits."""
        hf = rmsnorm(np.asarray(x, F32), self.norms[(-1, 0)], self.c.eps)
        return self.lin[(-1, 0)](hf[-1:])[0]


def greedy(logits):
    """First maximum, as the GPU's (value, ~index) key order resolves ties."""
    return int(np.argmax(logits))
