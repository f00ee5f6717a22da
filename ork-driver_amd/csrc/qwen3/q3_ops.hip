// q3_ops.hip -- the non-matmul operators of the Qwen3-shaped decoder harness, for gfx950.
//
// The reference runs these on the host CPU between NPU matmuls (examples/bench.c:74-78 rmsnorm / rope /
// silu, :83-90 the int8 activation round trip, :115-127 flash-style GQA attention; examples/layer.c:21-30,
// examples/decode.c:21-26; the per-row activation quantisation of examples/quant.c:34-37). Here they are
// small fused kernels on the library's stream, so activations never leave HBM between the matmuls:
//   k_norm_quant_*    [embedding lookup | residual add of a matmul result] + RMSNorm + per-row int8 quant
//   k_qkv_post        q/k/v dequant + per-head RMSNorm (Qwen3 q_norm / k_norm) + RoPE + KV-cache append
//   k_attn_part       causal GQA attention over one Q3_CHUNK-key chunk: running max, sum and P.V per query head
//   k_attn_quant      combine the chunks (log-sum-exp) + per-row int8 quant of the attention output
//   k_swiglu_quant    gate/up dequant + silu(g) * u + per-row int8 quant
//   k_argmax          greedy sampling: dequantised logits -> one 64-bit atomic max per workgroup
// Decode reads its position and its input token from device memory (st[], best), so one captured HIP
// graph per decode step replays unchanged. Compiled with -ffp-contract=off: every product and sum is
// rounded as the reference's C code rounds it (no fused multiply-add).
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <math.h>
#include <stdint.h>

#include "q3_ops.h"
#include "orkh_rowops.h"

namespace {
using namespace orkr;


// Token of a greedy-sampling key (see k_argmax): low 32 bits hold ~index.
__device__ inline int key_token(unsigned long long k) { return (int)(0xFFFFFFFFu - (unsigned)(k & 0xFFFFFFFFull)); }

// The row source of k_norm_quant, fixed per launch so that every load of the row is issued up front.
enum { NQ_ACC = 0, NQ_EMB = 1, NQ_X = 2 };

template <int E, int MODE>
__device__ inline void norm_quant_body(const q3_nq &p) {
    __shared__ __align__(16) float red[16];
    const int t = blockIdx.x, H = p.H;
    float *__restrict__ xr = p.x + (size_t)t * H;
    float v[E], nw[E];
    int tok = 0;
    if constexpr (MODE == NQ_EMB) {
        tok = p.tok ? p.tok[t] : key_token(*p.best);
        if (tok < 0 || tok >= p.V) tok = 0; // an unset key; the host validates tokens it uploads
        const __half *__restrict__ e = p.emb + (size_t)tok * H;
        load_row(nw, p.nw, H);
#pragma unroll
        for (int k = 0; k < E; k++) {
            const int i = threadIdx.x + k * blockDim.x;
            const float x = __half2float(e[min(i, H - 1)]);
            v[k] = i < H ? x : 0.f;
        }
    } else {
        load_row(v, (const float *)xr, H);
        if constexpr (MODE == NQ_ACC) { // residual add of the previous projection: x += (c * a_scale) * w_scale
            int32_t c[E];
            float w[E];
            load_row(c, p.acc + (size_t)t * H, H);
            load_row(w, p.acc_ws, H);
            const float as = p.acc_as[t];
            load_row(nw, p.nw, H);
#pragma unroll
            for (int k = 0; k < E; k++) v[k] = v[k] + ((float)c[k] * as) * w[k];
        } else {
            load_row(nw, p.nw, H);
        }
    }
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < E; k++) {
        const int i = threadIdx.x + k * blockDim.x;
        if (i < H) xr[i] = v[k];
        ss += v[k] * v[k];
    }
    ss = block_sum(ss, red); // its barrier also orders every read of *best before the clear below
    if (MODE == NQ_EMB && threadIdx.x == 0) {
        if (p.tok) {
            p.toks[p.st[0] + t] = tok;
            if (t == 0 && p.best) *p.best = 0ull;
        } else { // decode: this row is the next position
            const int pos = p.st[1];
            p.toks[pos] = tok;
            p.st[0] = pos;
            p.st[1] = pos + 1;
            *p.best = 0ull;
        }
    }
    const float r = 1.0f / sqrtf(ss / (float)H + p.eps);
#pragma unroll
    for (int k = 0; k < E; k++) v[k] = (v[k] * r) * nw[k];
    quant_regs(v, H, p.a8 + (size_t)t * H, p.as + t);
}
template <int E> __global__ __launch_bounds__(512) void k_norm_quant_acc(q3_nq p) { norm_quant_body<E, NQ_ACC>(p); }
template <int E> __global__ __launch_bounds__(512) void k_norm_quant_emb(q3_nq p) { norm_quant_body<E, NQ_EMB>(p); }
template <int E> __global__ __launch_bounds__(512) void k_norm_quant_x(q3_nq p) { norm_quant_body<E, NQ_X>(p); }

__global__ __launch_bounds__(256) void k_qkv_post(q3_qkv p) {
    __shared__ float v[Q3_MAX_HD];
    __shared__ __align__(16) float red[16];
    const int HD = p.HD, half = HD >> 1, d = threadIdx.x;
    const int h = blockIdx.x, t = blockIdx.y;
    const int QD = p.NH * HD, KVD = p.NKV * HD;
    const int pos = p.st[0] + t;
    if (pos >= p.max_ctx) return; // the host refuses such a step; never write past the cache
    const bool kv = h >= p.NH;
    const int g = h - p.NH;
    const int32_t *__restrict__ c = kv ? p.ck + (size_t)t * KVD + g * HD : p.cq + (size_t)t * QD + h * HD;
    const float *__restrict__ ws = kv ? p.wsk + g * HD : p.wsq + h * HD;
    const float *__restrict__ nw = kv ? p.kn : p.qn;
    // every load first
    const int i = d < half ? d : d - half;
    const int32_t cd = c[d];
    const float wd = ws[d], nwd = nw[d], as = p.as[t];
    const float cs = p.rcos[(size_t)pos * half + i], sn = p.rsin[(size_t)pos * half + i];
    const int gv = kv ? g : 0; // unconditional loads (q heads read kv head 0's and drop it)
    const int32_t cvd = p.cv[(size_t)t * KVD + gv * HD + d];
    const float wvd = p.wsv[gv * HD + d];
    const float x = ((float)cd * as) * wd;
    const float ss = block_sum(x * x, red);
    const float r = 1.0f / sqrtf(ss / (float)HD + p.eps);
    v[d] = (x * r) * nwd;
    __syncthreads();
    // NeoX rotate-halves (examples/bench.c:76): pairs (i, i + HD/2) at angle pos * theta^(-2i/HD)
    const float a = v[i], b = v[i + half];
    const float o = d < half ? a * cs - b * sn : a * sn + b * cs;
    if (kv) {
        p.kc[(size_t)pos * KVD + g * HD + d] = o;
        p.vc[(size_t)pos * KVD + g * HD + d] = ((float)cvd * as) * wvd;
    } else {
        p.q[(size_t)t * QD + h * HD + d] = o;
    }
}

// One workgroup per (kv head, sub-group of GW query heads, Q3_CHUNK-key chunk, query row), GW * HD <= 256
// threads: thread (g, d) = query head g of the sub-group, dimension d. Every global load is issued up
// front and unconditionally (rows past the chunk's last key repeat that key; their probabilities are
// zero): the chunk's K rows go to LDS as float4, each thread's V column stays in registers. Query head g's
// keys are scored one per lane on Q3_CHUNK consecutive lanes, so the chunk's softmax statistics are two
// lane-group reductions. 32-key chunks (rather than 64) halve each workgroup's K/V bytes, which bound it.
// FUSED (one query row, decode): the workgroup also does k_qkv_post's work for itself -- dequantises,
// normalises and rotates its query heads from the q/k/v matmul results, and the workgroup whose chunk
// holds the current position builds that position's K/V row (appending it to the cache) -- which saves
// a launch and a round trip through HBM per layer.
template <int GW, bool FUSED>
__global__ __launch_bounds__(256) void k_attn_part(q3_att p) {
    extern __shared__ float sm[];
    __shared__ float red[32];
    // the kernel arguments in one batch of scalar loads behind one wait (the compiler issued them where first used:
    // four waits in a row); 0.852 -> 0.842 ms per decode token, three alternations on one box
    asm volatile("" ::"s"(p.NH), "s"(p.NKV), "s"(p.HD), "s"(p.S), "s"(p.max_ctx), "s"(p.q), "s"(p.kc), "s"(p.vc),
                 "s"(p.st), "s"(p.scale), "s"(p.part));
    if constexpr (FUSED)
        asm volatile("" ::"s"(p.cq), "s"(p.ck), "s"(p.cv), "s"(p.as), "s"(p.wsq), "s"(p.wsk), "s"(p.wsv), "s"(p.qn),
                     "s"(p.kn), "s"(p.eps), "s"(p.rcos), "s"(p.rsin));
    const int HD = p.HD, half = HD >> 1, G = p.NH / p.NKV, KVD = p.NKV * HD, QD = p.NH * HD;
    const int nsub = G / GW, sub = blockIdx.x % nsub;
    const int kvh = blockIdx.x / nsub, h0 = kvh * G + sub * GW; // first query head
    const int s = blockIdx.y, t = blockIdx.z, tid = threadIdx.x;
    const int g = tid / HD, d = tid - g * HD;
    const int pos = p.st[0] + t;
    const int L = min(pos + 1, p.max_ctx); // causal: keys 0 .. pos (never past the cache)
    const int j0 = s * Q3_CHUNK;
    const int n = min(Q3_CHUNK, L - j0);
    float *out = p.part + (((size_t)t * p.NH + h0 + g) * p.S + s) * (HD + 2);
    if (n <= 0) { // whole workgroup: this chunk is beyond the row's keys
        out[d] = 0.f;
        if (d == 0) {
            out[HD] = -INFINITY;
            out[HD + 1] = 0.f;
        }
        return;
    }
    const int KS = HD + 4; // LDS row stride: 16-byte rows, 8 consecutive lanes of a float4 read hit distinct banks
    float *Ks = sm;
    float *qs = Ks + Q3_CHUNK * KS;
    float *P = qs + GW * HD;
    float *ml = P + GW * Q3_CHUNK; // [GW][2]: max, sum
    float *xs = ml + 2 * GW;       // FUSED: [GW][HD] normalised q, then [HD] k and [HD] v of the new row
    const float *__restrict__ kb = p.kc + (size_t)j0 * KVD + kvh * HD;
    const float *__restrict__ vb = p.vc + (size_t)j0 * KVD + kvh * HD + d;
    float vv[Q3_CHUNK];
#pragma unroll
    for (int j = 0; j < Q3_CHUNK; j++) vv[j] = vb[(size_t)min(j, n - 1) * KVD];
    // the chunk's Q3_CHUNK * HD / 4 float4s are exactly Q3_CHUNK / 4 / GW per thread (blockDim = GW * HD)
    const int HD4 = HD >> 2;
    constexpr int KR = Q3_CHUNK / 4 / GW;
    float4 kreg[KR];
#pragma unroll
    for (int k = 0; k < KR; k++) {
        const int f = tid + k * blockDim.x, j = f / HD4, c4 = f - j * HD4;
        kreg[k] = *(const float4 *)(kb + (size_t)min(j, n - 1) * KVD + 4 * c4);
    }
    const bool own = FUSED && pos - j0 < Q3_CHUNK; // this chunk holds the new row (row n - 1)
    int32_t cqd = 0, ckd = 0, cvd = 0;
    float wq = 0.f, wk = 0.f, wv = 0.f, qn = 0.f, kn = 0.f, as = 0.f, cs = 0.f, sn = 0.f;
    const int ri = d < half ? d : d - half;
    if (FUSED) {
        const int h = h0 + g;
        cqd = p.cq[h * HD + d];
        wq = p.wsq[h * HD + d];
        qn = p.qn[d];
        as = p.as[0];
        cs = p.rcos[(size_t)pos * half + ri];
        sn = p.rsin[(size_t)pos * half + ri];
        // the new row's k / v inputs: loaded by every workgroup (unconditional loads), used by the owner
        ckd = p.ck[kvh * HD + d];
        cvd = p.cv[kvh * HD + d];
        wk = p.wsk[kvh * HD + d];
        wv = p.wsv[kvh * HD + d];
        kn = p.kn[d];
    } else {
        qs[tid] = p.q[(size_t)t * QD + h0 * HD + tid];
    }
#pragma unroll
    for (int k = 0; k < KR; k++) {
        const int f = tid + k * blockDim.x, j = f / HD4, c4 = f - j * HD4;
        *(float4 *)(Ks + j * KS + 4 * c4) = kreg[k];
    }
    const int jn = n - 1;
    if (FUSED) {
        // per-head RMSNorm of q (and of the new k row): sums of squares over head g's HD threads
        const float xq = ((float)cqd * as) * wq;
        const float xk = ((float)ckd * as) * wk;
        const float a = wave_sum(xq * xq), b = wave_sum(xk * xk);
        const int w = tid >> 6, wph = HD >> 6;
        if ((tid & 63) == 0) {
            red[2 * w] = a;
            red[2 * w + 1] = b;
        }
        __syncthreads();
        float sq = 0.f, sk = 0.f;
        for (int i = 0; i < wph; i++) {
            sq += red[2 * (g * wph + i)];
            sk += red[2 * (g * wph + i) + 1];
        }
        const float rq = 1.0f / sqrtf(sq / (float)HD + p.eps);
        const float rk = 1.0f / sqrtf(sk / (float)HD + p.eps);
        xs[tid] = (xq * rq) * qn;
        float *kx = xs + GW * HD, *vx = kx + HD;
        if (own && g == 0) kx[d] = (xk * rk) * kn;
        __syncthreads();
        // NeoX rotate-halves (examples/bench.c:76)
        const float qa = xs[g * HD + ri], qb = xs[g * HD + ri + half];
        qs[tid] = d < half ? qa * cs - qb * sn : qa * sn + qb * cs;
        if (own && g == 0) {
            const float ka = kx[ri], kbv = kx[ri + half];
            const float ko = d < half ? ka * cs - kbv * sn : ka * sn + kbv * cs;
            const float vo = ((float)cvd * as) * wv;
            Ks[jn * KS + d] = ko;
            vx[d] = vo;
            if (sub == 0) { // one workgroup per kv head appends the row
                p.kc[(size_t)pos * KVD + kvh * HD + d] = ko;
                p.vc[(size_t)pos * KVD + kvh * HD + d] = vo;
            }
        }
    }
    __syncthreads();
    if (tid < GW * Q3_CHUNK) { // head gg's keys on Q3_CHUNK consecutive lanes
        const int gg = tid / Q3_CHUNK, j = tid % Q3_CHUNK;
        const float4 *qr = (const float4 *)(qs + gg * HD), *kr = (const float4 *)(Ks + j * KS);
        float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
        // unrolled so that eight iterations' LDS reads are in flight together (HD is a runtime value)
#pragma unroll 8
        for (int e = 0; e < HD4; e++) {
            const float4 qv = qr[e], kv = kr[e];
            a0 += qv.x * kv.x;
            a1 += qv.y * kv.y;
            a2 += qv.z * kv.z;
            a3 += qv.w * kv.w;
        }
        const float sc = j < n ? ((a0 + a1) + (a2 + a3)) * p.scale : -INFINITY;
        const float m = group_max<Q3_CHUNK>(sc);
        const float pj = j < n ? expf(sc - m) : 0.f;
        const float l = group_sum<Q3_CHUNK>(pj);
        P[gg * Q3_CHUNK + j] = pj;
        if (j == 0) {
            ml[2 * gg] = m;
            ml[2 * gg + 1] = l;
        }
    }
    __syncthreads();
    // in the chunk that holds the new row, rows jn.. of vv were loaded before that row existed (the cache
    // there is unwritten, possibly not even finite): the new V row replaces jn, zeros the rest
    const float vnew = own ? xs[GW * HD + HD + d] : 0.f;
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < Q3_CHUNK; j++)
        acc += P[g * Q3_CHUNK + j] * ((own && j >= jn) ? (j == jn ? vnew : 0.f) : vv[j]);
    out[d] = acc;
    if (d == 0) {
        out[HD] = ml[2 * g];
        out[HD + 1] = ml[2 * g + 1];
    }
}

// k_attn_rows: the prefill form of k_attn_part (M > 1 rows, rotated queries in p.q): one workgroup per (kv head's
// query-head group, key chunk, block of HD / Q3_CHUNK rows). The chunk's keys go to LDS and its values to registers
// once and serve every row of the block, every thread scoring one (row, head, key), instead of one workgroup
// reloading the chunk for each row. (Blocks of 16 rows measured slower, both as four such passes per workgroup and
// with register-blocked scores -- each wave scoring four rows per K row read from LDS: the scoring is per-thread
// latency, and 4x fewer workgroups left most CUs idle.) Each row's partials are computed with
// k_attn_part's operations in its order (the score sums, the 32-lane max and sum, the P.V accumulation), and a row
// with no key in the chunk gets k_attn_part's empty partial, so the partials are bit-identical to it.
template <int GW>
__global__ __launch_bounds__(256) void k_attn_rows(q3_att p) {
    extern __shared__ float sm[];
    const int HD = p.HD, G = p.NH / p.NKV, KVD = p.NKV * HD, QD = p.NH * HD;
    const int nsub = G / GW, sub = blockIdx.x % nsub;
    const int kvh = blockIdx.x / nsub, h0 = kvh * G + sub * GW; // first query head
    const int s = blockIdx.y, tid = threadIdx.x;
    const int g = tid / HD, d = tid - g * HD;
    const int RR = HD / Q3_CHUNK; // rows per workgroup: GW * Q3_CHUNK * RR threads score them together
    const int t0 = blockIdx.z * RR, t1 = min(t0 + RR, p.M); // rows t0 .. t1 - 1
    const int j0 = s * Q3_CHUNK;
    const int nmax = min(Q3_CHUNK, min(p.st[0] + t1, p.max_ctx) - j0); // keys of the block's last row
    if (nmax <= 0) { // no row of the block reaches this chunk
        for (int t = t0; t < t1; t++) {
            float *out = p.part + (((size_t)t * p.NH + h0 + g) * p.S + s) * (HD + 2);
            out[d] = 0.f;
            if (d == 0) {
                out[HD] = -INFINITY;
                out[HD + 1] = 0.f;
            }
        }
        return;
    }
    const int KS = HD + 4; // LDS row stride: 16-byte rows, 8 consecutive lanes of a float4 read hit distinct banks
    float *Ks = sm;
    float *qs = Ks + Q3_CHUNK * KS; // [RR][GW][HD]
    float *P = qs + RR * GW * HD;   // [RR][GW][Q3_CHUNK]
    float *ml = P + RR * GW * Q3_CHUNK; // [RR][GW][2]
    const float *__restrict__ kb = p.kc + (size_t)j0 * KVD + kvh * HD;
    const float *__restrict__ vb = p.vc + (size_t)j0 * KVD + kvh * HD + d;
    float vv[Q3_CHUNK];
#pragma unroll
    for (int j = 0; j < Q3_CHUNK; j++) vv[j] = vb[(size_t)min(j, nmax - 1) * KVD];
    const int HD4 = HD >> 2;
    constexpr int KR = Q3_CHUNK / 4 / GW;
    float4 kreg[KR];
#pragma unroll
    for (int k = 0; k < KR; k++) {
        const int f = tid + k * blockDim.x, j = f / HD4, c4 = f - j * HD4;
        kreg[k] = *(const float4 *)(kb + (size_t)min(j, nmax - 1) * KVD + 4 * c4);
    }
#pragma unroll
    for (int k = 0; k < KR; k++) {
        const int f = tid + k * blockDim.x, j = f / HD4, c4 = f - j * HD4;
        *(float4 *)(Ks + j * KS + 4 * c4) = kreg[k];
    }
    for (int r0 = t0; r0 < t1; r0 += RR) {
        for (int rr = 0; rr < RR; rr++) {
            const int t = min(r0 + rr, t1 - 1);
            qs[rr * GW * HD + tid] = p.q[(size_t)t * QD + h0 * HD + tid];
        }
        __syncthreads(); // keys (first pass) and this pass's queries
        {   // scores: thread = (row rr, head gg, key j)
            const int rr = tid / (GW * Q3_CHUNK), gg = (tid / Q3_CHUNK) % GW, j = tid % Q3_CHUNK;
            const int t = r0 + rr;
            const int n = min(Q3_CHUNK, min(p.st[0] + t + 1, p.max_ctx) - j0);
            const float4 *qr = (const float4 *)(qs + (rr * GW + gg) * HD), *kr = (const float4 *)(Ks + j * KS);
            float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll 8
            for (int e = 0; e < HD4; e++) {
                const float4 qv = qr[e], kv = kr[e];
                a0 += qv.x * kv.x;
                a1 += qv.y * kv.y;
                a2 += qv.z * kv.z;
                a3 += qv.w * kv.w;
            }
            const float sc = j < n ? ((a0 + a1) + (a2 + a3)) * p.scale : -INFINITY;
            const float m = group_max<Q3_CHUNK>(sc);
            const float pj = j < n ? expf(sc - m) : 0.f;
            const float l = group_sum<Q3_CHUNK>(pj);
            P[(rr * GW + gg) * Q3_CHUNK + j] = pj;
            if (j == 0) {
                ml[2 * (rr * GW + gg)] = m;
                ml[2 * (rr * GW + gg) + 1] = l;
            }
        }
        __syncthreads();
        for (int rr = 0; rr < RR && r0 + rr < t1; rr++) {
            const int t = r0 + rr;
            float *out = p.part + (((size_t)t * p.NH + h0 + g) * p.S + s) * (HD + 2);
            const int n = min(Q3_CHUNK, min(p.st[0] + t + 1, p.max_ctx) - j0);
            if (n <= 0) { // k_attn_part's empty partial
                out[d] = 0.f;
                if (d == 0) {
                    out[HD] = -INFINITY;
                    out[HD + 1] = 0.f;
                }
                continue;
            }
            float acc = 0.f;
#pragma unroll
            for (int j = 0; j < Q3_CHUNK; j++) acc += P[(rr * GW + g) * Q3_CHUNK + j] * vv[j];
            out[d] = acc;
            if (d == 0) {
                out[HD] = ml[2 * (rr * GW + g)];
                out[HD + 1] = ml[2 * (rr * GW + g) + 1];
            }
        }
        __syncthreads(); // this pass's P and queries read before the next pass writes them
    }
}


// Combine the chunks of every head (log-sum-exp weights), then quantise the row. Each thread's partial
// sums are loaded before the chunk weights are known, so the kernel pays one round trip to memory.
template <int E, int MS>
__device__ inline void attn_quant_body(const q3_aq &p) {
    extern __shared__ float sm[];
    const int HD = p.HD, NH = p.NH, S = p.S, QD = NH * HD, t = blockIdx.x;
    const float *__restrict__ part = p.part + (size_t)t * NH * S * (HD + 2);
    float *w = sm, *ls = sm + NH * S, *inv = ls + NH * S;
    float acc[E][MS];
#pragma unroll
    for (int k = 0; k < E; k++) {
        const int i = min((int)(threadIdx.x + k * blockDim.x), QD - 1);
        const int h = i / HD, d = i - h * HD;
        const float *ph = part + (size_t)h * S * (HD + 2) + d;
#pragma unroll
        for (int s = 0; s < MS; s++) {
            const float x = ph[(size_t)min(s, S - 1) * (HD + 2)];
            acc[k][s] = s < S ? x : 0.f;
        }
    }
    for (int i = threadIdx.x; i < NH * S; i += blockDim.x) {
        w[i] = part[(size_t)i * (HD + 2) + HD];
        ls[i] = part[(size_t)i * (HD + 2) + HD + 1];
    }
    __syncthreads();
    // chunk weights, one wave per head, lane s = chunk s (S <= Q3_MAX_S <= 64): e_s = exp(m_s - max m) and
    // 1 / sum_s l_s e_s
    for (int h = (int)(threadIdx.x >> 6); h < NH; h += (int)(blockDim.x >> 6)) {
        const int ln = threadIdx.x & 63, sc = min(ln, S - 1);
        const float m0 = w[h * S + sc], l0 = ls[h * S + sc];
        const float m = ln < S ? m0 : -INFINITY;
        const float mx = wave_max(m);
        const float e = m == -INFINITY ? 0.f : expf(m - mx);
        const float den = wave_sum(ln < S ? l0 * e : 0.f);
        if (ln < S) w[h * S + ln] = e;
        if (ln == 0) inv[h] = den > 0.f ? 1.0f / den : 0.f;
    }
    __syncthreads();
    float y[E];
#pragma unroll
    for (int k = 0; k < E; k++) {
        const int i = threadIdx.x + k * blockDim.x;
        const int h = min(i, QD - 1) / HD;
        float num = 0.f;
#pragma unroll
        for (int s = 0; s < MS; s++)
            if (s < S) num += acc[k][s] * w[h * S + s];
        y[k] = i < QD ? num * inv[h] : 0.f;
    }
    quant_regs(y, QD, p.a8 + (size_t)t * QD, p.as + t);
}
template <int E> __global__ __launch_bounds__(1024) void k_attn_quant8(q3_aq p) { attn_quant_body<E, 8>(p); }
template <int E> __global__ __launch_bounds__(1024) void k_attn_quant16(q3_aq p) { attn_quant_body<E, 16>(p); }
template <int E> __global__ __launch_bounds__(1024) void k_attn_quant32(q3_aq p) { attn_quant_body<E, 32>(p); }

template <int E>
__global__ __launch_bounds__(1024) void k_swiglu_quant(q3_glu p) {
    const int F = p.F, t = blockIdx.x;
    int32_t cg[E], cu[E];
    float wg[E], wu[E], y[E];
    load_row(cg, p.cg + (size_t)t * F, F);
    load_row(cu, p.cu + (size_t)t * F, F);
    load_row(wg, p.wsg, F);
    load_row(wu, p.wsu, F);
    const float as = p.as_in[t];
#pragma unroll
    for (int k = 0; k < E; k++) {
        const float gv = ((float)cg[k] * as) * wg[k];
        const float uv = ((float)cu[k] * as) * wu[k];
        y[k] = (gv / (1.0f + expf(-gv))) * uv;
    }
    quant_regs(y, F, p.a8 + (size_t)t * F, p.as_out + t);
}

// Order-preserving map of a float to 32 bits (larger float -> larger unsigned).
__device__ inline unsigned ord_bits(float v) {
    const unsigned u = __float_as_uint(v);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__global__ void k_argmax(q3_amax p) {
    __shared__ unsigned long long red[16];
    const float as = *p.as;
    unsigned long long best = 0ull;
    for (int n = blockIdx.x * blockDim.x + threadIdx.x; n < p.V; n += gridDim.x * blockDim.x) {
        const float v = ((float)p.c[n] * as) * p.ws[n];
        // ties resolve to the smaller index (the first maximum), as a sequential scan does
        const unsigned long long k = ((unsigned long long)ord_bits(v) << 32) | (0xFFFFFFFFu - (unsigned)n);
        best = k > best ? k : best;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const unsigned long long x = __shfl_xor(best, o, 64);
        best = x > best ? x : best;
    }
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int i = 1; i < (int)(blockDim.x >> 6); i++) best = red[i] > best ? red[i] : best;
        atomicMax(p.best, best);
    }
}

// k_attn_combine: one workgroup per query head, thread d = dimension d: the log-sum-exp combine of the head's
// chunks with attn_quant_body's operations in its order, so the row equals the one that kernel quantises.
__global__ __launch_bounds__(Q3_MAX_HD) void k_attn_combine(q3_comb p) {
    __shared__ float w[Q3_MAX_S];
    __shared__ float inv;
    const int h = blockIdx.x, HD = p.HD, S = p.S, d = threadIdx.x;
    const float *__restrict__ ph = p.part + (size_t)h * S * (HD + 2);
    float acc[Q3_MAX_S];
#pragma unroll
    for (int s = 0; s < Q3_MAX_S; s++) {
        const float x = ph[(size_t)min(s, S - 1) * (HD + 2) + d];
        acc[s] = s < S ? x : 0.f;
    }
    if (threadIdx.x < 64) {
        const int ln = threadIdx.x, sc = min(ln, S - 1);
        const float m0 = ph[(size_t)sc * (HD + 2) + HD], l0 = ph[(size_t)sc * (HD + 2) + HD + 1];
        const float m = ln < S ? m0 : -INFINITY;
        const float mxm = wave_max(m);
        const float e = m == -INFINITY ? 0.f : expf(m - mxm);
        const float den = wave_sum(ln < S ? l0 * e : 0.f);
        if (ln < S) w[ln] = e;
        if (ln == 0) inv = den > 0.f ? 1.0f / den : 0.f;
    }
    __syncthreads();
    float num = 0.f;
#pragma unroll
    for (int s = 0; s < Q3_MAX_S; s++)
        if (s < S) num += acc[s] * w[s];
    p.out[(size_t)h * HD + d] = num * inv;
}

inline int launch_ok() { return hipGetLastError() == hipSuccess ? 0 : -1; }

// A plain copy of n floats (the decoder's layer-input trace); a kernel rather than a copy command, so that it is
// an ordinary node of a captured decode step.
__global__ __launch_bounds__(256) void k_copy_f32(float *__restrict__ dst, const float *__restrict__ src, long long n) {
    const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
    if (i < n) dst[i] = src[i];
}

} // namespace

extern "C" {

// Register-row templates: E elements per thread, the smallest instantiated width that covers the row.
#define Q3_ROW_DISPATCH(KERNEL, THREADS, N, GRID, LDS, STREAM, ARG)                                           \
    do {                                                                                                      \
        const int e_ = ((N) + (THREADS)-1) / (THREADS);                                                       \
        if (e_ <= 1) hipLaunchKernelGGL(KERNEL<1>, GRID, dim3(THREADS), LDS, STREAM, ARG);                     \
        else if (e_ <= 2) hipLaunchKernelGGL(KERNEL<2>, GRID, dim3(THREADS), LDS, STREAM, ARG);                \
        else if (e_ <= 3) hipLaunchKernelGGL(KERNEL<3>, GRID, dim3(THREADS), LDS, STREAM, ARG);                \
        else if (e_ <= 4) hipLaunchKernelGGL(KERNEL<4>, GRID, dim3(THREADS), LDS, STREAM, ARG);                \
        else if (e_ <= 6) hipLaunchKernelGGL(KERNEL<6>, GRID, dim3(THREADS), LDS, STREAM, ARG);                \
        else if (e_ <= 8) hipLaunchKernelGGL(KERNEL<8>, GRID, dim3(THREADS), LDS, STREAM, ARG);                \
        else if (e_ <= 12) hipLaunchKernelGGL(KERNEL<12>, GRID, dim3(THREADS), LDS, STREAM, ARG);              \
        else if (e_ <= 16) hipLaunchKernelGGL(KERNEL<16>, GRID, dim3(THREADS), LDS, STREAM, ARG);              \
        else return -2;                                                                                       \
    } while (0)

int q3k_norm_quant(const q3_nq *p, void *stream) {
    if (p->M < 1 || p->H < 64 || p->H > 512 * 16 || (p->emb && !p->tok && p->M != 1) || (p->emb && p->acc)) return -2;
    if (p->emb) Q3_ROW_DISPATCH(k_norm_quant_emb, 512, p->H, dim3(p->M), 0, (hipStream_t)stream, *p);
    else if (p->acc) Q3_ROW_DISPATCH(k_norm_quant_acc, 512, p->H, dim3(p->M), 0, (hipStream_t)stream, *p);
    else Q3_ROW_DISPATCH(k_norm_quant_x, 512, p->H, dim3(p->M), 0, (hipStream_t)stream, *p);
    return launch_ok();
}

int q3k_copy_f32(float *dst, const float *src, long long n, void *stream) {
    if (n < 1 || !dst || !src) return -2;
    const long long grid = (n + 255) / 256;
    if (grid >= (1LL << 31)) return -2;
    hipLaunchKernelGGL(k_copy_f32, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream, dst, src, n);
    return launch_ok();
}

int q3k_qkv_post(const q3_qkv *p, void *stream) {
    if (p->M < 1 || p->HD < 64 || p->HD > Q3_MAX_HD || p->HD % 64) return -2;
    hipLaunchKernelGGL(k_qkv_post, dim3(p->NH + p->NKV, p->M), dim3(p->HD), 0, (hipStream_t)stream, *p);
    return launch_ok();
}

int q3k_attn_part(const q3_att *p, void *stream) {
    const int G = p->NKV > 0 ? p->NH / p->NKV : 0;
    if (p->M < 1 || G < 1 || G * p->NKV != p->NH || p->HD % 64 || p->HD > Q3_MAX_HD || p->HD < Q3_CHUNK ||
        p->S < 1 || (long)p->S * Q3_CHUNK < p->max_ctx || (p->cq && p->M != 1) || (!p->cq && !p->q))
        return -2;
    int GW = 256 / p->HD; // query heads per workgroup: the largest divisor of G with GW * HD <= 256
    if (GW > G) GW = G;
    while (G % GW) GW--;
    const size_t lds = Q3_ATT_LDS(GW, p->HD);
    if (lds > 64 * 1024) return -2;
    const dim3 grid(p->NKV * (G / GW), p->S, p->M), block(GW * p->HD);
    const hipStream_t st = (hipStream_t)stream;
    const bool fused = p->cq != nullptr;
    if (!fused && p->rows) { // prefill: the chunk once per block of rows
        const size_t lr = (size_t)(Q3_CHUNK * (p->HD + 4) + (p->HD / Q3_CHUNK) * GW * (p->HD + Q3_CHUNK + 2)) * 4;
        const int rr = p->HD / Q3_CHUNK;
        const dim3 gr(p->NKV * (G / GW), p->S, (p->M + rr - 1) / rr);
        if (lr > 64 * 1024) return -2;
        if (GW == 1) hipLaunchKernelGGL((k_attn_rows<1>), gr, block, lr, st, *p);
        else if (GW == 2) hipLaunchKernelGGL((k_attn_rows<2>), gr, block, lr, st, *p);
        else if (GW == 4) hipLaunchKernelGGL((k_attn_rows<4>), gr, block, lr, st, *p);
        else return -2;
        return launch_ok();
    }
    if (GW == 1) {
        if (fused) hipLaunchKernelGGL((k_attn_part<1, true>), grid, block, lds, st, *p);
        else hipLaunchKernelGGL((k_attn_part<1, false>), grid, block, lds, st, *p);
    } else if (GW == 2) {
        if (fused) hipLaunchKernelGGL((k_attn_part<2, true>), grid, block, lds, st, *p);
        else hipLaunchKernelGGL((k_attn_part<2, false>), grid, block, lds, st, *p);
    } else if (GW == 4) {
        if (fused) hipLaunchKernelGGL((k_attn_part<4, true>), grid, block, lds, st, *p);
        else hipLaunchKernelGGL((k_attn_part<4, false>), grid, block, lds, st, *p);
    } else {
        return -2;
    }
    return launch_ok();
}

int q3k_attn_quant(const q3_aq *p, void *stream) {
    const size_t lds = (size_t)(2 * p->NH * p->S + p->NH) * sizeof(float);
    if (p->M < 1 || p->NH * p->HD > 1024 * 16 || p->S > Q3_MAX_S || lds > 32 * 1024) return -2;
    // chunk loop bound: the smallest instantiated one covering S (each chunk is one load per element)
    if (p->S <= 8) Q3_ROW_DISPATCH(k_attn_quant8, 1024, p->NH * p->HD, dim3(p->M), lds, (hipStream_t)stream, *p);
    else if (p->S <= 16) Q3_ROW_DISPATCH(k_attn_quant16, 1024, p->NH * p->HD, dim3(p->M), lds, (hipStream_t)stream, *p);
    else Q3_ROW_DISPATCH(k_attn_quant32, 1024, p->NH * p->HD, dim3(p->M), lds, (hipStream_t)stream, *p);
    return launch_ok();
}

int q3k_swiglu_quant(const q3_glu *p, void *stream) {
    if (p->M < 1 || p->F > 1024 * 16) return -2;
    Q3_ROW_DISPATCH(k_swiglu_quant, 1024, p->F, dim3(p->M), 0, (hipStream_t)stream, *p);
    return launch_ok();
}

int q3k_argmax(const q3_amax *p, void *stream) {
    if (p->V < 1) return -2;
    int grid = (p->V + 1023) / 1024;
    if (grid > 512) grid = 512;
    hipLaunchKernelGGL(k_argmax, dim3(grid), dim3(256), 0, (hipStream_t)stream, *p);
    return launch_ok();
}

int q3k_attn_combine(const q3_comb *p, void *stream) {
    if (p->NH < 1 || p->HD < 64 || p->HD > Q3_MAX_HD || p->HD % 64 || p->S < 1 || p->S > Q3_MAX_S || !p->part ||
        !p->out)
        return -2;
    hipLaunchKernelGGL(k_attn_combine, dim3(p->NH), dim3(p->HD), 0, (hipStream_t)stream, *p);
    return launch_ok();
}

// ---- HIP graphs for the decode step ----------------------------------------------------------------------
int q3g_begin(void *stream) {
    return hipStreamBeginCapture((hipStream_t)stream, hipStreamCaptureModeThreadLocal) == hipSuccess ? 0 : -1;
}

int q3g_end(void *stream, void **exec) {
    hipGraph_t g = nullptr;
    if (hipStreamEndCapture((hipStream_t)stream, &g) != hipSuccess || !g) return -1;
    hipGraphExec_t e = nullptr;
    const hipError_t rc = hipGraphInstantiate(&e, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (rc != hipSuccess) return -1;
    *exec = e;
    return 0;
}

int q3g_launch(void *exec, void *stream) {
    return hipGraphLaunch((hipGraphExec_t)exec, (hipStream_t)stream) == hipSuccess ? 0 : -1;
}

void q3g_destroy(void *exec) {
    if (exec) (void)hipGraphExecDestroy((hipGraphExec_t)exec);
}

int q3g_sync(void *stream) { return hipStreamSynchronize((hipStream_t)stream) == hipSuccess ? 0 : -1; }

// Event-timed region on the stream: q3t_begin records a start event, q3t_end a stop event, waits for it
// and returns the elapsed milliseconds (negative on error).
int q3t_begin(void *stream, void **ev) {
    hipEvent_t e[2];
    if (hipEventCreate(&e[0]) != hipSuccess) return -1;
    if (hipEventCreate(&e[1]) != hipSuccess) { (void)hipEventDestroy(e[0]); return -1; }
    if (hipEventRecord(e[0], (hipStream_t)stream) != hipSuccess) {
        (void)hipEventDestroy(e[0]);
        (void)hipEventDestroy(e[1]);
        return -1;
    }
    ev[0] = e[0];
    ev[1] = e[1];
    return 0;
}

double q3t_end(void *stream, void **ev) {
    hipEvent_t e0 = (hipEvent_t)ev[0], e1 = (hipEvent_t)ev[1];
    float ms = -1.f;
    if (hipEventRecord(e1, (hipStream_t)stream) != hipSuccess || hipEventSynchronize(e1) != hipSuccess ||
        hipEventElapsedTime(&ms, e0, e1) != hipSuccess)
        ms = -1.f;
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    return ms;
}

} // extern "C"
