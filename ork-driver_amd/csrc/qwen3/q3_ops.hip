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

namespace {


// Wave-wide sum / max in every lane, on the cross-lane paths of the VALU: DPP quad_perm swaps (lanes
// l ^ 1, l ^ 2), DPP row_half_mirror and row_mirror (the other quad of an 8-lane half, the other half of a
// 16-lane row), then v_permlane16_swap / v_permlane32_swap (l ^ 16, l ^ 32). Every step combines the same two
// partials in every lane (a + b == b + a), so all lanes hold the identical result. Six LDS-crossbar shuffles
// (ds_bpermute) did the same in ~5x the latency.
template <int CTRL> __device__ inline float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ inline float xor16(float v) {
    const auto s = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(int, v), __builtin_bit_cast(int, v), false, false);
    return __builtin_bit_cast(float, (int)((threadIdx.x & 16) == 0 ? s[1] : s[0]));
}
__device__ inline float xor32(float v) {
    const auto s = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(int, v), __builtin_bit_cast(int, v), false, false);
    return __builtin_bit_cast(float, (int)((threadIdx.x & 32) == 0 ? s[1] : s[0]));
}
__device__ inline float wave_sum(float v) {
    v = v + dpp<0xB1>(v);  // quad_perm [1,0,3,2]
    v = v + dpp<0x4E>(v);  // quad_perm [2,3,0,1]
    v = v + dpp<0x141>(v); // row_half_mirror
    v = v + dpp<0x140>(v); // row_mirror
    v = v + xor16(v);
    return v + xor32(v);
}
__device__ inline float wave_max(float v) {
    v = fmaxf(v, dpp<0xB1>(v));
    v = fmaxf(v, dpp<0x4E>(v));
    v = fmaxf(v, dpp<0x141>(v));
    v = fmaxf(v, dpp<0x140>(v));
    v = fmaxf(v, xor16(v));
    return fmaxf(v, xor32(v));
}
// The same over aligned groups of W lanes (W = 32 or 64): a group's result in each of its lanes.
template <int W> __device__ inline float group_sum(float v) {
    static_assert(W == 32 || W == 64, "group width");
    v = v + dpp<0xB1>(v);
    v = v + dpp<0x4E>(v);
    v = v + dpp<0x141>(v);
    v = v + dpp<0x140>(v);
    v = v + xor16(v);
    if constexpr (W == 64) v = v + xor32(v);
    return v;
}
template <int W> __device__ inline float group_max(float v) {
    static_assert(W == 32 || W == 64, "group width");
    v = fmaxf(v, dpp<0xB1>(v));
    v = fmaxf(v, dpp<0x4E>(v));
    v = fmaxf(v, dpp<0x141>(v));
    v = fmaxf(v, dpp<0x140>(v));
    v = fmaxf(v, xor16(v));
    if constexpr (W == 64) v = fmaxf(v, xor32(v));
    return v;
}

// Block-wide sum / max (blockDim a multiple of 64, at most 1024). red[] holds 16 floats, 16-byte aligned, and
// must not be in use by another reduction of the same workgroup (each call site has its own): one barrier,
// after which every thread folds the waves' partials in wave order (float4 LDS reads where they fill).
__device__ inline float block_sum(float v, float *red) {
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    const int nw = (int)(blockDim.x >> 6);
    float s = 0.f;
    if ((nw & 3) == 0) {
        const float4 *r4 = (const float4 *)red;
        for (int i = 0; i < nw >> 2; i++) {
            const float4 q = r4[i];
            s = s + q.x;
            s = s + q.y;
            s = s + q.z;
            s = s + q.w;
        }
    } else {
        for (int i = 0; i < nw; i++) s = s + red[i];
    }
    return s;
}
__device__ inline float block_max(float v, float *red) {
    v = wave_max(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    const int nw = (int)(blockDim.x >> 6);
    float m = -INFINITY;
    if ((nw & 3) == 0) {
        const float4 *r4 = (const float4 *)red;
        for (int i = 0; i < nw >> 2; i++) {
            const float4 q = r4[i];
            m = fmaxf(fmaxf(m, q.x), fmaxf(q.y, fmaxf(q.z, q.w)));
        }
    } else {
        for (int i = 0; i < nw; i++) m = fmaxf(m, red[i]);
    }
    return m;
}

// Rows live in registers: thread i holds elements i, i + blockDim, ... (E of them, E a compile-time
// bound), so every global load of a row is issued before the first arithmetic that needs it. Loads are
// unconditional (from a clamped index, zeroed after): a load under a per-lane condition becomes a branch
// whose join waits for that load, which would serialise the row's loads into one round trip each.
template <int E, typename T>
__device__ inline void load_row(T (&v)[E], const T *__restrict__ src, int n) {
#pragma unroll
    for (int k = 0; k < E; k++) {
        const int i = threadIdx.x + k * blockDim.x;
        const T x = src[min(i, n - 1)];
        v[k] = i < n ? x : T(0);
    }
}

// Per-row symmetric int8 (examples/quant.c:34-37): s = max|x| / 127 (1 when the row is zero),
// q = clamp(rint(x / s), -127, 127). x * (1/s) is within 2 ulp of the correctly rounded x / s, so it
// rounds to the same integer unless it lies within 1e-4 of a half-way point (|x / s| <= 127.5, where
// 2 ulp < 1.6e-5); there the exact quotient decides.
template <int E>
__device__ inline void quant_regs(const float (&y)[E], int n, int8_t *__restrict__ q, float *s_out) {
    __shared__ __align__(16) float redq[16];
    float mx = 0.f;
#pragma unroll
    for (int k = 0; k < E; k++)
        if (threadIdx.x + k * blockDim.x < (unsigned)n) mx = fmaxf(mx, fabsf(y[k]));
    mx = block_max(mx, redq);
    const float s = mx > 0.f ? mx / 127.0f : 1.0f;
    const float inv = 1.0f / s;
#pragma unroll
    for (int k = 0; k < E; k++) {
        const int i = threadIdx.x + k * blockDim.x;
        if (i < n) {
            float r = y[k] * inv;
            if (fabsf(r - floorf(r) - 0.5f) < 1e-4f) r = y[k] / s;
            r = fminf(fmaxf(rintf(r), -127.f), 127.f);
            q[i] = (int8_t)(int)r;
        }
    }
    if (threadIdx.x == 0) *s_out = s;
}

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

// ---- fused M = 1 matmul of the decode step ------------------------------------------------------------------
// k_fgemv: one 16-column panel per workgroup (pair mode: the same columns of two weights), 8 waves splitting the
// panel's K-blocks, on the library's resident layout (lane l of a 1 KiB block holds 16 bytes of column l % 16,
// k-group l / 16); with H, half a panel per workgroup (8 columns, twice the workgroups: the bytes spread evenly
// over the CUs where whole panels would leave some CUs one panel and others two, or none). Around that GEMV:
//   prologue: the int8 row, built in LDS by every workgroup: PRO_NORM = RMSNorm of the residual row then the
//     per-row quant (norm_quant_body's operations with its 512-thread element mapping, so the sum of squares is
//     rounded identically: elements past K add exact zeros, so any E >= K / 512 gives the same sums);
//     PRO_QUANT = the per-row quant of a float row (quant_regs' operations; the absmax is order-independent).
//     Each wave's weight blocks (PRE >= its share, no more: a load past the share would fetch another wave's
//     bytes again) are loaded once the row has arrived: their latency hides behind the reductions and the
//     quant, and the row's own loads do not queue behind them in the CU's memory pipeline (measured: issuing
//     them first delayed the row by 1-2 us).
//   epilogue on each column's int32 sum: STORE; RESID x[n] += (c * a_scale) * ws[n] (the residual add that
//     k_norm_quant_acc would do next); SWIGLU y[n] = silu(g) * u from the gate and up sums (k_swiglu_quant's
//     operations).
// So the rows, scales and results equal those of the unfused kernels bit for bit.
typedef int v4i_t __attribute__((ext_vector_type(4)));

struct FgLut { uint32_t l0, l1, l2, l3; };
// One dword of NF4 codes -> the int8 codebook values of its low nibbles (lo) and of its high nibbles (hi):
// v_perm selects within the 8 bytes of two LUT words by the low 3 bits of each code, and a second v_perm takes
// that from the upper or the lower LUT half by the code's top bit.
__device__ inline void fg_nf4_map8(uint32_t x, const FgLut &L, uint32_t &lo, uint32_t &hi) {
    const uint32_t i0 = x & 0x07070707u, i1 = (x >> 4) & 0x07070707u;
    const uint32_t s0 = ((x >> 1) & 0x04040404u) | 0x03020100u;
    const uint32_t s1 = ((x >> 5) & 0x04040404u) | 0x03020100u;
    lo = __builtin_amdgcn_perm(__builtin_amdgcn_perm(L.l3, L.l2, i0), __builtin_amdgcn_perm(L.l1, L.l0, i0), s0);
    hi = __builtin_amdgcn_perm(__builtin_amdgcn_perm(L.l3, L.l2, i1), __builtin_amdgcn_perm(L.l1, L.l0, i1), s1);
}

// One lane's 16 bytes of a block against the row: int8 = 16 k; nibble kinds = 32 k, dword d holding
// k = 8 d .. 8 d + 3 in its low nibbles and 8 d + 4 .. 8 d + 7 in its high nibbles. Uniform int4 codes are
// widened as 16 v (the sum is shifted back once, exactly); NF4 codes map through the codebook.
template <int KIND>
__device__ inline int fg_dot(v4i_t raw, const int *__restrict__ a, int acc, const FgLut &L) {
    const uint32_t xs[4] = {(uint32_t)raw.x, (uint32_t)raw.y, (uint32_t)raw.z, (uint32_t)raw.w};
#pragma unroll
    for (int d = 0; d < 4; d++) {
        if constexpr (KIND == 0) {
            acc = __builtin_amdgcn_sdot4(a[d], (int)xs[d], acc, false);
        } else {
            uint32_t lo, hi;
            if constexpr (KIND == 1) {
                lo = (xs[d] << 4) & 0xf0f0f0f0u;
                hi = xs[d] & 0xf0f0f0f0u;
            } else {
                fg_nf4_map8(xs[d], L, lo, hi);
            }
            acc = __builtin_amdgcn_sdot4(a[2 * d], (int)lo, acc, false);
            acc = __builtin_amdgcn_sdot4(a[2 * d + 1], (int)hi, acc, false);
        }
    }
    return acc;
}

constexpr int FG_WAVES = 8; // 512 threads: norm_quant_body's element mapping

template <int PRO, int EPI, int KIND, int E, int PRE, int H>
__global__ __launch_bounds__(FG_WAVES * 64) void k_fgemv(q3_fg p) {
    __shared__ __align__(16) int8_t arow[Q3_FG_KMAX];
    __shared__ __align__(16) float red[16];
    __shared__ __align__(16) float redq[16];
    __shared__ int racc[FG_WAVES][2][16];
    constexpr bool PAIR = EPI == Q3_EPI_SWIGLU;
    constexpr int KPB = KIND == 0 ? 64 : 128;
    const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int K = p.K, KB = p.KB;

    // ---- this workgroup's panel(s) and this wave's K-blocks; H: columns 8 hh .. 8 hh + 7 of the panel(s), lane l
    // taking block kb + l / 32, k-group (l / 8) % 4, column 8 hh + l % 8 (a half block is four whole 128-byte lines)
    int t = 0, pnl = H ? (int)(blockIdx.x >> 1) : (int)blockIdx.x;
    const int hh = H ? (int)(blockIdx.x & 1) : 0, sub = H ? lane >> 5 : 0, grp = H ? (lane >> 3) & 3 : lane >> 4;
    const int loff = H ? grp * 16 + hh * 8 + (lane & 7) : lane;
    if constexpr (!PAIR) {
        while (t < p.nt - 1 && pnl >= p.nb[t]) {
            pnl -= p.nb[t];
            t++;
        }
    }
    const int kbw = (KB + FG_WAVES - 1) / FG_WAVES, kb0 = min(wv * kbw, KB), kb1 = min(kb0 + kbw, KB);
    const v4i_t *b0 = (const v4i_t *)p.B[t] + (size_t)pnl * KB * 64 + loff;
    const v4i_t *b1 = PAIR ? (const v4i_t *)p.B[1] + (size_t)pnl * KB * 64 + loff : b0;
    // ---- prologue: the int8 row in LDS
    float y[E], nw[E];
    load_row(y, p.row, K);
    if constexpr (PRO == Q3_PRO_NORM) load_row(nw, p.nw, K);
    float mx = 0.f, ss = 0.f;
    if constexpr (PRO == Q3_PRO_NORM) {
#pragma unroll
        for (int k = 0; k < E; k++) ss += y[k] * y[k];
    } else {
#pragma unroll
        for (int k = 0; k < E; k++)
            if (threadIdx.x + k * blockDim.x < (unsigned)K) mx = fmaxf(mx, fabsf(y[k]));
    }
    // the weight blocks, issued after the first use of the row (which waits for it); clamped to the wave's own
    // last block, branch-free (a wave without blocks re-reads the panel's last one and discards it). H: PRE load
    // instructions of two half blocks each
    v4i_t r0[PRE], r1[PRE];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < PRE; u++) {
        const size_t o = (size_t)min(kb0 + (H ? 2 * u + sub : u), kb1 - 1) * 64;
        r0[u] = __builtin_nontemporal_load(b0 + o);
        if constexpr (PAIR) r1[u] = __builtin_nontemporal_load(b1 + o);
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (PRO == Q3_PRO_NORM) {
        ss = block_sum(ss, red);
        const float r = 1.0f / sqrtf(ss / (float)K + p.eps);
#pragma unroll
        for (int k = 0; k < E; k++) y[k] = (y[k] * r) * nw[k];
#pragma unroll
        for (int k = 0; k < E; k++)
            if (threadIdx.x + k * blockDim.x < (unsigned)K) mx = fmaxf(mx, fabsf(y[k]));
    }
    mx = block_max(mx, redq);
    const float as = mx > 0.f ? mx / 127.0f : 1.0f;
    {
        const float inv = 1.0f / as;
#pragma unroll
        for (int k = 0; k < E; k++) {
            const int i = threadIdx.x + k * blockDim.x;
            if (i < K) {
                float r = y[k] * inv;
                if (fabsf(r - floorf(r) - 0.5f) < 1e-4f) r = y[k] / as;
                r = fminf(fmaxf(rintf(r), -127.f), 127.f);
                arow[i] = (int8_t)(int)r;
            }
        }
        for (int i = K + (int)threadIdx.x; i < KB * KPB; i += (int)blockDim.x) arow[i] = 0;
    }
    if (blockIdx.x == 0 && threadIdx.x == 0 && p.as_out) *p.as_out = as;
    __syncthreads();

    // ---- the GEMV: the preloaded blocks, then any further ones of this wave
    const FgLut L = {p.lut[0], p.lut[1], p.lut[2], p.lut[3]};
    const int aoff = grp * (KPB / 4);
    int acc0 = 0, acc1 = 0;
    if constexpr (H) {
        // a lane whose block lies past the run (the second half of an odd run's last instruction) adds nothing
#pragma unroll
        for (int u = 0; u < PRE; u++) {
            const int blk = kb0 + 2 * u + sub;
            const bool ok = blk < kb1;
            const int *a = (const int *)(arow + min(blk, kb1 - 1) * KPB + aoff);
            const int d0 = fg_dot<KIND>(r0[u], a, 0, L);
            acc0 += ok ? d0 : 0;
            if constexpr (PAIR) {
                const int d1 = fg_dot<KIND>(r1[u], a, 0, L);
                acc1 += ok ? d1 : 0;
            }
        }
        for (int kb = kb0 + 2 * PRE; kb < kb1; kb += 2) {
            const int blk = kb + sub;
            const bool ok = blk < kb1;
            const size_t o = (size_t)min(blk, kb1 - 1) * 64;
            const v4i_t s0 = __builtin_nontemporal_load(b0 + o);
            v4i_t s1 = s0;
            if constexpr (PAIR) s1 = __builtin_nontemporal_load(b1 + o);
            const int *a = (const int *)(arow + min(blk, kb1 - 1) * KPB + aoff);
            const int d0 = fg_dot<KIND>(s0, a, 0, L);
            acc0 += ok ? d0 : 0;
            if constexpr (PAIR) {
                const int d1 = fg_dot<KIND>(s1, a, 0, L);
                acc1 += ok ? d1 : 0;
            }
        }
    } else {
#pragma unroll
        for (int u = 0; u < PRE; u++) {
            if (kb0 + u < kb1) {
                const int *a = (const int *)(arow + (kb0 + u) * KPB + aoff);
                acc0 = fg_dot<KIND>(r0[u], a, acc0, L);
                if constexpr (PAIR) acc1 = fg_dot<KIND>(r1[u], a, acc1, L);
            }
        }
        for (int kb = kb0 + PRE; kb < kb1; kb++) {
            const v4i_t s0 = __builtin_nontemporal_load(b0 + (size_t)kb * 64);
            v4i_t s1 = s0;
            if constexpr (PAIR) s1 = __builtin_nontemporal_load(b1 + (size_t)kb * 64);
            const int *a = (const int *)(arow + kb * KPB + aoff);
            acc0 = fg_dot<KIND>(s0, a, acc0, L);
            if constexpr (PAIR) acc1 = fg_dot<KIND>(s1, a, acc1, L);
        }
    }
    // the k-groups of a column are lanes l, l ^ 16, l ^ 32, l ^ 48 (H: l ^ 8, l ^ 16, ..., l ^ 56: blocks and
    // k-groups); then the waves through LDS, in order
    {
        auto s32 = __builtin_amdgcn_permlane32_swap(acc0, acc0, false, false);
        acc0 += (int)((lane & 32) == 0 ? s32[1] : s32[0]);
        auto s16 = __builtin_amdgcn_permlane16_swap(acc0, acc0, false, false);
        acc0 += (int)((lane & 16) == 0 ? s16[1] : s16[0]);
        if constexpr (PAIR) {
            auto t32 = __builtin_amdgcn_permlane32_swap(acc1, acc1, false, false);
            acc1 += (int)((lane & 32) == 0 ? t32[1] : t32[0]);
            auto t16 = __builtin_amdgcn_permlane16_swap(acc1, acc1, false, false);
            acc1 += (int)((lane & 16) == 0 ? t16[1] : t16[0]);
        }
        if constexpr (H) {  // row_ror:8 -> lane l ^ 8 within its 16-lane row
            acc0 += __builtin_amdgcn_update_dpp(0, acc0, 0x128, 0xF, 0xF, false);
            if constexpr (PAIR) acc1 += __builtin_amdgcn_update_dpp(0, acc1, 0x128, 0xF, 0xF, false);
        }
    }
    if (lane < (H ? 8 : 16)) {
        racc[wv][0][lane] = acc0;
        racc[wv][1][lane] = acc1;
    }
    __syncthreads();
    if (threadIdx.x >= (H ? 8 : 16)) return;
    const int j = threadIdx.x;
    int c0 = 0, c1 = 0;
#pragma unroll
    for (int w = 0; w < FG_WAVES; w++) {
        c0 += racc[w][0][j];
        if constexpr (PAIR) c1 += racc[w][1][j];
    }
    if constexpr (KIND == 1) { // every block's partial is 16 x an integer
        c0 >>= 4;
        c1 >>= 4;
    }
    const int n = pnl * 16 + hh * 8 + j;
    if constexpr (EPI == Q3_EPI_STORE) {
        p.C[t][n] = c0;
    } else if constexpr (EPI == Q3_EPI_RESID) {
        p.x[n] = p.x[n] + ((float)c0 * as) * p.ws0[n];
    } else {
        const float gv = ((float)c0 * as) * p.ws0[n];
        const float uv = ((float)c1 * as) * p.ws1[n];
        p.y[n] = (gv / (1.0f + expf(-gv))) * uv;
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

// Fused M = 1 matmul (k_fgemv), the instantiations the decoder uses: PRO_NORM + STORE (q/k/v, int8), PRO_QUANT +
// RESID (o, int8; down, int8 / uniform int4 / NF4), PRO_NORM + SWIGLU (gate/up pairs, int8 / uniform int4 / NF4).
// E: row elements per thread, a bound of K / 512; PRE: the weight blocks per wave, a bound of its share (half
// panels, q3_fg.half: the load instructions of two half blocks each that cover it).
template <int PRO, int EPI, int KIND, int E>
void fg_launch_pre(const q3_fg *p, int grid, int pre, hipStream_t s) {
    const dim3 b(FG_WAVES * 64);
    if (p->half) {
        // load instructions (two half blocks each) covering the wave's share: every count the decoder's shapes take
        const int ni = (pre + 1) / 2, g2 = 2 * grid;
        if (ni <= 1) hipLaunchKernelGGL((k_fgemv<PRO, EPI, KIND, E, 1, 1>), dim3(g2), b, 0, s, *p);
        else if (ni <= 2) hipLaunchKernelGGL((k_fgemv<PRO, EPI, KIND, E, 2, 1>), dim3(g2), b, 0, s, *p);
        else if (ni <= 3) hipLaunchKernelGGL((k_fgemv<PRO, EPI, KIND, E, 3, 1>), dim3(g2), b, 0, s, *p);
        else if (ni <= 4) hipLaunchKernelGGL((k_fgemv<PRO, EPI, KIND, E, 4, 1>), dim3(g2), b, 0, s, *p);
        else if (ni <= 6) hipLaunchKernelGGL((k_fgemv<PRO, EPI, KIND, E, 6, 1>), dim3(g2), b, 0, s, *p);
        else hipLaunchKernelGGL((k_fgemv<PRO, EPI, KIND, E, 8, 1>), dim3(g2), b, 0, s, *p);
        return;
    }
    if (pre <= 4) hipLaunchKernelGGL((k_fgemv<PRO, EPI, KIND, E, 4, 0>), dim3(grid), b, 0, s, *p);
    else if (pre <= 8) hipLaunchKernelGGL((k_fgemv<PRO, EPI, KIND, E, 8, 0>), dim3(grid), b, 0, s, *p);
    else hipLaunchKernelGGL((k_fgemv<PRO, EPI, KIND, E, 16, 0>), dim3(grid), b, 0, s, *p);
}
template <int PRO, int EPI, int KIND> int fg_launch(const q3_fg *p, int grid, hipStream_t s) {
    const int e = (p->K + FG_WAVES * 64 - 1) / (FG_WAVES * 64), pre = (p->KB + FG_WAVES - 1) / FG_WAVES;
    if (e <= 4) fg_launch_pre<PRO, EPI, KIND, 4>(p, grid, pre, s);
    else if (e <= 8) fg_launch_pre<PRO, EPI, KIND, 8>(p, grid, pre, s);
    else if (e <= 12) fg_launch_pre<PRO, EPI, KIND, 12>(p, grid, pre, s);
    else if (e <= 16) fg_launch_pre<PRO, EPI, KIND, 16>(p, grid, pre, s);
    else return -2;
    return 0;
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

int q3k_fgemv(const q3_fg *p, void *stream) {
    const hipStream_t s_ = (hipStream_t)stream;
    if (p->kind < 0 || p->kind > 2 || p->epi < Q3_EPI_STORE || p->epi > Q3_EPI_SWIGLU) return -2;
    const int kpb = p->kind == 0 ? 64 : 128;
    const int pro = p->nw ? Q3_PRO_NORM : Q3_PRO_QUANT;
    const int nt = p->epi == Q3_EPI_SWIGLU ? 2 : p->epi == Q3_EPI_RESID ? 1 : p->nt;
    if (p->K < 32 || p->KB < 1 || (long)p->KB * kpb < p->K || (long)p->KB * kpb > Q3_FG_KMAX || nt < 1 || nt > 3 ||
        !p->row)
        return -2;
    int grid = 0;
    for (int i = 0; i < nt; i++) {
        if (!p->B[i] || p->nb[i] < 1) return -2;
        grid += p->nb[i];
    }
    int rc = -2;
    switch (p->epi) {
    case Q3_EPI_STORE:
        for (int i = 0; i < nt; i++)
            if (!p->C[i]) return -2;
        if (pro != Q3_PRO_NORM || p->kind != 0) return -2;
        rc = fg_launch<Q3_PRO_NORM, Q3_EPI_STORE, 0>(p, grid, s_);
        break;
    case Q3_EPI_RESID:
        if (pro != Q3_PRO_QUANT || !p->x || !p->ws0) return -2;
        if (p->kind == 0) rc = fg_launch<Q3_PRO_QUANT, Q3_EPI_RESID, 0>(p, grid, s_);
        else if (p->kind == 1) rc = fg_launch<Q3_PRO_QUANT, Q3_EPI_RESID, 1>(p, grid, s_);
        else rc = fg_launch<Q3_PRO_QUANT, Q3_EPI_RESID, 2>(p, grid, s_);
        break;
    default:
        if (pro != Q3_PRO_NORM || !p->y || !p->ws0 || !p->ws1 || p->nb[1] != p->nb[0]) return -2;
        grid = p->nb[0];
        if (p->kind == 0) rc = fg_launch<Q3_PRO_NORM, Q3_EPI_SWIGLU, 0>(p, grid, s_);
        else if (p->kind == 1) rc = fg_launch<Q3_PRO_NORM, Q3_EPI_SWIGLU, 1>(p, grid, s_);
        else rc = fg_launch<Q3_PRO_NORM, Q3_EPI_SWIGLU, 2>(p, grid, s_);
        break;
    }
    return rc ? rc : launch_ok();
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
