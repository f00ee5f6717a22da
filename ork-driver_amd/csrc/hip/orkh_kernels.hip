// orkh_kernels.hip -- gfx950 (MI355X, CDNA4) matmul kernels on resident panels, and their C-ABI launcher.
//
// These replace the reference's device programs for the matmul path: the int8 / fp16 / int4 regcmd
// synthesizers (src/npu/i8/regcmd.c:32-62, src/npu/f16/regcmd.c:303, src/npu/i4/run.c:97-124) and the
// host-side K-slice accumulation around them (src/npu.c:1764-1821). Panel layout: orkh.h.
//
// Two algorithms, both wave64 + MFMA:
//   k_stream  small M (<= 64): each wave streams a run of 1 KiB panel blocks straight from HBM into
//             registers (one coalesced 16 B load per lane per block), decodes int4 in registers and
//             issues v_mfma_i32_16x16x64_i8 / v_mfma_f32_16x16x32_f16 with the activations as the A
//             operand. The waves of a workgroup split K and reduce through LDS. HBM-bound by design:
//             the matrix cores idle most of the time, the load queue never does.
//   k_tiled   large M: 256-thread workgroup owns a BM x BN output tile; A fragments and B blocks are
//             staged through double-buffered LDS, each B byte crosses HBM once per XCD (the tile order
//             groups all M-tiles of an N-tile onto one XCD's L2).
// Integer results are exact (int32 accumulation, k order irrelevant). Uniform int4 nibbles are
// widened to 16*v in an int8 lane (v in [-8,7] -> [-128,112]); the int32 sum is then exactly 16x the
// true sum and an arithmetic >>4 recovers it.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include "orkh.h"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

template <int KIND> struct KT;
template <> struct KT<ORKH_I8> {
    static constexpr int KPB = 64, STEPS = 1, ESZ = 1;
    typedef v4i acc_t;
    typedef int32_t c_t;
};
template <> struct KT<ORKH_I4U> {
    static constexpr int KPB = 128, STEPS = 2, ESZ = 1;
    typedef v4i acc_t;
    typedef int32_t c_t;
};
template <> struct KT<ORKH_NF4> {
    static constexpr int KPB = 128, STEPS = 2, ESZ = 1;
    typedef v4i acc_t;
    typedef int32_t c_t;
};
template <> struct KT<ORKH_F16> {
    static constexpr int KPB = 32, STEPS = 1, ESZ = 2;
    typedef v4f acc_t;
    typedef float c_t;
};

// First k (within a K-block) of the 16-byte A chunk that lane group g feeds to MFMA step s. Must match
// the B byte -> k assignment of the panel layout.
template <int KIND> __device__ __forceinline__ int a_koff(int s, int g) {
    if constexpr (KIND == ORKH_I8) return g * 16;
    else if constexpr (KIND == ORKH_F16) return g * 8;
    else return g * 32 + s * 16;
}

struct Lut { uint32_t l0, l1, l2, l3; };

// 4 NF4 indices (one per byte, 0..15) -> 4 int8 codebook values.
__device__ __forceinline__ uint32_t nf4_map4(uint32_t idx, const Lut &L) {
    const uint32_t lo = __builtin_amdgcn_perm(L.l1, L.l0, idx);               // entries 0..7
    const uint32_t hi = __builtin_amdgcn_perm(L.l3, L.l2, idx & 0x07070707u); // entries 8..15
    const uint32_t m = (idx >> 3) & 0x01010101u;                              // bit 3 per byte
    const uint32_t sel = (m << 8) - m;                                        // 0xff where idx >= 8
    return (hi & sel) | (lo & ~sel);
}

// Raw 16-byte panel chunk -> STEPS MFMA B operands.
template <int KIND> __device__ __forceinline__ void decode(v4i raw, v4i *op, const Lut &L) {
    if constexpr (KIND == ORKH_I8 || KIND == ORKH_F16) {
        op[0] = raw;
    } else if constexpr (KIND == ORKH_I4U) {
        const uint32_t x0 = raw.x, x1 = raw.y, x2 = raw.z, x3 = raw.w;
        op[0] = v4i{(int)((x0 << 4) & 0xf0f0f0f0u), (int)(x0 & 0xf0f0f0f0u),
                    (int)((x1 << 4) & 0xf0f0f0f0u), (int)(x1 & 0xf0f0f0f0u)};
        op[1] = v4i{(int)((x2 << 4) & 0xf0f0f0f0u), (int)(x2 & 0xf0f0f0f0u),
                    (int)((x3 << 4) & 0xf0f0f0f0u), (int)(x3 & 0xf0f0f0f0u)};
    } else {
        const uint32_t x0 = raw.x, x1 = raw.y, x2 = raw.z, x3 = raw.w;
        op[0] = v4i{(int)nf4_map4(x0 & 0x0f0f0f0fu, L), (int)nf4_map4((x0 >> 4) & 0x0f0f0f0fu, L),
                    (int)nf4_map4(x1 & 0x0f0f0f0fu, L), (int)nf4_map4((x1 >> 4) & 0x0f0f0f0fu, L)};
        op[1] = v4i{(int)nf4_map4(x2 & 0x0f0f0f0fu, L), (int)nf4_map4((x2 >> 4) & 0x0f0f0f0fu, L),
                    (int)nf4_map4(x3 & 0x0f0f0f0fu, L), (int)nf4_map4((x3 >> 4) & 0x0f0f0f0fu, L)};
    }
}

__device__ __forceinline__ v4i mma(v4i a, v4i b, v4i c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ v4f mma(v4i a, v4i b, v4f c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, a), __builtin_bit_cast(v8h, b), c, 0, 0, 0);
}

template <int KIND> __device__ __forceinline__ typename KT<KIND>::c_t finish(typename KT<KIND>::c_t v) {
    if constexpr (KIND == ORKH_I4U) return v >> 4;  // exact: every partial is 16 * integer
    else return v;
}

// A chunk load: 16 bytes of row `row` starting at element k, or zero outside [0,M) x [0,K).
template <int KIND>
__device__ __forceinline__ v4i load_a(const char *A, int lda_bytes, int row, int k, int M, int K) {
    v4i a = {0, 0, 0, 0};
    if (row < M && k < K) a = *(const v4i *)(A + (size_t)row * lda_bytes + (size_t)k * KT<KIND>::ESZ);
    return a;
}

// ------------------------------------------------------------------------------------------------
// k_stream: grid (N/16, ksplit), WPG waves. Workgroup (nb, ks) owns panel nb and K-blocks
// [ks*kbs, ks*kbs+kbs); wave w takes kbw of them. KU blocks are loaded before any is consumed.
template <int KIND, int MT, int WPG, int KU>
__global__ __launch_bounds__(WPG * 64) void k_stream(orkh_mm p, int kbw, int kbs, int ksplit, void *ws) {
    using T = KT<KIND>;
    typedef typename T::acc_t acc_t;
    typedef typename T::c_t c_t;
    __shared__ c_t red[WPG][MT * 256];

    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int nb = blockIdx.x, ks = blockIdx.y;
    const int kb_hi = min(ks * kbs + kbs, p.KB);
    const int kb0 = ks * kbs + w * kbw;
    const int kb1 = min(kb0 + kbw, kb_hi);
    const int r16 = lane & 15, g = lane >> 4;
    const char *A = (const char *)p.A;
    const int lda_b = p.lda * T::ESZ;
    const Lut L = {p.lut[0], p.lut[1], p.lut[2], p.lut[3]};
    const v4i *bp = (const v4i *)p.B + (size_t)nb * p.KB * 64 + lane;

    acc_t acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) acc[mt] = acc_t{0, 0, 0, 0};

    auto consume = [&](v4i raw, int kb) {
        v4i op[T::STEPS];
        decode<KIND>(raw, op, L);
#pragma unroll
        for (int s = 0; s < T::STEPS; s++) {
            const int k = kb * T::KPB + a_koff<KIND>(s, g);
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
                acc[mt] = mma(load_a<KIND>(A, lda_b, mt * 16 + r16, k, p.M, p.K), op[s], acc[mt]);
        }
    };

    int kb = kb0;
    for (; kb + KU <= kb1; kb += KU) {
        v4i raw[KU];
#pragma unroll
        for (int u = 0; u < KU; u++) raw[u] = __builtin_nontemporal_load(bp + (size_t)(kb + u) * 64);
#pragma unroll
        for (int u = 0; u < KU; u++) consume(raw[u], kb + u);
    }
    for (; kb < kb1; kb++) consume(__builtin_nontemporal_load(bp + (size_t)kb * 64), kb);

#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int r = 0; r < 4; r++) red[w][mt * 256 + r * 64 + lane] = acc[mt][r];
    __syncthreads();

    c_t *C = (c_t *)p.C;
    c_t *W = (c_t *)ws;
    for (int e = threadIdx.x; e < MT * 256; e += WPG * 64) {
        c_t s = red[0][e];
#pragma unroll
        for (int ww = 1; ww < WPG; ww++) s += red[ww][e];
        const int mt = e >> 8, r = (e >> 6) & 3, ln = e & 63;
        const int m = mt * 16 + (ln >> 4) * 4 + r;
        const int n = nb * 16 + (ln & 15);
        if (m < p.M) {
            if (ksplit == 1) C[(size_t)m * p.ldc + n] = finish<KIND>(s);
            else W[((size_t)ks * p.M + m) * p.N + n] = finish<KIND>(s);
        }
    }
}

// Fixed-order sum of split-K partials (deterministic for fp32 as well as exact for int32).
template <typename c_t>
__global__ __launch_bounds__(256) void k_splitk_reduce(const c_t *ws, c_t *C, int M, int N, int ldc, int ksplit) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t MN = (size_t)M * N;
    if (i >= MN) return;
    c_t s = ws[i];
    for (int k = 1; k < ksplit; k++) s += ws[(size_t)k * MN + i];
    C[(i / N) * ldc + (i % N)] = s;
}

// ------------------------------------------------------------------------------------------------
// k_tiled: one 256-thread workgroup (2 x 2 waves) per BM x BN tile, KS panel K-blocks per LDS stage.
template <int KIND, int BM, int BN, int KS>
__global__ __launch_bounds__(256) void k_tiled(orkh_mm p, int mtiles) {
    using T = KT<KIND>;
    typedef typename T::acc_t acc_t;
    constexpr int MB = BM / 16, NBK = BN / 16;
    constexpr int MTW = MB / 2, NTW = NBK / 2;
    constexpr int AF = MB * KS * T::STEPS;  // A fragments (1 KiB) per stage
    constexpr int BF = NBK * KS;            // B blocks (1 KiB) per stage
    constexpr int AV = (AF * 64 + 255) / 256, BV = (BF * 64 + 255) / 256;
    static_assert(MB % 2 == 0 && NBK % 2 == 0, "tile must split over 2x2 waves");
    __shared__ v4i lds[2][(AF + BF) * 64];

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int wm = wv & 1, wn = wv >> 1;
    // XCD-aware order: WG b runs on XCD b%8; give each XCD a contiguous run of tiles, M fastest, so
    // every M-tile that reads a given B column panel shares one L2.
    const int nT = gridDim.x, bid = blockIdx.x;
    const int per = nT / 8, rem = nT % 8, x = bid % 8, j = bid / 8;
    const int tile = (x < rem) ? x * (per + 1) + j : rem * (per + 1) + (x - rem) * per + j;
    const int m0 = (tile % mtiles) * BM;
    const int nb0 = (tile / mtiles) * NBK;
    const int NBtot = p.N / 16;

    const char *A = (const char *)p.A;
    const int lda_b = p.lda * T::ESZ;
    const v4i *Bp = (const v4i *)p.B;
    const Lut L = {p.lut[0], p.lut[1], p.lut[2], p.lut[3]};

    v4i ra[AV], rb[BV];
    auto gload = [&](int st) {
#pragma unroll
        for (int i = 0; i < AV; i++) {
            const int idx = i * 256 + tid;
            ra[i] = v4i{0, 0, 0, 0};
            if (idx < AF * 64) {
                const int f = idx >> 6, ln = idx & 63;
                const int mb = f / (KS * T::STEPS), ksub = f % (KS * T::STEPS);
                const int kbl = ksub / T::STEPS, s = ksub % T::STEPS;
                const int row = m0 + mb * 16 + (ln & 15);
                const int k = (st * KS + kbl) * T::KPB + a_koff<KIND>(s, ln >> 4);
                ra[i] = load_a<KIND>(A, lda_b, row, k, p.M, p.K);
            }
        }
#pragma unroll
        for (int i = 0; i < BV; i++) {
            const int idx = i * 256 + tid;
            rb[i] = v4i{0, 0, 0, 0};
            if (idx < BF * 64) {
                const int b = idx >> 6, ln = idx & 63;
                const int nb = nb0 + b / KS, kb = st * KS + b % KS;
                if (nb < NBtot && kb < p.KB) rb[i] = Bp[((size_t)nb * p.KB + kb) * 64 + ln];
            }
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < AV; i++) {
            const int idx = i * 256 + tid;
            if (idx < AF * 64) lds[buf][idx] = ra[i];
        }
#pragma unroll
        for (int i = 0; i < BV; i++) {
            const int idx = i * 256 + tid;
            if (idx < BF * 64) lds[buf][AF * 64 + idx] = rb[i];
        }
    };

    acc_t acc[MTW][NTW];
#pragma unroll
    for (int i = 0; i < MTW; i++)
#pragma unroll
        for (int jn = 0; jn < NTW; jn++) acc[i][jn] = acc_t{0, 0, 0, 0};

    const int nst = (p.KB + KS - 1) / KS;
    gload(0);
    lstore(0);
    __syncthreads();
    for (int st = 0; st < nst; st++) {
        const int cur = st & 1;
        if (st + 1 < nst) gload(st + 1);
#pragma unroll
        for (int kbl = 0; kbl < KS; kbl++) {
            v4i op[NTW][T::STEPS];
#pragma unroll
            for (int jn = 0; jn < NTW; jn++)
                decode<KIND>(lds[cur][AF * 64 + ((wn * NTW + jn) * KS + kbl) * 64 + lane], op[jn], L);
#pragma unroll
            for (int s = 0; s < T::STEPS; s++) {
#pragma unroll
                for (int i = 0; i < MTW; i++) {
                    const v4i a = lds[cur][(((wm * MTW + i) * KS + kbl) * T::STEPS + s) * 64 + lane];
#pragma unroll
                    for (int jn = 0; jn < NTW; jn++) acc[i][jn] = mma(a, op[jn][s], acc[i][jn]);
                }
            }
        }
        if (st + 1 < nst) lstore(cur ^ 1);
        __syncthreads();
    }

    typedef typename T::c_t c_t;
    c_t *C = (c_t *)p.C;
#pragma unroll
    for (int i = 0; i < MTW; i++)
#pragma unroll
        for (int jn = 0; jn < NTW; jn++) {
            const int nbk = nb0 + wn * NTW + jn;
            if (nbk >= NBtot) continue;
            const int n = nbk * 16 + (lane & 15);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = m0 + (wm * MTW + i) * 16 + (lane >> 4) * 4 + r;
                if (m < p.M) C[(size_t)m * p.ldc + n] = finish<KIND>(acc[i][jn][r]);
            }
        }
}

// ------------------------------------------------------------------------------------------------
thread_local char g_lerr[256];

template <int KIND, int MT, int WPG>
int launch_stream_v(const orkh_mm *p, const orkh_plan *q, hipStream_t s) {
    constexpr int KU = (KIND == ORKH_I4U || KIND == ORKH_NF4) ? 4 : 8;
    dim3 grid(p->N / 16, q->ksplit), block(WPG * 64);
    hipLaunchKernelGGL((k_stream<KIND, MT, WPG, KU>), grid, block, 0, s, *p, q->kbw, q->kbs, q->ksplit, q->ws);
    return 0;
}

template <int KIND, int MT>
int launch_stream_w(const orkh_mm *p, const orkh_plan *q, hipStream_t s) {
    if (q->wpg == 8) return launch_stream_v<KIND, MT, 8>(p, q, s);
    return launch_stream_v<KIND, MT, 4>(p, q, s);
}

template <int KIND>
int launch_stream(const orkh_mm *p, const orkh_plan *q, hipStream_t s) {
    switch (q->mt) {
    case 1: return launch_stream_w<KIND, 1>(p, q, s);
    case 2: return launch_stream_w<KIND, 2>(p, q, s);
    case 3: return launch_stream_w<KIND, 3>(p, q, s);
    case 4: return launch_stream_w<KIND, 4>(p, q, s);
    }
    snprintf(g_lerr, sizeof g_lerr, "stream plan: mt=%d unsupported", q->mt);
    return -2;
}

template <int KIND, int BM, int BN>
int launch_tiled_v(const orkh_mm *p, hipStream_t s) {
    constexpr int KS = (KIND == ORKH_I4U || KIND == ORKH_NF4) ? 1 : 2;
    const int mtiles = (p->M + BM - 1) / BM;
    const int ntiles = (p->N / 16 + BN / 16 - 1) / (BN / 16);
    hipLaunchKernelGGL((k_tiled<KIND, BM, BN, KS>), dim3(mtiles * ntiles), dim3(256), 0, s, *p, mtiles);
    return 0;
}

template <int KIND>
int launch_tiled(const orkh_mm *p, const orkh_plan *q, hipStream_t s) {
    if (q->bm == 128 && q->bn == 96) return launch_tiled_v<KIND, 128, 96>(p, s);
    if (q->bm == 128 && q->bn == 128) return launch_tiled_v<KIND, 128, 128>(p, s);
    if (q->bm == 64 && q->bn == 64) return launch_tiled_v<KIND, 64, 64>(p, s);
    snprintf(g_lerr, sizeof g_lerr, "tiled plan: %dx%d unsupported", q->bm, q->bn);
    return -2;
}

}  // namespace

extern "C" int orkh_mm_launch(const orkh_mm *p, const orkh_plan *q, void *stream) {
    hipStream_t s = (hipStream_t)stream;
    int rc;
    if (q->algo == ORKH_ALGO_STREAM) {
        switch (p->kind) {
        case ORKH_I8: rc = launch_stream<ORKH_I8>(p, q, s); break;
        case ORKH_I4U: rc = launch_stream<ORKH_I4U>(p, q, s); break;
        case ORKH_NF4: rc = launch_stream<ORKH_NF4>(p, q, s); break;
        case ORKH_F16: rc = launch_stream<ORKH_F16>(p, q, s); break;
        default: rc = -2;
        }
        if (rc == 0 && q->ksplit > 1) {
            const size_t MN = (size_t)p->M * p->N;
            dim3 grid((unsigned)((MN + 255) / 256)), block(256);
            if (p->kind == ORKH_F16)
                hipLaunchKernelGGL(k_splitk_reduce<float>, grid, block, 0, s, (const float *)q->ws, (float *)p->C,
                                   p->M, p->N, p->ldc, q->ksplit);
            else
                hipLaunchKernelGGL(k_splitk_reduce<int32_t>, grid, block, 0, s, (const int32_t *)q->ws,
                                   (int32_t *)p->C, p->M, p->N, p->ldc, q->ksplit);
        }
    } else {
        switch (p->kind) {
        case ORKH_I8: rc = launch_tiled<ORKH_I8>(p, q, s); break;
        case ORKH_I4U: rc = launch_tiled<ORKH_I4U>(p, q, s); break;
        case ORKH_NF4: rc = launch_tiled<ORKH_NF4>(p, q, s); break;
        case ORKH_F16: rc = launch_tiled<ORKH_F16>(p, q, s); break;
        default: rc = -2;
        }
    }
    if (rc) return rc;
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        snprintf(g_lerr, sizeof g_lerr, "launch: %s", hipGetErrorString(e));
        return -1;
    }
    return 0;
}

extern "C" const char *orkh_mm_variant(const orkh_mm *p, const orkh_plan *q) {
    static thread_local char b[96];
    static const char *kn[] = {"i8", "i4u", "nf4", "f16"};
    const char *k = (p->kind >= 0 && p->kind <= 3) ? kn[p->kind] : "?";
    if (q->algo == ORKH_ALGO_STREAM)
        snprintf(b, sizeof b, "stream_%s_mt%d_w%d_kbw%d_ks%d", k, q->mt, q->wpg, q->kbw, q->ksplit);
    else
        snprintf(b, sizeof b, "tiled_%s_%dx%d", k, q->bm, q->bn);
    return b;
}
