// orkh_kernels.hip -- gfx950 (MI355X, CDNA4) matmul kernels on resident panels, and their C-ABI launcher.
//
// These replace the reference's device programs for the matmul path: the int8 / fp16 / int4 regcmd
// synthesizers (src/npu/i8/regcmd.c:32-62, src/npu/f16/regcmd.c:303, src/npu/i4/run.c:97-124) and the
// host-side K-slice accumulation around them (src/npu.c:1764-1821). Panel layout: orkh.h.
//
// Three algorithms, all wave64:
//   k_gemv    M = 1 (decode): the k_stream data flow with the MFMA replaced by VALU dot products
//             (v_dot4_i32_i8 / v_dot2_f32_f16). Each lane's activation chunk arrives by a DPP row
//             broadcast of one dword per lane, and the four K-groups of a column fold with
//             v_permlane32/16_swap. Measured on MI355X at K=2048, N=6144 int8: 3.83 us against
//             4.08 us for the same flow on MFMA (the MFMA issue itself adds ~0.4 us per launch).
//             k_gemv_half, the planner's default, gives each workgroup half a panel (8 columns) so
//             that the bytes spread evenly over the CUs.
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
#include <string.h>

#include <atomic>
#include <type_traits>

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

// One dword of NF4 codes (8 nibbles) -> the int8 codebook values of its low nibbles (lo) and of its high
// nibbles (hi), byte for byte. Both 8-entry halves of the codebook are looked up with the code's low 3 bits
// (v_perm: selector bytes 0-3 pick from its second operand, 4-7 from its first), then a third v_perm takes
// byte j from the upper half where bit 3 of code j is set: its selector byte is j + 4 * bit3. Six VALU
// operations per four codes (the select mask built from bit 3 by shift-and-subtract took eight).
__device__ __forceinline__ void nf4_map8(uint32_t x, const Lut &L, uint32_t &lo, uint32_t &hi) {
    const uint32_t i0 = x & 0x07070707u, i1 = (x >> 4) & 0x07070707u;
    const uint32_t s0 = ((x >> 1) & 0x04040404u) | 0x03020100u; // bit 3 of each low nibble -> byte select
    const uint32_t s1 = ((x >> 5) & 0x04040404u) | 0x03020100u; // bit 7 (bit 3 of the high nibble)
    lo = __builtin_amdgcn_perm(__builtin_amdgcn_perm(L.l3, L.l2, i0), __builtin_amdgcn_perm(L.l1, L.l0, i0), s0);
    hi = __builtin_amdgcn_perm(__builtin_amdgcn_perm(L.l3, L.l2, i1), __builtin_amdgcn_perm(L.l1, L.l0, i1), s1);
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
        uint32_t a0, b0, a1, b1, a2, b2, a3, b3;
        nf4_map8((uint32_t)raw.x, L, a0, b0);
        nf4_map8((uint32_t)raw.y, L, a1, b1);
        nf4_map8((uint32_t)raw.z, L, a2, b2);
        nf4_map8((uint32_t)raw.w, L, a3, b3);
        op[0] = v4i{(int)a0, (int)b0, (int)a1, (int)b1};
        op[1] = v4i{(int)a2, (int)b2, (int)a3, (int)b3};
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

// ------------------------------------------------------------------------------------------------
// Raw buffer loads: the hardware returns 0 for any byte offset >= num_records, so out-of-range rows,
// K tails and stages past the end cost no clamping or select instructions, and can never fault.
typedef unsigned v4u __attribute__((ext_vector_type(4)));
constexpr uint32_t OOB = 0x80000000u;  // an offset past every buffer this path addresses (< 2 GiB)
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ v4i bload(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return (v4i)__builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}

// Write-through vector stores at device scope (global_store_* ... sc1): the L2 passes the data on to memory as it
// comes instead of holding it dirty until the end of the kernel. Written as asm because the compiler merges a store
// that carries a cache-policy modifier with an otherwise identical plain store on the other side of a branch, and
// drops the modifier.
__device__ __forceinline__ void store_wt(int *p, int v) {
    asm volatile("global_store_dword %0, %1, off sc1" ::"v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void store_wt(float *p, float v) {
    asm volatile("global_store_dword %0, %1, off sc1" ::"v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void store_wt4(void *p, v4i v) {
    asm volatile("global_store_dwordx4 %0, %1, off sc1" ::"v"(p), "v"(v) : "memory");
}
// ------------------------------------------------------------------------------------------------
// k_stream: grid (N/16, ksplit), WPG waves. Workgroup (nb, ks) owns panel nb and K-blocks
// [ks*kbs, ks*kbs+kbs); wave w takes kbw of them. KU blocks are loaded before any is consumed.
// NP = 2 (paired panels): grid (G, 1) with N/16 / 2 <= G < N/16; the first N/16 - G workgroups own two
// adjacent panels each and the rest one, so every CU holds about the same bytes; a wave loads each A chunk
// once for both of its panels.
// HF = 1 (half panels): grid (N/8, ksplit); workgroup x owns columns 8 (x % 2) .. 8 (x % 2) + 7 of panel x / 2:
// only the lanes holding those columns load B (half of every block's lines), and only they store. The MFMA still
// runs on 16 columns; the other 8 (their B lanes left zero, or NF4's code 0) are discarded.
template <int KIND, int MT, int WPG, int KU, int NP = 1, int HF = 0>
__global__ __launch_bounds__(WPG * 64) void k_stream(orkh_mm p, int kbw, int kbs, int ksplit, void *ws) {
    static_assert(!(HF && NP == 2), "half panels are single panels");
    using T = KT<KIND>;
    typedef typename T::acc_t acc_t;
    typedef typename T::c_t c_t;
    __shared__ c_t red[WPG][NP][MT * 256];

    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int ks = blockIdx.y, NBtot = p.N / 16;
    const int two = NP == 2 ? NBtot - (int)gridDim.x : 0;   // workgroups that own two panels
    const int nb = HF ? (int)blockIdx.x >> 1
                      : NP == 2 ? ((int)blockIdx.x < two ? 2 * (int)blockIdx.x : two + (int)blockIdx.x) : (int)blockIdx.x;
    const int np = NP == 2 && (int)blockIdx.x < two ? 2 : 1;
    const int hh = HF ? (int)blockIdx.x & 1 : 0;             // half panels: which 8 columns
    const bool bcol = !HF || ((threadIdx.x >> 3) & 1) == hh; // this lane's column (lane % 16) is one of them
    const int kb_hi = min(ks * kbs + kbs, p.KB);
    const int kb0 = ks * kbs + w * kbw;
    const int kb1 = min(kb0 + kbw, kb_hi);
    const int r16 = lane & 15, g = lane >> 4;
    const char *A = (const char *)p.A;
    const int lda_b = p.lda * T::ESZ;
    const Lut L = {p.lut[0], p.lut[1], p.lut[2], p.lut[3]};
    const v4i *bp = (const v4i *)p.B + (size_t)nb * p.KB * 64 + lane;
    const size_t pstride = (size_t)p.KB * 64; // the second panel's blocks (paired workgroups only)

    acc_t acc[NP][MT];
#pragma unroll
    for (int pi = 0; pi < NP; pi++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++) acc[pi][mt] = acc_t{0, 0, 0, 0};

    // One batch of U blocks: every A chunk (L2-resident, short latency) is requested first, then every
    // B block (HBM), and only then is anything consumed, so the wave has all its loads in flight at once.
    // A loads are unconditional from a clamped, always-valid address (row 0, k 0) and the chunks outside
    // [0,M) x [0,K) are zeroed where they are consumed: a select right after the load would make the
    // wave wait for it, and buffer loads measured slower on this path.
    auto batch = [&](int kb, auto U_) {
        constexpr int U = decltype(U_)::value;
        v4i av[U][T::STEPS][MT];
#pragma unroll
        for (int u = 0; u < U; u++)
#pragma unroll
            for (int s = 0; s < T::STEPS; s++)
#pragma unroll
                for (int mt = 0; mt < MT; mt++) {
                    const int row = mt * 16 + r16, k = (kb + u) * T::KPB + a_koff<KIND>(s, g);
                    const bool ok = row < p.M && k < p.K;
                    av[u][s][mt] = *(const v4i *)(A + (size_t)(ok ? row : 0) * lda_b + (size_t)(ok ? k : 0) * T::ESZ);
                }
        v4i raw[NP][U];
#pragma unroll
        for (int pi = 0; pi < NP; pi++)
            if (pi == 0 || np == 2) // workgroup-uniform
#pragma unroll
                for (int u = 0; u < U; u++)
                    raw[pi][u] = bcol ? __builtin_nontemporal_load(bp + pi * pstride + (size_t)(kb + u) * 64) : v4i{0, 0, 0, 0};
#pragma unroll
        for (int u = 0; u < U; u++) {
#pragma unroll
            for (int pi = 0; pi < NP; pi++) {
                if (pi == 1 && np == 1) continue;
                v4i op[T::STEPS];
                decode<KIND>(raw[pi][u], op, L);
#pragma unroll
                for (int s = 0; s < T::STEPS; s++)
#pragma unroll
                    for (int mt = 0; mt < MT; mt++) {
                        const int row = mt * 16 + r16, k = (kb + u) * T::KPB + a_koff<KIND>(s, g);
                        const v4i a = (row < p.M && k < p.K) ? av[u][s][mt] : v4i{0, 0, 0, 0};
                        acc[pi][mt] = mma(a, op[s], acc[pi][mt]);
                    }
            }
        }
    };

    int kb = kb0;
    for (; kb + KU <= kb1; kb += KU) batch(kb, std::integral_constant<int, KU>{});
    if constexpr (KU > 4)
        if (kb + 4 <= kb1) { batch(kb, std::integral_constant<int, 4>{}); kb += 4; }
    for (; kb < kb1; kb++) batch(kb, std::integral_constant<int, 1>{});

#pragma unroll
    for (int pi = 0; pi < NP; pi++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int r = 0; r < 4; r++) red[w][pi][mt * 256 + r * 64 + lane] = acc[pi][mt][r];
    __syncthreads();

    c_t *C = (c_t *)p.C;
    c_t *W = (c_t *)ws;
    for (int e = threadIdx.x; e < np * MT * 256; e += WPG * 64) {
        const int pi = e / (MT * 256), el = e - pi * (MT * 256);
        c_t s = red[0][pi][el];
#pragma unroll
        for (int ww = 1; ww < WPG; ww++) s += red[ww][pi][el];
        const int mt = el >> 8, r = (el >> 6) & 3, ln = el & 63;
        const int m = mt * 16 + (ln >> 4) * 4 + r;
        const int n = (nb + pi) * 16 + (ln & 15);
        if (m < p.M && (!HF || ((ln >> 3) & 1) == hh)) {
            if (ksplit == 1) C[(size_t)m * p.ldc + n] = finish<KIND>(s);
            else W[((size_t)ks * p.M + m) * p.N + n] = finish<KIND>(s);
        }
    }
}

// ------------------------------------------------------------------------------------------------
// k_gemv: M = 1. Grid (N/16, ksplit), WPG waves; workgroup (nb, ks) owns panel nb and K-blocks
// [ks*kbs, ks*kbs+kbs), wave w a run of kbw of them, loaded KU at a time (all activation dwords, then
// all panel blocks, then the dot products). Lane (g, i) of a wave needs, per block, the W activation
// dwords of K-group g; one dword load per lane fetches them for BPL = 16/W blocks at once (lane i of
// row g takes dword i%W of block i/W), and v_mov_dpp row_newbcast hands dword d of block b to the
// whole row. Dwords past K or past the wave's run are loaded from a clamped address and zeroed before
// the broadcast (K % 32 == 0, so a dword never straddles K).
template <int I, int N, typename F> __device__ __forceinline__ void static_for(F &&f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<I + 1, N>(f);
    }
}
template <int LANE> __device__ __forceinline__ int row_bcast(int x) {
    return __builtin_amdgcn_update_dpp(0, x, 0x150 + LANE, 0xF, 0xF, false);  // row_newbcast:LANE
}
typedef _Float16 v2h __attribute__((ext_vector_type(2)));

// One panel (nb) x one K range (ks) of a GEMV: the body shared by k_gemv and k_gemv_group.
template <int KIND, int WPG, int KU>
__device__ __forceinline__ void gemv_panel(const orkh_mm &p, int nb, int ks, int kbw, int kbs, int ksplit, void *ws,
                                           typename KT<KIND>::c_t (*red)[16]) {
    using T = KT<KIND>;
    typedef typename T::c_t c_t;
    constexpr int W = (KIND == ORKH_I4U || KIND == ORKH_NF4) ? 8 : 4;  // activation dwords per group per block
    constexpr int BPL = 16 / W;                                         // blocks per activation load
    constexpr int KPBB = T::KPB * T::ESZ;                               // activation bytes per block
    static_assert(KU % BPL == 0, "a full batch must cover whole activation loads");

    // the wave index is wave-uniform: keep it (and every bound derived from it) in SGPRs
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), g = lane >> 4, i = lane & 15;
    const int kb_hi = min(ks * kbs + kbs, p.KB);
    const int kb0 = ks * kbs + w * kbw;
    const int kb1 = min(kb0 + kbw, kb_hi);
    const char *A = (const char *)p.A;
    const Lut L = {p.lut[0], p.lut[1], p.lut[2], p.lut[3]};
    const v4i *bp = (const v4i *)p.B + (size_t)nb * p.KB * 64 + lane;
    c_t acc = 0;

    auto batch = [&](int kb, auto U_) {
        constexpr int U = decltype(U_)::value;
        constexpr int NQ = (U + BPL - 1) / BPL;
        int ad[NQ];
        bool ok[NQ];
#pragma unroll
        for (int q = 0; q < NQ; q++) {
            const int blk = kb + q * BPL + i / W;
            const int byte = blk * KPBB + g * (W * 4) + (i % W) * 4;
            ok[q] = blk < kb1 && byte / T::ESZ < p.K;
            ad[q] = *(const int *)(A + (ok[q] ? byte : 0));
        }
        v4i raw[U];
#pragma unroll
        for (int u = 0; u < U; u++) raw[u] = __builtin_nontemporal_load(bp + (size_t)(kb + u) * 64);
        int src[NQ];
#pragma unroll
        for (int q = 0; q < NQ; q++) src[q] = ok[q] ? ad[q] : 0;
        static_for<0, U>([&](auto uc) {
            constexpr int u = decltype(uc)::value;
            v4i op[T::STEPS];
            decode<KIND>(raw[u], op, L);
            static_for<0, W>([&](auto dc) {
                constexpr int d = decltype(dc)::value;
                const int a = row_bcast<(u % BPL) * W + d>(src[u / BPL]);
                const int b = op[d / 4][d % 4];
                if constexpr (KIND == ORKH_F16)
                    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(v2h, a), __builtin_bit_cast(v2h, b), acc, false);
                else
                    acc = __builtin_amdgcn_sdot4(a, b, acc, false);
            });
        });
    };

    int kb = kb0;
    for (; kb + KU <= kb1; kb += KU) batch(kb, std::integral_constant<int, KU>{});
    if constexpr (KU > BPL)
        for (; kb + BPL <= kb1; kb += BPL) batch(kb, std::integral_constant<int, BPL>{});
    for (; kb < kb1; kb++) batch(kb, std::integral_constant<int, 1>{});

    // Fold the four K-groups of each column: lanes l <-> l^32, then l <-> l^16.
    if constexpr (KIND == ORKH_F16) {
        const auto s32 = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(int, acc), __builtin_bit_cast(int, acc), false, false);
        acc += __builtin_bit_cast(float, (int)(lane < 32 ? s32[1] : s32[0]));
        const auto s16 = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(int, acc), __builtin_bit_cast(int, acc), false, false);
        acc += __builtin_bit_cast(float, (int)((lane & 16) == 0 ? s16[1] : s16[0]));
    } else {
        const auto s32 = __builtin_amdgcn_permlane32_swap(acc, acc, false, false);
        acc += (int)(lane < 32 ? s32[1] : s32[0]);
        const auto s16 = __builtin_amdgcn_permlane16_swap(acc, acc, false, false);
        acc += (int)((lane & 16) == 0 ? s16[1] : s16[0]);
    }
    if (lane < 16) red[w][lane] = acc;
    __syncthreads();
    if (threadIdx.x < 16) {
        c_t s = red[0][threadIdx.x];
#pragma unroll
        for (int ww = 1; ww < WPG; ww++) s += red[ww][threadIdx.x];
        const int n = nb * 16 + threadIdx.x;
        if (ksplit == 1) ((c_t *)p.C)[n] = finish<KIND>(s);
        else ((c_t *)ws)[(size_t)ks * p.N + n] = finish<KIND>(s);
    }
}

template <int KIND, int WPG, int KU>
__global__ __launch_bounds__(WPG * 64) void k_gemv(orkh_mm p, int kbw, int kbs, int ksplit, void *ws) {
    __shared__ typename KT<KIND>::c_t red[WPG][16];
    gemv_panel<KIND, WPG, KU>(p, blockIdx.x, blockIdx.y, kbw, kbs, ksplit, ws, red);
}

// k_gemv_half: M = 1 with half a panel per workgroup. Grid (N/8, ksplit), WPG waves; workgroup (b, ks) owns
// columns 8h .. 8h+7 (h = b % 2) of panel b / 2 over K-blocks [ks*kbs, ks*kbs+kbs), wave w a run of kbw of them.
// Whole panels put two panels on some CUs and one on others whenever N/16 is not a multiple of the CU count
// (N = 6144: 384 panels on 256 CUs); halves spread the bytes three to a CU there, and fill twice the CUs where
// there are fewer panels than CUs. In a 1 KiB block, column c's k-group g is the 16 bytes at (16 g + c) * 16, so
// a half is four whole 128-byte lines, and one load instruction fetches the halves of two blocks: lane l takes
// block kb + l/32, k-group (l/8) % 4, column 8h + l%8. A wave issues all NI instructions of its run at once (the
// launcher picks NI = ceil(kbw / 2) where it is instantiated, so only an odd run's last half re-reads a block;
// runs past 16 blocks go in batches of 8 instructions), then each lane
// loads its k-group's activation bytes (16, or 32 for the nibble kinds: the same few addresses across lanes,
// served by the L1) and accumulates with v_dot4 / v_dot2. The eight lanes of a column (block l/32, k-group
// (l/8)%4) fold with permlane32 / permlane16 swaps and a row rotation by 8; the waves reduce through LDS.
template <int KIND, int WPG, int NI>
__global__ __launch_bounds__(WPG * 64) void k_gemv_half(orkh_mm p, int kbw, int kbs, int ksplit, void *ws) {
    using T = KT<KIND>;
    typedef typename T::c_t c_t;
    constexpr int W = (KIND == ORKH_I4U || KIND == ORKH_NF4) ? 8 : 4;  // activation dwords per k-group per block
    constexpr int KPBB = T::KPB * T::ESZ;                               // activation bytes per block
    __shared__ c_t red[WPG][8];
    // the kernel arguments in one batch of scalar loads behind one wait (the compiler put the activation pointer's
    // load in a second batch, waited on before the first weight load): int8 K=2048 N=6144 3.78 -> 3.75-3.76 us
    asm volatile("" ::"s"(p.K), "s"(p.KB), "s"(p.A), "s"(p.B), "s"(p.C), "s"(kbw), "s"(kbs), "s"(ksplit));
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nb = blockIdx.x >> 1, h = blockIdx.x & 1, ks = blockIdx.y;
    const int kb_hi = min(ks * kbs + kbs, p.KB);
    const int kb0 = ks * kbs + w * kbw, kb1 = min(kb0 + kbw, kb_hi);
    const int g = (lane >> 3) & 3, sub = lane >> 5;
    const v4i *bp = (const v4i *)p.B + (size_t)nb * p.KB * 64 + g * 16 + h * 8 + (lane & 7);
    const char *A = (const char *)p.A;
    const Lut L = {p.lut[0], p.lut[1], p.lut[2], p.lut[3]};
    c_t acc = 0;
    for (int kb = kb0; kb < kb1; kb += 2 * NI) {
        v4i raw[NI], act[NI][W / 4];
        bool ok[NI];
#pragma unroll
        for (int q = 0; q < NI; q++)  // past the run's end: its last block again (no branches), with activations 0
            raw[q] = __builtin_nontemporal_load(bp + (size_t)min(kb + 2 * q + sub, kb1 - 1) * 64);
#pragma unroll
        for (int q = 0; q < NI; q++) {
            const int blk = kb + 2 * q + sub, byte = blk * KPBB + g * (W * 4);
            ok[q] = blk < kb1 && byte / T::ESZ < p.K;
#pragma unroll
            for (int j = 0; j < W / 4; j++) act[q][j] = *(const v4i *)(A + (ok[q] ? byte + 16 * j : 0));
        }
#pragma unroll
        for (int q = 0; q < NI; q++) {
            v4i op[T::STEPS];
            decode<KIND>(raw[q], op, L);
#pragma unroll
            for (int d = 0; d < W; d++) {
                const int a = ok[q] ? act[q][d / 4][d % 4] : 0;
                const int b = op[d / 4][d % 4];
                if constexpr (KIND == ORKH_F16)
                    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(v2h, a), __builtin_bit_cast(v2h, b), acc, false);
                else
                    acc = __builtin_amdgcn_sdot4(a, b, acc, false);
            }
        }
    }
    // the column's eight lanes: l ^ 32, l ^ 16, then l ^ 8 (row_ror:8 within each 16-lane row)
    {
        int x = __builtin_bit_cast(int, acc);
        const auto s32 = __builtin_amdgcn_permlane32_swap(x, x, false, false);
        acc += __builtin_bit_cast(c_t, (int)(lane < 32 ? s32[1] : s32[0]));
        x = __builtin_bit_cast(int, acc);
        const auto s16 = __builtin_amdgcn_permlane16_swap(x, x, false, false);
        acc += __builtin_bit_cast(c_t, (int)((lane & 16) == 0 ? s16[1] : s16[0]));
        x = __builtin_bit_cast(int, acc);
        acc += __builtin_bit_cast(c_t, __builtin_amdgcn_update_dpp(0, x, 0x128, 0xF, 0xF, false));
    }
    if (lane < 8) red[w][lane] = acc;
    __syncthreads();
    if (threadIdx.x < 8) {
        c_t s = red[0][threadIdx.x];
#pragma unroll
        for (int ww = 1; ww < WPG; ww++) s += red[ww][threadIdx.x];
        const int n = nb * 16 + h * 8 + threadIdx.x;
        // C stored write-through: the row is not left dirty in L2 for the end of the kernel. Graph-timed against plain
        // stores, three alternations on one box: int8 K=2048 N=6144 3.82 -> 3.77 us, W4A8 NF4 3.29 -> 3.23, uniform
        // 3.14 -> 3.11, fp16 K=N=2048 unchanged (the streaming kernel's M=16 rows measured 1.2% slower so, the grouped
        // GEMVs of a chain up to 1.3%: both keep plain stores)
        if (ksplit == 1) store_wt(&((c_t *)p.C)[n], finish<KIND>(s));
        else ((c_t *)ws)[(size_t)ks * p.N + n] = finish<KIND>(s);
    }
}

// k_gemv_group: up to ORKH_GROUP_MAX independent M = 1 GEMVs of one kind in a single launch (the
// multi-matmul submit). Task t owns workgroups [t.wg0, t.wg0 + N/16), one panel each, whole K.
template <int KIND, int WPG, int KU>
__global__ __launch_bounds__(WPG * 64) void k_gemv_group(orkh_group g) {
    __shared__ typename KT<KIND>::c_t red[WPG][16];
    int t = g.n - 1;
    while (t > 0 && (int)blockIdx.x < g.t[t].wg0) t--;
    const orkh_gtask &tk = g.t[t];
    gemv_panel<KIND, WPG, KU>(tk.p, (int)blockIdx.x - tk.wg0, 0, tk.kbw, tk.p.KB, 1, nullptr, red);
}

// Fixed-order sum of split-K partials (deterministic for fp32 as well as exact for int32). A separate
// launch on purpose: combining the partials inside k_stream (last-arriving workgroup reduces) needs a
// device-scope release/acquire per workgroup, which on gfx950 is an L2 write-back + invalidate
// (buffer_wbl2 sc1 / buffer_inv sc1) and measured 34-120 us per launch for a 4 us GEMV; a second
// launch costs ~2 us.
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
// Grouped runs (per-(row, K-group) activation scales and per-(K-group, column) weight scales): the scales
// cannot be factored out of the K sum, so each K-group's int32 partial is produced exactly, scaled, and the
// scaled terms are summed in ascending group order -- the float sequence of the reference's grouped
// accumulate (src/npu/core/buf.c:501-520): c = 0; c = c + ((float)P_g * aS[m][g]) * bS[g][n], no fused
// multiply-adds.
// k_grouped_gemv: grouped scales at M = 1 on half panels (k_gemv_half's data flow): grid N/8, WPG waves, wave w a
// run of kbw K-blocks loaded NI instructions (two half blocks each) at a time. A lane's 16 (int8) or 32 (nibble
// kinds) k lie in one K-group (G % 32 == 0), so each dot product is added exactly, as int32, into that group's and
// column's partial in LDS (order-free). Then every thread forms some of the scaled terms ((float)P_g * aS[g]) *
// bS[g][n], their scales loaded at the start, and 8 threads add them in ascending g: k_grouped's operations in its
// order (src/npu/core/buf.c:501-520), so the results are bit-identical.
#define ORKH_GGEMV_SK_MAX 512
template <int KIND, int WPG, int NI>
__global__ __launch_bounds__(WPG * 64) void k_grouped_gemv(orkh_mm p, int G, const float *aS, const float *bS, float *C,
                                                          int kbw) {
#pragma clang fp contract(off)
    using T = KT<KIND>;
    constexpr int W = (KIND == ORKH_I4U || KIND == ORKH_NF4) ? 8 : 4; // activation dwords per k-group per block
    constexpr int NT = WPG * 64, SPT = ORKH_GGEMV_SK_MAX * 8 / NT;    // scaled terms per thread, at most
    __shared__ int P[ORKH_GGEMV_SK_MAX * 8];                           // [group][column]: int32 partials, then terms
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nb = blockIdx.x >> 1, h = blockIdx.x & 1, n0 = nb * 16 + h * 8;
    const int Sk = p.K / G, nterm = Sk * 8;
    // this thread's terms' scales, requested first (term e = group e / 8, column e % 8)
    float sa[SPT], sb[SPT];
#pragma unroll
    for (int q = 0; q < SPT; q++) {
        if (q * NT >= nterm) break; // workgroup-uniform: only the rounds that hold terms
        const int e = min((int)threadIdx.x + q * NT, nterm - 1);
        sa[q] = aS[e >> 3];
        sb[q] = bS[(size_t)(e >> 3) * p.N + n0 + (e & 7)];
    }
    for (int e = threadIdx.x; e < nterm; e += NT) P[e] = 0;
    __syncthreads();
    const int kb0 = w * kbw, kb1 = min(kb0 + kbw, p.KB);
    const int g4 = (lane >> 3) & 3, sub = lane >> 5, col = lane & 7;
    const v4i *bp = (const v4i *)p.B + (size_t)nb * p.KB * 64 + g4 * 16 + h * 8 + col;
    const char *A = (const char *)p.A;
    const Lut L = {p.lut[0], p.lut[1], p.lut[2], p.lut[3]};
    // a lane's dot products run on while its group stays the same; where every block lies in one group (G a multiple
    // of the block's k, so K has no tail inside a block and a 32-lane half's lanes always share their group) the four
    // k-group lanes of a column are summed first (l ^ 8, l ^ 16), and one of them adds the sum
    const bool whole = G % T::KPB == 0;
    int run = 0, rg = -1;
    auto flush = [&]() {
        int v = run;
        if (whole) {
            v += __builtin_amdgcn_update_dpp(0, v, 0x128, 0xF, 0xF, false); // row_ror:8 -> lane l ^ 8
            const auto sw = __builtin_amdgcn_permlane16_swap(v, v, false, false);
            v += (int)((lane & 16) == 0 ? sw[1] : sw[0]);
        }
        if (rg >= 0 && (!whole || g4 == 0)) atomicAdd(&P[rg * 8 + col], v);
    };
    for (int kb = kb0; kb < kb1; kb += 2 * NI) {
        v4i raw[NI], act[NI][W / 4];
        bool ok[NI];
#pragma unroll
        for (int q = 0; q < NI; q++)
            raw[q] = __builtin_nontemporal_load(bp + (size_t)min(kb + 2 * q + sub, kb1 - 1) * 64);
#pragma unroll
        for (int q = 0; q < NI; q++) {
            const int blk = kb + 2 * q + sub, k0 = blk * T::KPB + g4 * (W * 4);
            ok[q] = blk < kb1 && k0 < p.K;
#pragma unroll
            for (int j = 0; j < W / 4; j++) act[q][j] = *(const v4i *)(A + (ok[q] ? k0 + 16 * j : 0));
        }
#pragma unroll
        for (int q = 0; q < NI; q++) {
            v4i op[T::STEPS];
            decode<KIND>(raw[q], op, L);
            int dot = 0;
#pragma unroll
            for (int d = 0; d < W; d++) dot = __builtin_amdgcn_sdot4(act[q][d / 4][d % 4], op[d / 4][d % 4], dot, false);
            const int g = ok[q] ? ((kb + 2 * q + sub) * T::KPB + g4 * (W * 4)) / G : rg; // past the run: adds 0 to rg
            if (g != rg) { // uniform across a 32-lane half when whole, since its lanes share the block
                flush();
                run = 0;
                rg = g;
            }
            run += ok[q] ? dot : 0;
        }
    }
    flush();
    __syncthreads();
#pragma unroll
    for (int q = 0; q < SPT; q++) {
        if (q * NT >= nterm) break;
        const int e = (int)threadIdx.x + q * NT;
        if (e < nterm) {
            const float t = ((float)finish<KIND>(P[e]) * sa[q]) * sb[q];
            P[e] = __builtin_bit_cast(int, t);
        }
    }
    __syncthreads();
    if (threadIdx.x < 8) {
        float c = 0.0f;
        for (int g = 0; g < Sk; g++) c = c + __builtin_bit_cast(float, P[g * 8 + threadIdx.x]);
        C[n0 + threadIdx.x] = c;
    }
}

// k_grouped: grid (N/16, row tiles of 16*MT), 4 waves. Workgroup (nb, mtile) owns panel nb and walks its
// K-groups QG at a time: wave w computes groups w, w+4, ... of the chunk over the blocks holding
// k in [g*G, g*G + G) (every A chunk is 16 k wide and 16-k aligned and G % 32 == 0, so a chunk lies wholly
// inside or outside a group: chunks outside are zero; a block shared by two groups is read by both),
// writes the scaled terms to LDS, and after a barrier each thread adds the chunk's terms of its own output
// elements in group order.
constexpr int QG = 8; // groups per LDS chunk

template <int KIND, int MT>
__global__ __launch_bounds__(256) void k_grouped(orkh_mm p, int G, const float *aS, const float *bS, float *C, int ldc) {
#pragma clang fp contract(off)
    using T = KT<KIND>;
    __shared__ float xs[QG][MT * 256];
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nb = blockIdx.x, m0 = blockIdx.y * 16 * MT;
    const int Sk = p.K / G;
    const int r16 = lane & 15, gq = lane >> 4;
    const char *A = (const char *)p.A;
    const Lut L = {p.lut[0], p.lut[1], p.lut[2], p.lut[3]};
    const v4i *bp = (const v4i *)p.B + (size_t)nb * p.KB * 64 + lane;
    const int ncol = nb * 16 + (lane & 15);

    float c[MT]; // this thread's output elements e = threadIdx.x + 256 * i, summed in group order
#pragma unroll
    for (int i = 0; i < MT; i++) c[i] = 0.0f;

    for (int g0 = 0; g0 < Sk; g0 += QG) {
        const int nq = min(QG, Sk - g0);
        for (int q = w; q < nq; q += 4) {
            const int grp = g0 + q, k_lo = grp * G, k_hi = k_lo + G;
            const int kb_lo = k_lo / T::KPB, kb_hi = (k_hi + T::KPB - 1) / T::KPB;
            v4i acc[MT];
#pragma unroll
            for (int mt = 0; mt < MT; mt++) acc[mt] = v4i{0, 0, 0, 0};
            for (int kb = kb_lo; kb < kb_hi; kb++) {
                v4i av[T::STEPS][MT];
#pragma unroll
                for (int s = 0; s < T::STEPS; s++)
#pragma unroll
                    for (int mt = 0; mt < MT; mt++) {
                        const int row = m0 + mt * 16 + r16, k = kb * T::KPB + a_koff<KIND>(s, gq);
                        const bool ok = row < p.M && k >= k_lo && k < k_hi;
                        av[s][mt] = *(const v4i *)(A + (size_t)(ok ? row : 0) * p.lda + (ok ? k : 0));
                        if (!ok) av[s][mt] = v4i{0, 0, 0, 0};
                    }
                v4i op[T::STEPS];
                decode<KIND>(__builtin_nontemporal_load(bp + (size_t)kb * 64), op, L);
#pragma unroll
                for (int s = 0; s < T::STEPS; s++)
#pragma unroll
                    for (int mt = 0; mt < MT; mt++) acc[mt] = mma(av[s][mt], op[s], acc[mt]);
            }
            // scaled term of each output element of the tile: acc[mt][r] is row (lane/16)*4 + r, column lane%16
            const float bsn = bS[(size_t)grp * p.N + ncol];
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int m = min(m0 + mt * 16 + (lane >> 4) * 4 + r, p.M - 1);
                    xs[q][mt * 256 + r * 64 + lane] = ((float)finish<KIND>(acc[mt][r]) * aS[(size_t)m * Sk + grp]) * bsn;
                }
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < MT; i++)
            for (int q = 0; q < nq; q++) c[i] = c[i] + xs[q][threadIdx.x + 256 * i];
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < MT; i++) {
        const int e = threadIdx.x + 256 * i;
        const int mt = e >> 8, r = (e >> 6) & 3, ln = e & 63;
        const int m = m0 + mt * 16 + (ln >> 4) * 4 + r;
        const int n = nb * 16 + (ln & 15);
        if (m < p.M) C[(size_t)m * ldc + n] = c[i];
    }
}

// ------------------------------------------------------------------------------------------------
// k_tiled2: one 16-wave workgroup per BM x BN output tile (waves 4 x 4 over the tile; on 32-row tiles, groups
// of waves that split each stage's K-blocks, see T2). Both operands
// go HBM/L2 -> LDS with direct-to-LDS buffer loads (no VGPR round trip), issued in MFMA fragment order so
// the LDS image of a stage is already the operand layout: A fragment (mb, kbl, step) = 16 rows x 16 bytes
// per lane row/k-group exactly as mma() takes it, B = the 1 KiB panel blocks verbatim. A ring of R stage
// slots keeps R - 1 stages in flight; each stage costs one barrier. Loads are hidden from the compiler
// (inline asm), so their completion is tracked by hand: every wave issues IPW loads per stage (padding
// loads land in a junk block) and waits until at most (R - 2) * IPW are outstanding before the barrier
// that publishes the stage. Raw buffer loads return 0 past a resource's end, which zero-fills M / N / K
// edges and the stages past the end of K.
// M0 carries the LDS destination; nothing else in these kernels uses M0 (checked in the ISA), so the
// clobber of that reserved register is safe and its warning is silenced here.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// SITE only numbers the call site in an asm comment: identical asm at several sites lets the compiler merge them
// through a phi it may place in a VGPR, which the "s" operand cannot take.
template <int SITE = 0>
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t lds_byte) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds ; site %3" ::"s"(lds_byte),
                 "v"(voff), "s"(r), "i"(SITE)
                 : "memory", "m0");
}
#pragma clang diagnostic pop
template <int VM> __device__ __forceinline__ void wait_vmcnt() {
    static_assert(VM >= 0 && VM < 64, "vmcnt");
    __builtin_amdgcn_s_waitcnt((VM & 15) | ((VM >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Waves across a tile's block columns: all of them up to 4, else 4 when they divide evenly, else 2.
constexpr int t2_wn(int nb) { return nb < 4 ? nb : (nb % 4 == 0 ? 4 : 2); }

template <int KIND, int BM, int BN, int KS, int XG = 0, int RC = 0> struct T2 {
    using T = KT<KIND>;
    static constexpr int MB = BM / 16, NB = BN / 16, NW = 16;
    // 16 waves: WM x WN over the tile's 16 x 16 blocks and, on tiles of fewer than 16 blocks (32- and 16-row tiles)
    // or whose 6 block columns take 2 waves (128 x 96: 32 x 48 of C per wave), WK groups that split each stage's
    // K-blocks; their partial tiles are summed through LDS after the loop, in group order (deterministic for fp16)
    static constexpr int WM = XG ? 2 : (MB < 4 ? MB : 4), WN = XG == 2 ? 2 : t2_wn(NB), WK = NW / (WM * WN);
    static constexpr int MTW = MB / WM, NTW = NB / WN, KPW = KS / WK; // blocks and K-blocks per wave
    static constexpr int NIA = MB * KS * T::STEPS, NIB = NB * KS, NI = NIA + NIB;  // loads per stage
    static constexpr int IPW = (NI + NW - 1) / NW;                               // per wave
    static constexpr int JUNK = IPW * NW > NI ? 1 : 0;
    static constexpr int SLOT = (NI + JUNK) * 1024;
    // NF4: a stage's B blocks are decoded once, into int8 MFMA operands in LDS, instead of by each of the
    // WM waves that read a block (the codebook decode is ~8x the VALU work of the uniform-int4 one)
    // Two stages of them where a ring of 3 slots still fits (the decode then runs a stage ahead: tiled2_body)
    static constexpr int DEC1 = KIND == ORKH_NF4 ? NIB * T::STEPS * 1024 : 0;
    static constexpr bool DEC2 = KIND == ORKH_NF4 && RC == 0 && (163840 - 2 * DEC1) / SLOT >= 3;
    static constexpr int DEC = DEC2 ? 2 * DEC1 : DEC1;
    // ring within 160 KiB: 4 slots. More bytes in flight per CU delay a stage's last lines (a CU's deliveries
    // interleave across the stages it has asked for) more than they feed the loop: 8 slots on the K-group tiles
    // measured slower (us: W4A8 M=64 K=2048 N=6144 32 x 64 6.12 -> 7.14, NF4 7.57 -> 8.61, int8 M=128 K=N=2048
    // 32 x 32 5.35 -> 6.34, fp16 8.26 -> 8.79), and so did 8 slots for the 12-16 KiB stages of the other tiles (int8
    // M=128 64 x 64 8.5 -> 9.4, fp16 M=512 13.0 -> 14.0); 3 slots lose too (W4A8 M=64 6.12 -> 6.48, fp16 M=512
    // 64 x 64 12.86 -> 14.68), and 2 lose badly
    static constexpr int RMAX = 4;
    // RC: a ring of RC slots instead (k_tiled2's two-workgroups-per-CU form, launch_tiled2_v)
    static constexpr int R = RC ? RC : ((163840 - DEC) / SLOT) < RMAX ? ((163840 - DEC) / SLOT) : RMAX;
    static constexpr size_t LDS = (size_t)R * SLOT + DEC;
    static constexpr size_t RED = (size_t)(WK - 1) * WM * WN * MTW * NTW * 1024; // K-group partial tiles
    // A stage whose rows are whole 128-byte lines (ALN of them a row: 1, 2 or 4) is loaded a line at a time (8 rows
    // x 128 B per instruction) instead of in MFMA fragment order (16 rows x 64 B: every line fetched by two
    // instructions), and read from a swizzled image (a_lds)
    static constexpr int ALN = KS * T::KPB * T::ESZ / 128;
    static constexpr bool LINE_OK = KS * T::KPB * T::ESZ % 128 == 0;
    static_assert(MB % WM == 0 && NB % WN == 0 && WM * WN * WK == NW && KS % WK == 0 && R >= 2 && (R - 2) * IPW < 64,
                  "tile");
    static_assert(RED <= (size_t)R * SLOT, "K-group partials must fit the ring");
    static_assert(!LINE_OK || NIA * 8 == BM * ALN, "line-loaded A: one instruction per 8 row lines");
};

// Wave grids other than 4 x 4 (grouped runs always keep it):
// 1: 2 x 4 with 2 K groups (each B block decoded by two waves instead of four), for the uniform-int4 64 x 192
//    tile. Measured against 4 x 4 (us): W4A8 K=2048 N=6144 M=512 14.7 -> 13.4, M=256 13.3 -> 12.5; W4A4 M=512
//    K=N=4096 22.0 -> 19.9. Not kept elsewhere: int8 M=512 64 x 192 13.9 -> 14.7, fp16 M=1024 20.5 -> 21.1,
//    uniform int4 128 x 128 21.9 -> 22.4 (W4A4 M=256), 64 x 64 unchanged.
// 2: 2 x 2 with 4 K groups (each wave 32 x 32 of C: half the LDS reads per MFMA of a 16 x 16 wave block, each B
//    block decoded by two waves), for the uniform-int4 64 x 64 tile: W4A4 M=256 K=N=4096 14.76 -> 14.00. Not
//    kept for fp16 (M=512 K=N=2048 13.98 -> 15.35).
template <int KIND, int BM, int BN, int GR> constexpr int t2_xg() {
    if (GR != 0) return 0;
    if (KIND == ORKH_I4U && BM == 64 && BN == 192) return 1;
    if (KIND == ORKH_I4U && BM == 64 && BN == 64) return 2;
    return 0;
}

// Where in a stage the waves of the LDS-ring kernel issue the loads of the stage R - 1 ahead: before K-block t2_issue_at
// of their stage work (0: right after the stage's barrier; KPW: after their last K-block). Every wave still issues each
// stage once, in stage order, inside the iteration, so the waits count as before. Issuing right after the barrier
// holds every wave of a SIMD on the issue of loads into a full memory pipeline at once with no MFMA ready behind
// them; later, the MFMAs of the waves not held go on. Graph-timed against right after the barrier (one build each,
// alternated twice on one box; int8 and fp16 through bench.py's config section too; exact): int8 64 x 192 M=512
// K=2048 N=6144 13.56-13.68 -> 13.15-13.28 us (after the first of two K-blocks; after both: -0.4 to -0.9%); NF4
// 128 x 128 M=512 16.62 -> 15.46 (after its one K-block); grouped W4A4 K=N=4096 G=128 64 x 64 M=256 18.33 -> 17.08
// (after the first of four); uniform int4 64 x 192 W4A4 M=512 18.54 -> 17.95, W4A8 M=512 12.67 -> 12.54, 32 x 64
// W4A8 M=64 6.03 -> 5.94 (after their one); int8 32 x 64 (four chained M=256 runs) 13.92 -> 13.32-13.80. No gain, so
// right after the barrier: fp16 64 x 64 M=512 (-0.3 to +0.6% either way), uniform int4 on the 2 x 2 x 4 wave grid
// (64 x 64, W4A4 M=256: +0.4 to +0.8%) and NF4 on the K-group tiles (its decode runs a stage ahead; -0.1 to -0.6%);
// the two-slot rings, whose second workgroup per CU already overlaps one's loads with the other's MFMAs, keep it too.
template <int KIND, int BM, int BN, class P> constexpr int t2_issue_at() {
    if (P::R <= 2 || (KIND == ORKH_NF4 && P::WK > 1) || (KIND == ORKH_F16 && BM == 64 && BN == 64) ||
        (KIND == ORKH_I4U && BM == 64 && BN == 64 && P::WK > 1)) // the 2 x 2 x 4 grid; grouped runs keep 4 x 4
        return 0;
    return 1;
}

// How many of the 16 waves issue a stage's loads (the others only compute: they never wait on the issue of a load
// into a full memory pipeline, so the matrix cores keep them). Wave wv < LW issues loads wv, wv + LW, ...; the
// stage's load count must divide evenly. Graph-timed against every wave issuing (one build each, alternated twice
// on one box; exact): 8 loader waves on uniform int4's 64 x 192 tile (2 x 4 x 2 grid): W4A4 K=N=4096 M=512 18.04 ->
// 16.80 us, W4A8 K=2048 N=6144 M=512 12.23 -> 11.70, M=256 12.07 -> 11.45; 4 on the NF4 K-group tiles (32 x 64, C3
// NF4 M=64 7.36 -> 6.98) and on 256 x 256 (M=K=N=4096 int8 67.1 -> 65.6, fp16 134.3 -> 126.0). Once A stages were
// line-loaded (rows of 2 and 4 lines included), 8 loader waves also on: uniform int4's 2 x 2 x 4 64 x 64 tile (W4A4
// K=N=4096 M=256 9.97 -> 9.14, W4A8 K=2048 N=6144 M=128 7.33 -> 6.65, M=96 7.03 -> 6.45; 4 loaders 9.66); the 32 x 32
// and 16 x 32 K-group tiles (fp16 K=N=2048 M=128 7.61 -> 7.25, M=48 6.84 -> 6.32; int8 M=128 5.52 -> 5.27, M=64 5.24
// -> 4.83, K=6144 N=2048 M=32 8.62 -> 8.05; W4A4 K=N=4096 M=64 6.90 -> 6.35; W4A8 K=N=2048 M=64 4.03 -> 3.87); int8
// 64 x 64 (K=2048 N=6144 M=128 7.89 -> 7.59, K=N=2048 M=512 7.85 -> 7.40); 128 x 128 (W4A8 K=2048 N=6144 M=512 13.28
// -> 12.46, fp16 21.85 -> 21.26, int8 K=N=4096 M=512 20.31 -> 19.83, K=2048 N=6144 12.51 -> 12.45). Elsewhere no gain
// (int8 64 x 192 M=512: 8 loaders -0.2 to -0.8%, 4 +2.6 to +3.0%; the two-slot rings +4 to +9%; the 32 x 64 tiles
// -0.3 to +1.6%; 128 x 96 and fp16 64 x 64 within 0.5%), so there every wave issues. NF4's 64 x 64 tile takes 4 (K=2048
// N=6144 M=128 9.58 -> 9.41, K=6144 N=2048 M=128 split 4 ways 12.66 -> 12.30; 8 loaders no gain); its 128 x 96 and
// 128 x 128 tiles gain nothing from 4 or 8. 4 loader waves on int8 128 x 96 (K=N=4096 M=512 18.97-19.01 -> 18.23-18.27,
// K=2048 N=6144 M=384 11.98 -> 11.65-11.72, M=512 12.76-12.86 -> 12.69-12.78; 8 measured no gain) and fp16 64 x 64
// (C2 M=512 12.39-12.44 -> 12.26-12.27); fp16 128 x 96 with 4: +0.6%.
template <int KIND, int BM, int BN, class P> constexpr int t2_loaders() {
    int lw = P::NW;
    if (P::R <= 2) return lw;
    if (KIND == ORKH_I4U && BM == 64 && BN == 192) lw = 8;
    else if (KIND == ORKH_NF4 && (P::WK > 1 || (BM == 64 && BN == 64))) lw = 4;
    else if ((KIND == ORKH_I8 || KIND == ORKH_F16) && BM == 256 && BN == 256) lw = 4;
    else if (KIND != ORKH_NF4 && BM == 128 && BN == 128) lw = 8;
    else if ((KIND == ORKH_I8 && BM == 128 && BN == 96) || (KIND == ORKH_F16 && BM == 64 && BN == 64)) lw = 4;
    else if (KIND == ORKH_I4U && BM == 64 && BN == 64 && P::WK > 1) lw = 8;
    else if (KIND == ORKH_I8 && BM == 64 && BN == 64) lw = 8;
    else if (KIND != ORKH_NF4 && BN == 32 && (BM == 32 || BM == 16)) lw = 8;
    return P::NI % lw == 0 ? lw : P::NW;
}

// Index (in 16-byte units) within a stage's A image of lane `lane`'s operand of fragment (mb, kbl, st).
// Fragment order: fragment f = (mb, kbl, st) is 1 KiB at f, lane-major, as mma() takes it.
// Line order: 1 KiB per (line li of the stage row, 8-row group g8), at li * BM8 + g8 (BM8 = the tile's 8-row
// groups); row r's 128-byte line li holds its 16-byte chunk c at slot c ^ (r & 7) ^ ((r >> 3) & 1). The swizzle
// puts the chunks that any 16 consecutive lanes of a fragment read (16 rows, one chunk) in 16 distinct bank
// groups, so the 128-bit LDS reads stay conflict-free; the loads write each instruction's 8 lines with the same
// permutation (lane l of instruction li * BM8 + g8: row 8 g8 + l/8, slot l % 8).
template <int KIND, int KS, bool LINE, int BM8>
__device__ __forceinline__ int a_lds(int mb, int kbl, int st, int lane) {
    using T = KT<KIND>;
    if constexpr (LINE) {
        const int c = (kbl * T::KPB + a_koff<KIND>(st, lane >> 4)) * T::ESZ / 16; // chunk within the stage row
        const int r7 = lane & 7, h = (lane >> 3) & 1;
        return ((c >> 3) * BM8 + mb * 2 + h) * 64 + r7 * 8 + ((c & 7) ^ r7 ^ h);
    } else {
        return ((mb * KS + kbl) * T::STEPS + st) * 64 + lane;
    }
}

// Quotient and remainder of a wave-uniform x / d (0 <= x, 1 <= d, both < 2^24) on the VALU: the correctly
// rounded float quotient is within one of the integer one, and one correction fixes it. A scalar integer
// division is ~35 instructions on the scalar unit, which a workgroup's 16 waves share; two of them per wave
// in a tiled kernel's prologue queue ~1,000 cycles there.
__device__ __forceinline__ void udivmod(int x, int d, int &q, int &r) {
    int qq = (int)((float)x / (float)d);
    int rr = x - qq * d;
    if (rr < 0) { qq--; rr += d; }
    else if (rr >= d) { qq++; rr -= d; }
    q = __builtin_amdgcn_readfirstlane(qq);
    r = __builtin_amdgcn_readfirstlane(rr);
}

// Grouped mode of k_tiled2 (ork_*_mm_run_grouped): C is fp32 and every output is the sum, in ascending g, of
// ((float)P_g * aS[m][g]) * bS[g][n] with P_g the exact int32 partial over K-group g (src/npu/core/buf.c:501-520).
struct T2Group {
    int G;            // group size in k; G % 32 == 0 and K % G == 0
    const float *aS;  // [M][K/G]
    const float *bS;  // [K/G][N]
};

// bid, nT: this workgroup's index among the launch's nT workgroups of this matmul (blockIdx.x and gridDim.x, or a
// task's share of a grouped launch, which starts at a multiple of 8 so that bid % 8 is still the XCD)
template <int KIND, int BM, int BN, int KS, int GR, bool AL, int RC = 0>
__device__ __forceinline__ void tiled2_body(const orkh_mm &p, int mtiles, int ntiles_all, int kbs, void *ws,
                                            const T2Group &gp, int bid, int nT) {
#pragma clang fp contract(off)
    using T = KT<KIND>;
    using P = T2<KIND, BM, BN, KS, t2_xg<KIND, BM, BN, GR>(), RC>;
    constexpr int R = P::R;
    constexpr bool LINE = AL && P::LINE_OK; // A stage as whole row lines (a_lds), else in fragment order
    typedef typename T::acc_t acc_t;
    typedef typename T::c_t c_t;
    extern __shared__ v4i sm[];
    // Every kernel argument this body reads is loaded here, in one batch behind one wait: left to itself the compiler
    // issues each scalar load at its first use, behind the branches and divisions of the tile index, five waits in a
    // row. Graph-timed against that, three alternations on one box, exact (us): int8 64 x 192 M=512 13.23 -> 13.02,
    // fp16 K=N=2048 64 x 64 M=512 12.72 -> 12.47, 32 x 32 M=128 8.22 -> 8.07, W4A8 32 x 64 M=64 5.94 -> 5.83, W4A4
    // 2 x 2 x 4 M=256 12.28 -> 12.00.
    asm volatile("" ::"s"(p.M), "s"(p.K), "s"(p.N), "s"(p.KB), "s"(p.lda), "s"(p.A), "s"(p.B), "s"(p.C), "s"(p.ldc),
                 "s"(p.c_wt), "s"(mtiles), "s"(ntiles_all), "s"(kbs), "s"(ws), "s"(nT));
    if constexpr (GR != 0) asm volatile("" ::"s"(gp.G), "s"(gp.aS), "s"(gp.bS));
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    static_assert(GR == 0 || P::WK == 1, "grouped runs walk every K-block in one wave");
    const int wk = P::WK > 1 ? wv / (P::WM * P::WN) : 0, wr = P::WK > 1 ? wv % (P::WM * P::WN) : wv;
    const int wm = wr % P::WM, wn = wr / P::WM;
    // XCD-aware order: WG b runs on XCD b%8; each XCD gets a contiguous run of tiles, M fastest, so every
    // M-tile that reads a given B column panel shares one L2.
    const int per = nT / 8, rem = nT % 8, x = bid % 8, j = bid / 8;
    const int tl = (x < rem) ? x * (per + 1) + j : rem * (per + 1) + (x - rem) * per + j;
    int ks, tile, tn, tm;
    udivmod(tl, ntiles_all, ks, tile);
    udivmod(tile, mtiles, tn, tm);
    const int m0 = tm * BM, nb0 = tn * P::NB;
    const int NBtot = p.N / 16;
    const int kb_lo = ks * kbs, kb_hi = min(kb_lo + kbs, p.KB);
    const int k_hi = min(kb_hi * T::KPB, p.K);
    const uint32_t lda_b = (uint32_t)p.lda * T::ESZ;
    const __amdgpu_buffer_rsrc_t Ar = make_rsrc(p.A, (uint32_t)p.M * lda_b);
    const __amdgpu_buffer_rsrc_t Br = make_rsrc(p.B, (uint32_t)NBtot * p.KB * 1024u);
    const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void *)sm;
    const Lut L = {p.lut[0], p.lut[1], p.lut[2], p.lut[3]};

    // this wave's loads: i = wv + q * LW (waves wv >= LW issue none); A fragment (mb, kbl, step) or B block (nbl, kbl).
    // Grouped runs: 8 loader waves, which also issue the tile's scale loads (before their ring loads, so their first
    // wait covers them): W4A4 K=N=4096 G=128 M=256 16.64-16.85 -> 16.07-16.26 us against every wave issuing, exact
    constexpr int LW = GR == 0 ? t2_loaders<KIND, BM, BN, P>() : (P::NI % 8 == 0 ? 8 : P::NW);
    constexpr int IPW = LW == P::NW ? P::IPW : P::NI / LW;
    static_assert(LW == P::NW || P::NI % LW == 0, "loader waves");
    static_assert((R - 2) * IPW < 64, "vmcnt");
    uint32_t voff[IPW];
    int kof[IPW];
#pragma unroll
    for (int q = 0; q < IPW; q++) {
        const int i = wv + q * LW;
        voff[q] = OOB;
        kof[q] = 0;
        if (i < P::NIA && LINE) {
            // line li of rows 8 g8 .. 8 g8 + 7 (i = li * BM / 8 + g8); lane l fills slot l % 8 of row 8 g8 + l / 8
            const int li = i / (BM / 8), g8 = i % (BM / 8);
            const int rr = lane >> 3, slot = lane & 7;
            const int row = m0 + g8 * 8 + rr;
            kof[q] = (li * 128 + (slot ^ rr ^ (g8 & 1)) * 16) / T::ESZ;
            if (row < p.M) voff[q] = (uint32_t)row * lda_b + (uint32_t)kof[q] * T::ESZ;
        } else if (i < P::NIA) {
            const int mb = i / (KS * T::STEPS), rest = i % (KS * T::STEPS);
            const int kbl = rest / T::STEPS, st = rest % T::STEPS;
            const int row = m0 + mb * 16 + (lane & 15);
            kof[q] = kbl * T::KPB + a_koff<KIND>(st, lane >> 4);
            if (row < p.M) voff[q] = (uint32_t)row * lda_b + (uint32_t)kof[q] * T::ESZ;
        } else if (i < P::NI) {
            const int ii = i - P::NIA, nbl = ii / KS;
            kof[q] = ii % KS;
            if (nb0 + nbl < NBtot) voff[q] = ((uint32_t)(nb0 + nbl) * p.KB * 64 + lane) * 16;
        }
    }
    const int nst = (kb_hi - kb_lo + KS - 1) / KS;
    auto issue = [&](int st, auto site) { // site: std::integral_constant numbering the call site (lds_dma16)
        constexpr int SA = 2 * decltype(site)::value, SB = SA + 1;
        const uint32_t slot = lds0 + (uint32_t)(st % R) * P::SLOT;
        const int kb0 = kb_lo + st * KS;
        if (LW < P::NW && wv >= LW) return;
#pragma unroll
        for (int q = 0; q < IPW; q++) {
            const int i = wv + q * LW;
            if (i < P::NIA) {
                const int k = kb0 * T::KPB + kof[q];
                lds_dma16<SA>(Ar, (voff[q] != OOB && k < k_hi) ? voff[q] + (uint32_t)kb0 * T::KPB * T::ESZ : OOB,
                          slot + i * 1024);
            } else {
                const int kb = kb0 + kof[q];
                lds_dma16<SB>(Br, (i < P::NI && voff[q] != OOB && kb < kb_hi) ? voff[q] + (uint32_t)kb * 1024u : OOB,
                          slot + (i < P::NI ? i : P::NI) * 1024);
            }
        }
    };

    acc_t acc[P::MTW][P::NTW];
#pragma unroll
    for (int a = 0; a < P::MTW; a++)
#pragma unroll
        for (int b = 0; b < P::NTW; b++) acc[a][b] = acc_t{0, 0, 0, 0};

    // grouped mode: fp32 running sums, and this tile's scales in LDS after the ring -- aS rows m0.. (BM x Sk,
    // one contiguous run of aS) and bS columns n0.. of every group (Sk x BN) -- brought in by direct-to-LDS
    // loads issued before the ring's, so the first stage's wait covers them and no later wait drains the
    // ring. Rows past M read zeros and columns past N read a neighbouring row; neither is stored.
    const int Sk = GR ? p.K / gp.G : 1;
    const int sca_kib = GR ? (BM * Sk * 4 + 1023) / 1024 : 0;
    const int scb_kib = GR ? (Sk * BN * 4 + 1023) / 1024 : 0;
    const float *sAl = (const float *)(sm + P::LDS / 16);
    const float *sBl = sAl + sca_kib * 256;
    float cacc[P::MTW][P::NTW][4];
    float sa[P::MTW][4], sb[P::NTW]; // scales of the next group to close
    int gcur = 0, gend = GR ? gp.G : 0; // that group and the k where it ends
    const int gps = GR == 2 ? gp.G / T::KPB : 1; // K-blocks per group (groups of whole K-blocks)
    int sgs = 0;                                   // K-blocks of the current group done
    auto load_sc = [&](int g) {
#pragma unroll
        for (int i = 0; i < P::MTW; i++)
#pragma unroll
            for (int r = 0; r < 4; r++) sa[i][r] = sAl[((wm * P::MTW + i) * 16 + (lane >> 4) * 4 + r) * Sk + g];
#pragma unroll
        for (int jn = 0; jn < P::NTW; jn++) sb[jn] = sBl[g * BN + (wn * P::NTW + jn) * 16 + (lane & 15)];
    };
    // close group gcur: its exact partial, scaled, joins the fp32 sums in group order; read the next scales
    auto close_group = [&]() {
#pragma unroll
        for (int i = 0; i < P::MTW; i++)
#pragma unroll
            for (int jn = 0; jn < P::NTW; jn++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float t = ((float)finish<KIND>(acc[i][jn][r]) * sa[i][r]) * sb[jn];
                    cacc[i][jn][r] = cacc[i][jn][r] + t;
                    acc[i][jn][r] = 0;
                }
        gcur++;
        if (gcur < Sk) load_sc(gcur); // read ahead: waited for at the next close
    };
    if constexpr (GR) {
#pragma unroll
        for (int i = 0; i < P::MTW; i++)
#pragma unroll
            for (int jn = 0; jn < P::NTW; jn++)
#pragma unroll
                for (int r = 0; r < 4; r++) cacc[i][jn][r] = 0.0f;
        const uint32_t scl = lds0 + (uint32_t)P::LDS;
        const __amdgpu_buffer_rsrc_t Sa = make_rsrc(gp.aS, (uint32_t)p.M * Sk * 4u);
        const __amdgpu_buffer_rsrc_t Sb = make_rsrc(gp.bS, (uint32_t)Sk * p.N * 4u);
        for (int i = wv; wv < LW && i < sca_kib + scb_kib; i += LW) {
            if (i < sca_kib) {
                lds_dma16<8>(Sa, (uint32_t)m0 * Sk * 4u + (uint32_t)i * 1024u + lane * 16u, scl + i * 1024);
            } else {
                const int f = (i - sca_kib) * 256 + lane * 4; // first float of this lane within the Sk x BN tile
                const int g = f / BN, c = f - g * BN;
                lds_dma16<9>(Sb, g < Sk ? ((uint32_t)g * p.N + nb0 * 16 + c) * 4u : OOB, scl + i * 1024);
            }
        }
    }

    // NF4 (plain runs): a stage's B blocks are decoded once, into int8 MFMA operands in LDS, one stage ahead of
    // their MFMAs -- iteration s decodes stage s + 1 into one half of Dec while its MFMAs read stage s from the
    // other, so the codebook decode (VALU) overlaps the matrix work and the stage keeps a single barrier.
    // Measured against decoding each stage before its MFMAs behind a second barrier (us, K=2048 N=6144 unless
    // given): 32 x 64 M=64 9.19 -> 8.63, K=6144 N=2048 17.96 -> 15.65; 64 x 64 M=256 15.77 -> 14.49, M=512
    // K=6144 N=2048 27.50 -> 23.82; 128 x 128 M=512 18.84 -> 17.60, M=1024 34.83 -> 29.58.
    // Who decodes, and when (measured, same shapes): on the K-group tiles (32 x 64: 8 blocks a stage) every wave
    // takes an equal share of dwords and decodes before its MFMAs (8.74 -> 8.63, 16.04 -> 15.65 against a block
    // per wave after them); on the others a block per wave decodes after the wave's MFMAs (64 x 64 M=256 15.54
    // -> 14.49, 128 x 128 M=1024 32.96 -> 29.58 against equal shares before them). Equal shares with half the
    // waves of each SIMD decoding first and half after measured slower than both.
    constexpr bool PIPE = P::DEC2 && GR == 0;
    constexpr bool EARLY = PIPE && P::WK > 1;
    static_assert(!PIPE || R >= 3, "NF4 ring: the decode runs a stage ahead");
    v4i *const Dec = sm + P::R * (P::SLOT / 16); // [stage parity, if PIPE][block][step]
    static_assert(P::DEC >= (PIPE ? 2 : 1) * P::DEC1, "NF4 decode buffers");
    auto decode_stage = [&](int st) {
        const v4i *Bs = sm + (st % R) * (P::SLOT / 16) + P::NIA * 64;
        v4i *D = Dec + (PIPE ? (st & 1) : 0) * (P::NIB * T::STEPS * 64); // one buffer unless pipelined
        // every wave an equal share where the stage's NIB x 4 dword columns divide evenly (dword j of each lane's
        // 16 bytes of block b is column 4 b + j): DPW of them, at wave-uniform offsets; dword j's low and high
        // nibbles go where decode() puts them, operand j / 2, dwords 2 (j % 2) and 2 (j % 2) + 1
        constexpr int DPW = P::NIB * 4 % P::NW ? 0 : P::NIB * 4 / P::NW;
        if constexpr (EARLY && (DPW == 1 || DPW == 2 || DPW == 4)) {
            const int c0 = wv * DPW, b = c0 >> 2, j0 = c0 & 3;
            const uint32_t *src = (const uint32_t *)(Bs + b * 64 + lane) + j0;
            uint32_t x[DPW], lo[DPW], hi[DPW];
            if constexpr (DPW == 4) {
                const v4i r = *(const v4i *)src;
                x[0] = r.x, x[1] = r.y, x[2] = r.z, x[3] = r.w;
            } else if constexpr (DPW == 2) {
                const uint2 r = *(const uint2 *)src;
                x[0] = r.x, x[1] = r.y;
            } else {
                x[0] = *src;
            }
#pragma unroll
            for (int u = 0; u < DPW; u++) nf4_map8(x[u], L, lo[u], hi[u]);
            uint32_t *dst = (uint32_t *)(D + (b * T::STEPS + (j0 >> 1)) * 64 + lane) + (j0 & 1) * 2;
            if constexpr (DPW == 4) {
                *(v4i *)dst = v4i{(int)lo[0], (int)hi[0], (int)lo[1], (int)hi[1]};
                *(v4i *)(dst + 256) = v4i{(int)lo[2], (int)hi[2], (int)lo[3], (int)hi[3]};
            } else if constexpr (DPW == 2) {
                *(v4i *)dst = v4i{(int)lo[0], (int)hi[0], (int)lo[1], (int)hi[1]};
            } else {
                *(uint2 *)dst = make_uint2(lo[0], hi[0]);
            }
        } else {
            for (int b = wv; b < P::NIB; b += P::NW) {
                v4i op[T::STEPS];
                decode<KIND>(Bs[b * 64 + lane], op, L);
#pragma unroll
                for (int u = 0; u < T::STEPS; u++) D[(b * T::STEPS + u) * 64 + lane] = op[u];
            }
        }
    };

    // where in a stage the waves issue the loads of the stage R - 1 ahead (t2_issue_at; grouped runs whose groups
    // close inside K-blocks walk the stage in another loop: right after the barrier)
    constexpr int IA = GR == 1 ? 0 : t2_issue_at<KIND, BM, BN, P>() < P::KPW ? t2_issue_at<KIND, BM, BN, P>() : P::KPW;
#pragma unroll
    for (int st = 0; st < R - 1; st++) issue(st, std::integral_constant<int, 0>{});
    if constexpr (PIPE) {
        if (nst > 0) {
            wait_vmcnt<(R - 2) * IPW>(); // stage 0 (every wave's share: the barrier below)
            __syncthreads();
            decode_stage(0);
        }
    }
    for (int s = 0; s < nst; s++) {
        // stage s has landed (NF4: stage s + 1, whose blocks this iteration decodes); the barrier also publishes
        // the decode of stage s
        wait_vmcnt<(PIPE ? R - 3 : R - 2) * IPW>();
        __syncthreads();
        // into the slot of stage s - 1, which every wave finished before the barrier (NF4: its blocks were decoded
        // in iteration s - 2)
        if constexpr (IA == 0) issue(s + R - 1, std::integral_constant<int, 1>{});
        const v4i *As = sm + (s % R) * (P::SLOT / 16);
        const v4i *Bs = As + P::NIA * 64;
        if constexpr (GR) {
            if (s == 0) load_sc(0); // the scales landed with stage 0 (older loads, same wait)
        }
        const v4i *Ds = Dec + (PIPE ? (s & 1) : 0) * (P::NIB * T::STEPS * 64);
        if constexpr (KIND == ORKH_NF4 && !PIPE) {
            decode_stage(s);
            __syncthreads();
        }
        if constexpr (EARLY) {
            if (s + 1 < nst) decode_stage(s + 1);
        }
        if constexpr (GR != 1) {
#pragma unroll
            for (int kk = 0; kk < P::KPW; kk++) {
                if (kk > 0 && kk == IA) issue(s + R - 1, std::integral_constant<int, 2>{});
                const int kbl = wk * P::KPW + kk; // this wave's K-blocks of the stage
                v4i op[P::NTW][T::STEPS];
#pragma unroll
                for (int jn = 0; jn < P::NTW; jn++) {
                    const int b = (wn * P::NTW + jn) * KS + kbl;
                    if constexpr (KIND == ORKH_NF4) {
#pragma unroll
                        for (int st = 0; st < T::STEPS; st++) op[jn][st] = Ds[(b * T::STEPS + st) * 64 + lane];
                    } else {
                        decode<KIND>(Bs[b * 64 + lane], op[jn], L);
                    }
                }
#pragma unroll
                for (int st = 0; st < T::STEPS; st++)
#pragma unroll
                    for (int i = 0; i < P::MTW; i++) {
                        const v4i a = As[a_lds<KIND, KS, LINE, BM / 8>(wm * P::MTW + i, kbl, st, lane)];
#pragma unroll
                        for (int jn = 0; jn < P::NTW; jn++) acc[i][jn] = mma(a, op[jn][st], acc[i][jn]);
                    }
                if constexpr (GR == 2) {
                    // groups of whole K-blocks: close the group this K-block ends (the zero-filled K-blocks past
                    // the end, in a last stage of fewer, count for none)
                    if (kb_lo + s * KS + kbl < kb_hi && ++sgs == gps) {
                        sgs = 0;
                        close_group();
                    }
                }
            }
            if constexpr (IA > 0 && IA == P::KPW) issue(s + R - 1, std::integral_constant<int, 3>{});
        }
        if constexpr (PIPE && !EARLY) {
            if (s + 1 < nst) decode_stage(s + 1);
        }
        if constexpr (GR == 1) {
            // every fragment of the stage is read first, as above, so the LDS latencies overlap; then the
            // K-blocks run group by group. A 16-k A chunk lies wholly inside one group (G % 32 == 0).
            v4i afr[KS][T::STEPS][P::MTW], bop[KS][P::NTW][T::STEPS];
#pragma unroll
            for (int kbl = 0; kbl < KS; kbl++) {
#pragma unroll
                for (int jn = 0; jn < P::NTW; jn++)
                    decode<KIND>(Bs[((wn * P::NTW + jn) * KS + kbl) * 64 + lane], bop[kbl][jn], L);
#pragma unroll
                for (int st = 0; st < T::STEPS; st++)
#pragma unroll
                    for (int i = 0; i < P::MTW; i++)
                        afr[kbl][st][i] = As[a_lds<KIND, KS, LINE, BM / 8>(wm * P::MTW + i, kbl, st, lane)];
            }
#pragma unroll
            for (int kbl = 0; kbl < KS; kbl++) {
                const int kb = kb_lo + s * KS + kbl;
                if (kb >= kb_hi) break;
                const int kb_k0 = kb * T::KPB, kb_k1 = min(kb_k0 + T::KPB, p.K);
                // the groups meeting [kb_k0, kb_k1) in order, from the running group gcur (no division: a
                // division per block on every wave saturates the CU's scalar unit)
                for (;;) {
                    const int ghi = gend, glo = gend - gp.G;
                    const bool whole = glo <= kb_k0 && ghi >= kb_k1;
#pragma unroll
                    for (int st = 0; st < T::STEPS; st++) {
                        const int kk = kb_k0 + a_koff<KIND>(st, lane >> 4);
                        const bool in = whole || (kk >= glo && kk < ghi);
#pragma unroll
                        for (int i = 0; i < P::MTW; i++) {
                            const v4i a = in ? afr[kbl][st][i] : v4i{0, 0, 0, 0};
#pragma unroll
                            for (int jn = 0; jn < P::NTW; jn++) acc[i][jn] = mma(a, bop[kbl][jn][st], acc[i][jn]);
                        }
                    }
                    if (ghi > kb_k1) break; // the group runs on into the next block
                    close_group(); // group gcur closes in this block
                    gend += gp.G;
                    if (ghi == kb_k1) break;
                }
            }
        }
    }
    wait_vmcnt<0>();

    // The 2 x 2 x 4 uniform-int4 tile (t2_xg 2) and the fp16 32 x 32 tile (4 K groups): all the K groups park
    // their partial tiles in the ring and all 16 waves sum them, in group order (the same fp32 sums as group 0
    // adding them below), and store C, 16 bytes a thread. Measured against group 0 alone summing and storing:
    // W4A4 M=256 K=N=4096 12.93 -> 12.62 us, fp16 M=128 K=N=2048 8.91 -> 8.77; slower on the other K-group tiles
    // (int8 M=128 32 x 32 6.35 -> 6.57, W4A8 M=64 32 x 64 7.16 -> 7.20) and on the tiles without K groups (int8
    // M=512 64 x 192 13.88 -> 14.51), so only here.
    if constexpr (GR == 0 && (t2_xg<KIND, BM, BN, GR>() == 2 || (KIND == ORKH_F16 && BM == 32 && BN == 32))) {
        constexpr int SPAD = BN + 4; // words per parked row: a row's 16-lane store groups start in different banks
        static_assert((size_t)P::WK * BM * SPAD * sizeof(c_t) <= (size_t)R * P::SLOT, "partial tiles fit the ring");
        c_t *Ts = (c_t *)sm;
        __syncthreads(); // every wave's loads have landed (vmcnt 0) and its reads of the ring are done
#pragma unroll
        for (int i = 0; i < P::MTW; i++)
#pragma unroll
            for (int jn = 0; jn < P::NTW; jn++)
#pragma unroll
                for (int r = 0; r < 4; r++)
                    Ts[(wk * BM + (wm * P::MTW + i) * 16 + (lane >> 4) * 4 + r) * SPAD + (wn * P::NTW + jn) * 16 +
                       (lane & 15)] = acc[i][jn][r];
        __syncthreads();
        const bool split = nT > ntiles_all;
        const size_t ldc = split ? (size_t)p.N : (size_t)p.ldc;
        c_t *Cb = split ? (c_t *)ws + (size_t)ks * p.M * p.N : (c_t *)p.C;
        const bool vec = ldc % 4 == 0 && ((uintptr_t)Cb & 15) == 0;
        constexpr int CPR = BN / 4; // 16-byte chunks per tile row
        for (int e = (int)threadIdx.x; e < BM * CPR; e += P::NW * 64) {
            const int row = e / CPR, c4 = (e % CPR) * 4;
            const int m = m0 + row, n = nb0 * 16 + c4; // N % 16 == 0: a chunk lies wholly inside or outside N
            if (m >= p.M || n >= p.N) continue;
            c_t v[4];
#pragma unroll
            for (int u = 0; u < 4; u++) v[u] = Ts[row * SPAD + c4 + u];
#pragma unroll
            for (int g = 1; g < P::WK; g++)
#pragma unroll
                for (int u = 0; u < 4; u++) v[u] += Ts[(g * BM + row) * SPAD + c4 + u];
            c_t *dst = Cb + (size_t)m * ldc + n;
            if (vec) {
                typedef c_t v4c __attribute__((ext_vector_type(4)));
                const v4c o = v4c{finish<KIND>(v[0]), finish<KIND>(v[1]), finish<KIND>(v[2]), finish<KIND>(v[3])};
                if (p.c_wt) store_wt4(dst, __builtin_bit_cast(v4i, o));
                else *(v4c *)dst = o;
            } else {
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    if (p.c_wt) store_wt(&dst[u], finish<KIND>(v[u]));
                    else dst[u] = finish<KIND>(v[u]);
                }
            }
        }
        return;
    }

    if constexpr (P::WK > 1) {
        // K groups 1.. park their partial tiles in the ring (every load has landed: vmcnt 0 on every wave, then
        // the barrier), group 0 adds them in group order and stores
        acc_t *red = (acc_t *)sm;
        __syncthreads();
        if (wk > 0)
#pragma unroll
            for (int i = 0; i < P::MTW; i++)
#pragma unroll
                for (int jn = 0; jn < P::NTW; jn++)
                    red[((((wk - 1) * P::WM * P::WN + wr) * P::MTW + i) * P::NTW + jn) * 64 + lane] = acc[i][jn];
        __syncthreads();
        if (wk > 0) return;
#pragma unroll
        for (int g = 1; g < P::WK; g++)
#pragma unroll
            for (int i = 0; i < P::MTW; i++)
#pragma unroll
                for (int jn = 0; jn < P::NTW; jn++)
                    acc[i][jn] += red[((((g - 1) * P::WM * P::WN + wr) * P::MTW + i) * P::NTW + jn) * 64 + lane];
    }

    // epilogue: one 64-bit base per lane (its first row and column), 32-bit offsets from it
    const int mr0 = m0 + wm * P::MTW * 16 + (lane >> 4) * 4, nc0 = (nb0 + wn * P::NTW) * 16 + (lane & 15);
    const bool split = !GR && nT > ntiles_all;
    const size_t ldc = split ? (size_t)p.N : (size_t)p.ldc;
    using o_t = typename std::conditional<GR != 0, float, c_t>::type;
    o_t *Cl = (split ? (o_t *)ws + (size_t)ks * p.M * p.N : (o_t *)p.C) + (size_t)mr0 * ldc + nc0;
#pragma unroll
    for (int i = 0; i < P::MTW; i++)
#pragma unroll
        for (int jn = 0; jn < P::NTW; jn++) {
            if (nb0 + wn * P::NTW + jn >= NBtot) continue;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                if (mr0 + i * 16 + r >= p.M) continue;
                const uint32_t off = (uint32_t)(i * 16 + r) * (uint32_t)ldc + (uint32_t)(jn * 16);
                if constexpr (GR) {
                    if (p.c_wt) store_wt(&Cl[off], cacc[i][jn][r]);
                    else Cl[off] = cacc[i][jn][r];
                } else if (p.c_wt) store_wt(&Cl[off], finish<KIND>(acc[i][jn][r]));
                else Cl[off] = finish<KIND>(acc[i][jn][r]);
            }
        }
}

template <int KIND, int BM, int BN, int KS, bool AL, int RC = 0>
__global__ __launch_bounds__(1024) void k_tiled2(orkh_mm p, int mtiles, int ntiles_all, int kbs, void *ws) {
    tiled2_body<KIND, BM, BN, KS, 0, AL, RC>(p, mtiles, ntiles_all, kbs, ws, T2Group{0, nullptr, nullptr},
                                             (int)blockIdx.x, (int)gridDim.x);
}

// k_tiled2m: up to ORKH_TGROUP_MAX matmuls of one kind, M and K in one launch (the multi-matmul submit): task t's
// tiles are workgroups [wg0[t], wg0[t] + tiles), each start a multiple of 8; the padding workgroups before the next
// start exit at once.
struct T2Multi {
    int n;
    int wg0[ORKH_TGROUP_MAX];
    int mtiles[ORKH_TGROUP_MAX], tiles[ORKH_TGROUP_MAX];
    orkh_mm p[ORKH_TGROUP_MAX];
};
template <int KIND, int BM, int BN, int KS, bool AL>
__global__ __launch_bounds__(1024) void k_tiled2m(T2Multi g) {
    int t = 0;
    while (t + 1 < g.n && (int)blockIdx.x >= g.wg0[t + 1]) t++;
    const int local = (int)blockIdx.x - g.wg0[t];
    if (local >= g.tiles[t]) return;
    tiled2_body<KIND, BM, BN, KS, 0, AL>(g.p[t], g.mtiles[t], g.tiles[t], g.p[t].KB, nullptr, T2Group{0, nullptr, nullptr},
                                         local, g.tiles[t]);
}

// Grouped runs (never K-split: the groups close in order inside one workgroup). GR 2: every group is whole
// K-blocks (G % KPB == 0), so the stage runs as in the plain kernel and a group closes after the K-block that ends
// it; GR 1: any G % 32 == 0, walked K-block by K-block with a group test per MFMA step.
template <int KIND, int BM, int BN, int KS, int GR, bool AL>
__global__ __launch_bounds__(1024) void k_tiled2g(orkh_mm p, int mtiles, int ntiles_all, T2Group gp) {
    tiled2_body<KIND, BM, BN, KS, GR, AL>(p, mtiles, ntiles_all, p.KB, nullptr, gp, (int)blockIdx.x, (int)gridDim.x);
}

// Dynamic LDS of k_tiled: KG groups x 2 stage buffers of A fragments, or (KG > 1) the 4-wave partial
// tile parked for the final cross-group sum, whichever is larger.
template <int KIND, int BM, int BN, int KS, int KG>
constexpr size_t tiled_lds_bytes() {
    const size_t stages = (size_t)KG * 2 * (BM / 16) * KS * KT<KIND>::STEPS * 1024;
    const size_t red = KG > 1 ? (size_t)4 * (BM / 32) * (BN / 32) * 64 * 16 : 0;
    return stages > red ? stages : red;
}

// k_tiled: one workgroup per BM x BN output tile, KG groups of 4 waves (2 x 2 over the tile). The
// groups split K stage by stage (group g takes stages g, g+KG, ...) and sum their partial tiles through
// LDS at the end; with KG = 2 each SIMD runs two waves, which the MFMA pipe needs to issue near peak.
// Per stage (KS panel K-blocks) and group:
//   A fragments (BM rows) are loaded cooperatively and staged through a double-buffered LDS region,
//   since all four waves read them;
//   B blocks go straight from HBM/L2 into the registers of the waves that use them (they are already
//   MFMA fragments in the panel layout), so weights never touch LDS.
// Both operands run D stages ahead through a ring of register slots (stage t in slot t % D); one
// barrier per stage. Loads are raw buffer loads: rows >= M, k >= K and stages past the end read 0
// through the hardware range check (no clamps, no selects, no faults).
// Split K (shapes with too few tiles to fill the CUs): the grid holds ntiles x ksplit workgroups; the
// one mapped to (tile, ks) covers K-blocks [ks*kbs, ks*kbs + kbs) and writes its partial tile to ws,
// summed afterwards by k_splitk_reduce in fixed order.
template <int KIND, int BM, int BN, int KS, int D, int KG>
__global__ __launch_bounds__(256 * KG) void k_tiled(orkh_mm p, int mtiles, int ntiles_all, int kbs, void *ws) {
    using T = KT<KIND>;
    typedef typename T::acc_t acc_t;
    constexpr int MB = BM / 16, NBK = BN / 16;
    constexpr int MTW = MB / 2, NTW = NBK / 2;
    constexpr int AF = MB * KS * T::STEPS;  // A fragments (1 KiB) per stage
    constexpr int AV = AF * 64 / 256;       // A fragment entries per thread per stage
    constexpr int STG = AF * 64;            // v4i per LDS stage buffer
    constexpr int KSPAN = KS * T::KPB;      // k per stage
    static_assert(MB % 2 == 0 && NBK % 2 == 0 && (AF * 64) % 256 == 0, "tile must split over 2x2 waves");
    extern __shared__ v4i lds_dyn[];  // tiled_lds_bytes<...>(): the stage buffers, or the reduction tile

    const int grp = threadIdx.x >> 8;
    const int tid = threadIdx.x & 255, lane = tid & 63, wv = tid >> 6;
    const int wm = wv & 1, wn = wv >> 1;
    v4i *lds = lds_dyn + grp * 2 * STG;
    // XCD-aware order: WG b runs on XCD b%8; each XCD gets a contiguous run of tiles, M fastest, so
    // every M-tile that reads a given B column panel shares one L2.
    const int nT = gridDim.x, bid = blockIdx.x;
    const int per = nT / 8, rem = nT % 8, x = bid % 8, j = bid / 8;
    const int tl = (x < rem) ? x * (per + 1) + j : rem * (per + 1) + (x - rem) * per + j;
    const int ks = tl / ntiles_all, tile = tl % ntiles_all;   // each XCD's run: one K range, M fastest
    const int m0 = (tile % mtiles) * BM;
    const int nb0 = (tile / mtiles) * NBK;
    const int NBtot = p.N / 16;
    const Lut L = {p.lut[0], p.lut[1], p.lut[2], p.lut[3]};
    const int kb_lo = ks * kbs, kb_hi = min(kb_lo + kbs, p.KB);   // this workgroup's K-blocks
    const int k_hi = min(kb_hi * T::KPB, p.K);

    const uint32_t lda_b = (uint32_t)p.lda * T::ESZ;
    const __amdgpu_buffer_rsrc_t Ar = make_rsrc(p.A, (uint32_t)p.M * lda_b);
    const __amdgpu_buffer_rsrc_t Br = make_rsrc(p.B, (uint32_t)NBtot * p.KB * 1024u);

    // Per-thread constant parts of every load: A entry i -> byte offset at stage 0 and its k within the
    // stage; B block jn of this wave -> byte offset at stage 0.
    uint32_t a_off[AV];
    int a_k[AV];
#pragma unroll
    for (int i = 0; i < AV; i++) {
        const int idx = i * 256 + tid, f = idx >> 6, ln = idx & 63;
        const int mb = f / (KS * T::STEPS), ksub = f % (KS * T::STEPS);
        const int kbl = ksub / T::STEPS, s = ksub % T::STEPS;
        const int row = m0 + mb * 16 + (ln & 15);
        a_k[i] = kbl * T::KPB + a_koff<KIND>(s, ln >> 4);
        a_off[i] = row < p.M ? (uint32_t)row * lda_b + (uint32_t)a_k[i] * T::ESZ : OOB;
    }
    uint32_t b_off[NTW];
#pragma unroll
    for (int jn = 0; jn < NTW; jn++) {
        const int nb = nb0 + wn * NTW + jn;
        b_off[jn] = nb < NBtot ? ((uint32_t)nb * p.KB * 64 + lane) * 16 : OOB;
    }

    v4i ra[D][AV], rb[D][NTW][KS];
    // ls = this group's local stage; its global stage is ls * KG + grp.
    auto gload = [&](int ls, v4i (&xa)[AV], v4i (&xb)[NTW][KS]) {
        const int st = ls * KG + grp, k0 = kb_lo * T::KPB + st * KSPAN;
#pragma unroll
        for (int i = 0; i < AV; i++)
            xa[i] = bload(Ar, k0 + a_k[i] < k_hi ? a_off[i] + (uint32_t)k0 * T::ESZ : OOB);
#pragma unroll
        for (int kbl = 0; kbl < KS; kbl++) {
            const int kb = kb_lo + st * KS + kbl;
#pragma unroll
            for (int jn = 0; jn < NTW; jn++) xb[jn][kbl] = bload(Br, kb < kb_hi ? b_off[jn] + (uint32_t)kb * 1024u : OOB);
        }
    };
    auto lstore = [&](int buf, const v4i (&xa)[AV]) {
#pragma unroll
        for (int i = 0; i < AV; i++) lds[buf * STG + i * 256 + tid] = xa[i];
    };

    acc_t acc[MTW][NTW];
#pragma unroll
    for (int i = 0; i < MTW; i++)
#pragma unroll
        for (int jn = 0; jn < NTW; jn++) acc[i][jn] = acc_t{0, 0, 0, 0};

    auto compute = [&](int cur, const v4i (&xb)[NTW][KS]) {
        const v4i *sb = lds + cur * STG;
#pragma unroll
        for (int kbl = 0; kbl < KS; kbl++) {
            v4i op[NTW][T::STEPS];
#pragma unroll
            for (int jn = 0; jn < NTW; jn++) decode<KIND>(xb[jn][kbl], op[jn], L);
#pragma unroll
            for (int s = 0; s < T::STEPS; s++) {
#pragma unroll
                for (int i = 0; i < MTW; i++) {
                    const v4i a = sb[(((wm * MTW + i) * KS + kbl) * T::STEPS + s) * 64 + lane];
#pragma unroll
                    for (int jn = 0; jn < NTW; jn++) acc[i][jn] = mma(a, op[jn][s], acc[i][jn]);
                }
            }
        }
    };

    // Each group's stage count is rounded up to a multiple of D (the extra stages read zeros and add
    // nothing), so the ring has no branches and every wait is a partial vmcnt.
    const int nst = (kb_hi - kb_lo + KS - 1) / KS;
    const int nls = ((nst + KG - 1) / KG + D - 1) / D * D;
#pragma unroll
    for (int jd = 0; jd < D; jd++) gload(jd, ra[jd], rb[jd]);
    lstore(0, ra[0]);
    __syncthreads();
    for (int s0 = 0; s0 < nls; s0 += D) {
#pragma unroll
        for (int jd = 0; jd < D; jd++) {
            const int ls = s0 + jd;
            compute(ls & 1, rb[jd]);          // A of stage ls from LDS, B of stage ls from slot jd
            gload(ls + D, ra[jd], rb[jd]);    // slot jd is free again: refill it D stages ahead
            lstore((ls + 1) & 1, ra[(jd + 1) % D]);
            __syncthreads();
        }
    }

    if constexpr (KG == 2) {
        // Every stage buffer is idle after the loop's last barrier: group 1 parks its partial tile in
        // the LDS, group 0 adds it in.
        acc_t *red = (acc_t *)lds_dyn;
        if (grp == 1)
#pragma unroll
            for (int i = 0; i < MTW; i++)
#pragma unroll
                for (int jn = 0; jn < NTW; jn++) red[((wv * MTW + i) * NTW + jn) * 64 + lane] = acc[i][jn];
        __syncthreads();
        if (grp == 1) return;
#pragma unroll
        for (int i = 0; i < MTW; i++)
#pragma unroll
            for (int jn = 0; jn < NTW; jn++) acc[i][jn] += red[((wv * MTW + i) * NTW + jn) * 64 + lane];
    }

    typedef typename T::c_t c_t;
    const bool split = gridDim.x > ntiles_all;
    c_t *C = split ? (c_t *)ws + (size_t)ks * p.M * p.N : (c_t *)p.C;
    const size_t ldc = split ? (size_t)p.N : (size_t)p.ldc;
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
                if (m < p.M) C[(size_t)m * ldc + n] = finish<KIND>(acc[i][jn][r]);
            }
        }
}

// ------------------------------------------------------------------------------------------------
thread_local char g_lerr[256];

template <int KIND, int WPG>
int launch_gemv_v(const orkh_mm *p, const orkh_plan *q, hipStream_t s) {
    constexpr int KU = (KIND == ORKH_I4U || KIND == ORKH_NF4) ? 4 : 8;
    dim3 grid(p->N / 16, q->ksplit), block(WPG * 64);
    hipLaunchKernelGGL((k_gemv<KIND, WPG, KU>), grid, block, 0, s, *p, q->kbw, q->kbs, q->ksplit, q->ws);
    return 0;
}

template <int KIND>
int launch_gemv(const orkh_mm *p, const orkh_plan *q, hipStream_t s) {
    if (p->M != 1) {
        snprintf(g_lerr, sizeof g_lerr, "gemv plan: M=%d (needs 1)", p->M);
        return -2;
    }
    if (q->half && ((uintptr_t)p->A & 15) == 0) {
        // NI: load instructions per batch (two blocks each), the smallest instantiated count that covers the run
        // (every count up to 8 on 8 waves, where the planner's runs are 5-16 blocks; 1-4 and 8 on 2 or 4 waves)
        const int need = (q->kbw + 1) / 2;
        if ((q->wpg != 2 && q->wpg != 4 && q->wpg != 8) || q->kbw < 1 || (p->N & 15)) {
            snprintf(g_lerr, sizeof g_lerr, "gemv half plan: wpg=%d kbw=%d N=%d unsupported", q->wpg, q->kbw, p->N);
            return -2;
        }
        dim3 grid(p->N / 8, q->ksplit), block(q->wpg * 64);
#define ORKH_GH(W_, N_) hipLaunchKernelGGL((k_gemv_half<KIND, W_, N_>), grid, block, 0, s, *p, q->kbw, q->kbs, q->ksplit, q->ws)
        if (q->wpg == 8) {
            switch (need < 8 ? need : 8) {
            case 1: ORKH_GH(8, 1); break;
            case 2: ORKH_GH(8, 2); break;
            case 3: ORKH_GH(8, 3); break;
            case 4: ORKH_GH(8, 4); break;
            case 5: ORKH_GH(8, 5); break;
            case 6: ORKH_GH(8, 6); break;
            case 7: ORKH_GH(8, 7); break;
            default: ORKH_GH(8, 8); break;
            }
        } else if (q->wpg == 4) {
            if (need <= 1) ORKH_GH(4, 1);
            else if (need <= 2) ORKH_GH(4, 2);
            else if (need <= 3) ORKH_GH(4, 3);
            else if (need <= 4) ORKH_GH(4, 4);
            else ORKH_GH(4, 8);
        } else {
            if (need <= 1) ORKH_GH(2, 1);
            else if (need <= 2) ORKH_GH(2, 2);
            else if (need <= 3) ORKH_GH(2, 3);
            else if (need <= 4) ORKH_GH(2, 4);
            else ORKH_GH(2, 8);
        }
#undef ORKH_GH
        return 0;
    }
    if (q->half) {
        // A not 16-byte aligned (the half kernel loads activations 16 bytes at a time): whole panels, same K split
        orkh_plan w = *q;
        w.wpg = q->wpg == 8 ? 8 : 4;
        w.kbw = (q->kbs + w.wpg - 1) / w.wpg;
        return w.wpg == 8 ? launch_gemv_v<KIND, 8>(p, &w, s) : launch_gemv_v<KIND, 4>(p, &w, s);
    }
    if (q->wpg == 8) return launch_gemv_v<KIND, 8>(p, q, s);
    if (q->wpg == 4) return launch_gemv_v<KIND, 4>(p, q, s);
    snprintf(g_lerr, sizeof g_lerr, "gemv plan: wpg=%d unsupported", q->wpg);
    return -2;
}

template <int KIND, int MT, int WPG>
int launch_stream_v(const orkh_mm *p, const orkh_plan *q, hipStream_t s) {
    constexpr int KU = (KIND == ORKH_I4U || KIND == ORKH_NF4) ? 4 : 8;
    dim3 grid(p->N / 16, q->ksplit), block(WPG * 64);
    if (q->half) {
        if (q->np == 2) {
            snprintf(g_lerr, sizeof g_lerr, "stream plan: half panels and paired panels exclude each other");
            return -2;
        }
        hipLaunchKernelGGL((k_stream<KIND, MT, WPG, KU, 1, 1>), dim3(p->N / 8, q->ksplit), block, 0, s, *p, q->kbw, q->kbs,
                           q->ksplit, q->ws);
        return 0;
    }
    if (q->np == 2) {
        // paired panels are built for one or two row tiles only (acc[2][MT] and both panels' raw blocks in registers)
        if constexpr (MT <= 2) {
            const int NB = p->N / 16, G = q->npg;
            if (q->ksplit != 1 || G < (NB + 1) / 2 || G >= NB) {
                snprintf(g_lerr, sizeof g_lerr, "stream plan: paired panels need ksplit 1 and N/32 <= %d < N/16", G);
                return -2;
            }
            hipLaunchKernelGGL((k_stream<KIND, MT, WPG, KU, 2>), dim3(G, 1), block, 0, s, *p, q->kbw, q->kbs, 1, q->ws);
            return 0;
        } else {
            snprintf(g_lerr, sizeof g_lerr, "stream plan: paired panels need mt <= 2 (got %d)", MT);
            return -2;
        }
    }
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

// Raise a kernel's dynamic-LDS limit once per (kernel, device): hipFuncSetAttribute holds per device, so the
// flags are per device, and atomic, since contexts may launch from several threads.
constexpr int ORKH_MAX_DEV = 64;
typedef std::atomic<bool> lds_flags[ORKH_MAX_DEV];
inline int lds_limit(const void *kern, int bytes, lds_flags &done) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= ORKH_MAX_DEV) {
        snprintf(g_lerr, sizeof g_lerr, "LDS limit: no current device below %d", ORKH_MAX_DEV);
        return -1;
    }
    if (done[dev].load(std::memory_order_acquire)) return 0;
    const hipError_t e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e != hipSuccess) {
        snprintf(g_lerr, sizeof g_lerr, "hipFuncSetAttribute(%d B of LDS): %s", bytes, hipGetErrorString(e));
        return -1;
    }
    done[dev].store(true, std::memory_order_release);
    return 0;
}

template <int KIND, int BM, int BN>
int launch_tiled_v(const orkh_mm *p, const orkh_plan *q, hipStream_t s) {
    constexpr int KS = 1;
    constexpr int D = (KIND == ORKH_I4U || KIND == ORKH_NF4) ? 3 : 4;
    constexpr int KG = 2;
    constexpr size_t lds = tiled_lds_bytes<KIND, BM, BN, KS, KG>();
    auto kern = k_tiled<KIND, BM, BN, KS, D, KG>;
    static lds_flags attr; // per instantiation: allow more than the default 64 KiB of dynamic LDS
    if (lds_limit((const void *)kern, (int)lds, attr)) return -1;
    const int mtiles = (p->M + BM - 1) / BM;
    const int ntiles = (p->N / 16 + BN / 16 - 1) / (BN / 16);
    const int ksplit = q->ksplit > 1 ? q->ksplit : 1;
    const int kbs = ksplit > 1 ? q->kbs : p->KB;
    hipLaunchKernelGGL(kern, dim3(mtiles * ntiles * ksplit), dim3(256 * KG), lds, s, *p, mtiles, mtiles * ntiles, kbs,
                       q->ws);
    return 0;
}

// K-blocks per stage of k_tiled2: ~128 bytes of each activation row per stage for small tiles, ~64 for the
// 256 x 256 tile (whose ring would not fit otherwise); at least one per K group of waves.
template <int KIND, int BM, int BN, int XG = 0> constexpr int t2_ks() {
    constexpr int mb = XG ? 2 : (BM / 16 < 4 ? BM / 16 : 4), nb = XG == 2 ? 2 : t2_wn(BN / 16), wk = 16 / (mb * nb);
    constexpr int base = (KIND == ORKH_I4U || KIND == ORKH_NF4) ? 1 : (BM * BN >= 65536 ? 1 : 2);
    return base > wk ? base : wk;
}

template <int KIND, int BM, int BN, int RC>
int launch_tiled2_r(const orkh_mm *p, const orkh_plan *q, hipStream_t s);

// Two-slot ring (plan.ring == 2): for the tiles whose ring of up to 4 slots holds the CU's LDS for one workgroup, a
// ring of two fits two workgroups on a CU, so on a grid of several rounds one's set-up and epilogue overlap the other's
// loop. Not built for NF4 (its decode runs a stage ahead and needs 3 slots).
template <int KIND, int BM, int BN, int XG, int KS>
constexpr bool t2_ring2_ok() {
    return KIND != ORKH_NF4 && T2<KIND, BM, BN, KS, XG>::LDS > 81920 && T2<KIND, BM, BN, KS, XG, 2>::LDS <= 81920;
}

template <int KIND, int BM, int BN>
int launch_tiled2_v(const orkh_mm *p, const orkh_plan *q, hipStream_t s) {
    constexpr int XG = t2_xg<KIND, BM, BN, 0>();
    constexpr int KS = t2_ks<KIND, BM, BN, XG>();
    if (q->ring == 2) {
        if constexpr (t2_ring2_ok<KIND, BM, BN, XG, KS>()) return launch_tiled2_r<KIND, BM, BN, 2>(p, q, s);
        snprintf(g_lerr, sizeof g_lerr, "tiled2 plan: no two-slot ring for %dx%d of this kind", BM, BN);
        return -2;
    }
    return launch_tiled2_r<KIND, BM, BN, 0>(p, q, s);
}

template <int KIND, int BM, int BN, int RC>
int launch_tiled2_r(const orkh_mm *p, const orkh_plan *q, hipStream_t s) {
    constexpr int XG = t2_xg<KIND, BM, BN, 0>();
    constexpr int KS = t2_ks<KIND, BM, BN, XG>();
    using P = T2<KIND, BM, BN, KS, XG, RC>;
    const bool al = q->aline && P::LINE_OK;
    auto kern = al ? k_tiled2<KIND, BM, BN, KS, true, RC> : k_tiled2<KIND, BM, BN, KS, false, RC>;
    static lds_flags attr[2]; // per instantiation: allow more than the default 64 KiB of dynamic LDS
    if (lds_limit((const void *)kern, (int)P::LDS, attr[al])) return -1;
    const int mtiles = (p->M + BM - 1) / BM;
    const int ntiles = (p->N / 16 + P::NB - 1) / P::NB;
    const int ksplit = q->ksplit > 1 ? q->ksplit : 1;
    const int kbs = ksplit > 1 ? q->kbs : p->KB;
    if ((long)mtiles * ntiles * ksplit >= (1L << 24)) { // the kernel's tile-index division is exact below 2^24
        snprintf(g_lerr, sizeof g_lerr, "tiled2: %ld workgroups", (long)mtiles * ntiles * ksplit);
        return -2;
    }
    orkh_mm pc = *p;
    pc.c_wt = q->cwt;
    hipLaunchKernelGGL(kern, dim3(mtiles * ntiles * ksplit), dim3(1024), P::LDS, s, pc, mtiles, mtiles * ntiles, kbs,
                       q->ws);
    return 0;
}

template <int KIND, int BM, int BN>
int launch_tiled2m_v(T2Multi &g, const orkh_plan *q, hipStream_t s) {
    constexpr int XG = t2_xg<KIND, BM, BN, 0>();
    constexpr int KS = t2_ks<KIND, BM, BN, XG>();
    using P = T2<KIND, BM, BN, KS, XG>;
    const bool al = q->aline && P::LINE_OK;
    auto kern = al ? k_tiled2m<KIND, BM, BN, KS, true> : k_tiled2m<KIND, BM, BN, KS, false>;
    static lds_flags attr[2];
    if (lds_limit((const void *)kern, (int)P::LDS, attr[al])) return -1;
    long wg = 0;
    for (int t = 0; t < g.n; t++) {
        const orkh_mm &p = g.p[t];
        g.mtiles[t] = (p.M + BM - 1) / BM;
        g.tiles[t] = g.mtiles[t] * ((p.N / 16 + P::NB - 1) / P::NB);
        g.wg0[t] = (int)wg;
        wg += ((long)g.tiles[t] + 7) / 8 * 8;
    }
    if (wg >= (1L << 24)) {
        snprintf(g_lerr, sizeof g_lerr, "tiled2 group: %ld workgroups", wg);
        return -2;
    }
    hipLaunchKernelGGL(kern, dim3((unsigned)wg), dim3(1024), P::LDS, s, g);
    return 0;
}

template <int KIND>
int launch_tiled2m(T2Multi &g, const orkh_plan *q, hipStream_t s) {
    if (q->bm == 256 && q->bn == 256) return launch_tiled2m_v<KIND, 256, 256>(g, q, s);
    if (q->bm == 128 && q->bn == 128) return launch_tiled2m_v<KIND, 128, 128>(g, q, s);
    if (q->bm == 128 && q->bn == 96) return launch_tiled2m_v<KIND, 128, 96>(g, q, s);
    if (q->bm == 64 && q->bn == 192) return launch_tiled2m_v<KIND, 64, 192>(g, q, s);
    if (q->bm == 64 && q->bn == 64) return launch_tiled2m_v<KIND, 64, 64>(g, q, s);
    if (q->bm == 32 && q->bn == 64) return launch_tiled2m_v<KIND, 32, 64>(g, q, s);
    if (q->bm == 32 && q->bn == 32) return launch_tiled2m_v<KIND, 32, 32>(g, q, s);
    if (q->bm == 16 && q->bn == 64) return launch_tiled2m_v<KIND, 16, 64>(g, q, s);
    if (q->bm == 16 && q->bn == 32) return launch_tiled2m_v<KIND, 16, 32>(g, q, s);
    snprintf(g_lerr, sizeof g_lerr, "tiled2 group plan: %dx%d unsupported", q->bm, q->bn);
    return -2;
}

template <int KIND>
int launch_tiled(const orkh_mm *p, const orkh_plan *q, hipStream_t s) {
    if (q->ksplit > 1 && (!q->ws || (long)q->ksplit * q->kbs < p->KB)) {
        snprintf(g_lerr, sizeof g_lerr, "tiled plan: ksplit=%d kbs=%d does not cover KB=%d or has no ws", q->ksplit,
                 q->kbs, p->KB);
        return -2;
    }
    if (q->algo == ORKH_ALGO_TILED2) {
        if (q->bm == 256 && q->bn == 256) return launch_tiled2_v<KIND, 256, 256>(p, q, s);
        if (q->bm == 128 && q->bn == 128) return launch_tiled2_v<KIND, 128, 128>(p, q, s);
        if (q->bm == 128 && q->bn == 96) return launch_tiled2_v<KIND, 128, 96>(p, q, s);
        if (q->bm == 64 && q->bn == 192) return launch_tiled2_v<KIND, 64, 192>(p, q, s);
        if (q->bm == 64 && q->bn == 64) return launch_tiled2_v<KIND, 64, 64>(p, q, s);
        if (q->bm == 32 && q->bn == 64) return launch_tiled2_v<KIND, 32, 64>(p, q, s);
        if (q->bm == 32 && q->bn == 32) return launch_tiled2_v<KIND, 32, 32>(p, q, s);
        if (q->bm == 16 && q->bn == 64) return launch_tiled2_v<KIND, 16, 64>(p, q, s);
        if (q->bm == 16 && q->bn == 32) return launch_tiled2_v<KIND, 16, 32>(p, q, s);
        snprintf(g_lerr, sizeof g_lerr, "tiled2 plan: %dx%d unsupported", q->bm, q->bn);
        return -2;
    }
    if (q->bm == 128 && q->bn == 96) return launch_tiled_v<KIND, 128, 96>(p, q, s);
    if (q->bm == 128 && q->bn == 128) return launch_tiled_v<KIND, 128, 128>(p, q, s);
    if (q->bm == 64 && q->bn == 64) return launch_tiled_v<KIND, 64, 64>(p, q, s);
    snprintf(g_lerr, sizeof g_lerr, "tiled plan: %dx%d unsupported", q->bm, q->bn);
    return -2;
}

}  // namespace

extern "C" const char *orkh_launch_error(void) { return g_lerr; }

extern "C" int orkh_mm_launch(const orkh_mm *p, const orkh_plan *q, void *stream) {
    hipStream_t s = (hipStream_t)stream;
    g_lerr[0] = 0;
    int rc;
    if (q->algo == ORKH_ALGO_GEMV) {
        switch (p->kind) {
        case ORKH_I8: rc = launch_gemv<ORKH_I8>(p, q, s); break;
        case ORKH_I4U: rc = launch_gemv<ORKH_I4U>(p, q, s); break;
        case ORKH_NF4: rc = launch_gemv<ORKH_NF4>(p, q, s); break;
        case ORKH_F16: rc = launch_gemv<ORKH_F16>(p, q, s); break;
        default: rc = -2;
        }
        if (rc == 0 && q->ksplit > 1) {
            dim3 grid((unsigned)((p->N + 255) / 256)), block(256);
            if (p->kind == ORKH_F16)
                hipLaunchKernelGGL(k_splitk_reduce<float>, grid, block, 0, s, (const float *)q->ws, (float *)p->C,
                                   1, p->N, p->ldc, q->ksplit);
            else
                hipLaunchKernelGGL(k_splitk_reduce<int32_t>, grid, block, 0, s, (const int32_t *)q->ws,
                                   (int32_t *)p->C, 1, p->N, p->ldc, q->ksplit);
        }
    } else if (q->algo == ORKH_ALGO_STREAM) {
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
    }
    if (rc) return rc;
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        snprintf(g_lerr, sizeof g_lerr, "launch: %s", hipGetErrorString(e));
        return -1;
    }
    return 0;
}

extern "C" int orkh_mm_launch_tgroup(const orkh_mm *p, int n, const orkh_plan *q, void *stream) {
    g_lerr[0] = 0;
    if (n < 2 || n > ORKH_TGROUP_MAX || !p || !q || q->algo != ORKH_ALGO_TILED2 || q->ksplit > 1) {
        snprintf(g_lerr, sizeof g_lerr, "tiled2 group: n=%d or plan (algo %d, ksplit %d) unsupported", n, q ? q->algo : -1,
                 q ? q->ksplit : 0);
        return -2;
    }
    T2Multi g;
    memset(&g, 0, sizeof g);
    g.n = n;
    for (int t = 0; t < n; t++) {
        if (p[t].kind != p[0].kind || p[t].M != p[0].M || p[t].K != p[0].K || p[t].KB != p[0].KB || p[t].M < 1 ||
            (p[t].N & 15) || p[t].N < 16) {
            snprintf(g_lerr, sizeof g_lerr, "tiled2 group: task %d differs in kind, M or K, or has N=%d", t, p[t].N);
            return -2;
        }
        g.p[t] = p[t];
    }
    hipStream_t s = (hipStream_t)stream;
    int rc;
    switch (p[0].kind) {
    case ORKH_I8: rc = launch_tiled2m<ORKH_I8>(g, q, s); break;
    case ORKH_I4U: rc = launch_tiled2m<ORKH_I4U>(g, q, s); break;
    case ORKH_NF4: rc = launch_tiled2m<ORKH_NF4>(g, q, s); break;
    case ORKH_F16: rc = launch_tiled2m<ORKH_F16>(g, q, s); break;
    default: snprintf(g_lerr, sizeof g_lerr, "tiled2 group: kind %d", p[0].kind); return -2;
    }
    if (rc) return rc;
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        snprintf(g_lerr, sizeof g_lerr, "launch: %s", hipGetErrorString(e));
        return -1;
    }
    return 0;
}

extern "C" int orkh_mm_launch_group(const orkh_group *g, int wpg, void *stream) {
    hipStream_t s = (hipStream_t)stream;
    g_lerr[0] = 0;
    if (g->n < 1 || g->n > ORKH_GROUP_MAX) {
        snprintf(g_lerr, sizeof g_lerr, "group: n=%d", g->n);
        return -2;
    }
    int wgs = 0;
    for (int i = 0; i < g->n; i++) {
        const orkh_mm &p = g->t[i].p;
        if (p.kind != g->t[0].p.kind || p.M != 1 || g->t[i].wg0 != wgs || (long)g->t[i].kbw * wpg < p.KB) {
            snprintf(g_lerr, sizeof g_lerr, "group: task %d inconsistent (kind %d M %d wg0 %d kbw %d)", i, p.kind, p.M,
                     g->t[i].wg0, g->t[i].kbw);
            return -2;
        }
        wgs += p.N / 16;
    }
    dim3 grid(wgs), block(wpg * 64);
#define ORKH_GROUP_CASE(KIND, KU)                                                                    \
    if (wpg == 4) hipLaunchKernelGGL((k_gemv_group<KIND, 4, KU>), grid, block, 0, s, *g);            \
    else if (wpg == 8) hipLaunchKernelGGL((k_gemv_group<KIND, 8, KU>), grid, block, 0, s, *g);       \
    else { snprintf(g_lerr, sizeof g_lerr, "group: wpg=%d unsupported", wpg); return -2; }
    switch (g->t[0].p.kind) {
    case ORKH_I8: ORKH_GROUP_CASE(ORKH_I8, 8) break;
    case ORKH_I4U: ORKH_GROUP_CASE(ORKH_I4U, 4) break;
    case ORKH_NF4: ORKH_GROUP_CASE(ORKH_NF4, 4) break;
    case ORKH_F16: ORKH_GROUP_CASE(ORKH_F16, 8) break;
    default: snprintf(g_lerr, sizeof g_lerr, "group: kind %d", g->t[0].p.kind); return -2;
    }
#undef ORKH_GROUP_CASE
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        snprintf(g_lerr, sizeof g_lerr, "launch: %s", hipGetErrorString(e));
        return -1;
    }
    return 0;
}

namespace {
// Stage depth of a grouped run whose groups are whole K-blocks: the plain kernel's, except for uniform int4, whose
// one-K-block stages (12 KiB on 64 x 64, whose plain runs take four K-blocks on the 2 x 2 x 4 wave grid that grouped
// runs cannot use) keep too few bytes in flight per CU: four K-blocks on 64 x 64, two on 64 x 192, or two, or the plain
// depth, where the larger ring and the tile's scales do not fit the LDS together. Measured against one K-block
// (graph-timed, us, W4A4 K=N=4096 unless given): 64 x 64 G=128 M=256 20.11 -> 18.54, M=128 19.72 -> 18.10, G=256
// 17.34 -> 15.65, K=8192 G=128 (two K-blocks) 36.49 -> 33.11; 64 x 192 M=512 35.79 -> 35.17, K=2048 N=6144 M=256
// 19.83 -> 19.48. With groups inside a K-block (GR 1) two K-blocks measured slower (G=64 34.88 -> 35.34), so those
// keep the plain depth.
template <int KIND, int BM, int BN> constexpr int t2g_ks() {
    return KIND != ORKH_I4U ? t2_ks<KIND, BM, BN>() : BN == 64 ? 4 : 2;
}

template <int KIND, int BM, int BN, int KS>
int launch_tiled2g_k(const orkh_mm *p, const T2Group &gp, hipStream_t s, size_t sc, bool aline) {
    using P = T2<KIND, BM, BN, KS>;
    const bool whole = gp.G % KT<KIND>::KPB == 0;
    const bool al = aline && P::LINE_OK;
    auto kern = whole ? (al ? k_tiled2g<KIND, BM, BN, KS, 2, true> : k_tiled2g<KIND, BM, BN, KS, 2, false>)
                      : (al ? k_tiled2g<KIND, BM, BN, KS, 1, true> : k_tiled2g<KIND, BM, BN, KS, 1, false>);
    const size_t lds = P::LDS + sc;
    const int Sk = p->K / gp.G;
    if (lds > 163840) {
        snprintf(g_lerr, sizeof g_lerr, "grouped tiled2 %dx%d: %d groups need %zu B of LDS", BM, BN, Sk, lds);
        return -2;
    }
    static lds_flags attr[2][2]; // per instantiation: allow up to 160 KiB of dynamic LDS
    if (lds_limit((const void *)kern, 163840, attr[whole][al])) return -1;
    const int mtiles = (p->M + BM - 1) / BM;
    const int ntiles = (p->N / 16 + P::NB - 1) / P::NB;
    if ((long)mtiles * ntiles >= (1L << 24)) { // the kernel's tile-index division is exact below 2^24
        snprintf(g_lerr, sizeof g_lerr, "grouped tiled2: %ld workgroups", (long)mtiles * ntiles);
        return -2;
    }
    hipLaunchKernelGGL(kern, dim3(mtiles * ntiles), dim3(1024), lds, s, *p, mtiles, mtiles * ntiles, gp);
    return 0;
}

template <int KIND, int BM, int BN>
int launch_tiled2g_v(const orkh_mm *p, const T2Group &gp, hipStream_t s, bool al) {
    const int Sk = p->K / gp.G;
    const size_t sc = (size_t)((BM * Sk * 4 + 1023) / 1024 + (Sk * BN * 4 + 1023) / 1024) * 1024; // the tile's scales
    constexpr int KD = t2g_ks<KIND, BM, BN>(), K1 = t2_ks<KIND, BM, BN>();
    const bool whole = gp.G % KT<KIND>::KPB == 0;
    if constexpr (KD != K1) {
        if (whole && T2<KIND, BM, BN, KD>::LDS + sc <= 163840) return launch_tiled2g_k<KIND, BM, BN, KD>(p, gp, s, sc, al);
    }
    if constexpr (KD > 2 && K1 < 2) {
        if (whole && T2<KIND, BM, BN, 2>::LDS + sc <= 163840) return launch_tiled2g_k<KIND, BM, BN, 2>(p, gp, s, sc, al);
    }
    return launch_tiled2g_k<KIND, BM, BN, K1>(p, gp, s, sc, al);
}

template <int KIND>
int launch_tiled2g(const orkh_mm *p, const orkh_plan *q, const T2Group &gp, hipStream_t s) {
    if (q->bm == 64 && q->bn == 192) return launch_tiled2g_v<KIND, 64, 192>(p, gp, s, q->aline);
    if (q->bm == 64 && q->bn == 64) return launch_tiled2g_v<KIND, 64, 64>(p, gp, s, q->aline);
    snprintf(g_lerr, sizeof g_lerr, "grouped tiled2 plan: %dx%d unsupported", q->bm, q->bn);
    return -2;
}
} // namespace

extern "C" int orkh_tiled2_ring2_ok(int kind, int bm, int bn) {
#define ORKH_RING2(KIND)                                                                                     \
    if (bm == 128 && bn == 128) return (int)t2_ring2_ok<KIND, 128, 128, t2_xg<KIND, 128, 128, 0>(),            \
                                                        t2_ks<KIND, 128, 128, t2_xg<KIND, 128, 128, 0>()>()>(); \
    if (bm == 128 && bn == 96) return (int)t2_ring2_ok<KIND, 128, 96, t2_xg<KIND, 128, 96, 0>(),               \
                                                       t2_ks<KIND, 128, 96, t2_xg<KIND, 128, 96, 0>()>()>();    \
    if (bm == 64 && bn == 192) return (int)t2_ring2_ok<KIND, 64, 192, t2_xg<KIND, 64, 192, 0>(),               \
                                                       t2_ks<KIND, 64, 192, t2_xg<KIND, 64, 192, 0>()>()>();    \
    return 0;
    switch (kind) {
    case ORKH_I8: ORKH_RING2(ORKH_I8)
    case ORKH_I4U: ORKH_RING2(ORKH_I4U)
    case ORKH_F16: ORKH_RING2(ORKH_F16)
    default: return 0;
    }
#undef ORKH_RING2
}

extern "C" int orkh_tiled2_ring_lds(int kind, int bm, int bn) {
#define ORKH_RING(KIND)                                                                                      \
    if (bm == 64 && bn == 64) return (int)T2<KIND, 64, 64, t2_ks<KIND, 64, 64>()>::LDS;                       \
    if (bm == 64 && bn == 192) return (int)T2<KIND, 64, 192, t2_ks<KIND, 64, 192>()>::LDS;                    \
    if (bm == 128 && bn == 128) return (int)T2<KIND, 128, 128, t2_ks<KIND, 128, 128>()>::LDS;                 \
    if (bm == 128 && bn == 96) return (int)T2<KIND, 128, 96, t2_ks<KIND, 128, 96>()>::LDS;                    \
    if (bm == 256 && bn == 256) return (int)T2<KIND, 256, 256, t2_ks<KIND, 256, 256>()>::LDS;                 \
    return -1;
    switch (kind) {
    case ORKH_I8: ORKH_RING(ORKH_I8)
    case ORKH_I4U: ORKH_RING(ORKH_I4U)
    case ORKH_NF4: ORKH_RING(ORKH_NF4)
    case ORKH_F16: ORKH_RING(ORKH_F16)
    default: return -1;
    }
#undef ORKH_RING
}

extern "C" int orkh_mm_launch_grouped(const orkh_mm *p, const orkh_plan *q, int G, const float *aS, const float *bS,
                                      float *C, int ldc, void *stream) {
    g_lerr[0] = 0;
    hipStream_t s = (hipStream_t)stream;
    if (G < 32 || G % 32 || p->K % G || p->N % 16 || p->M < 1 || ldc < p->N ||
        (p->kind != ORKH_I8 && p->kind != ORKH_I4U && p->kind != ORKH_NF4) ||
        (q->algo == ORKH_ALGO_TILED2 && p->kind == ORKH_NF4)) {
        snprintf(g_lerr, sizeof g_lerr, "grouped: kind %d M %d K %d N %d G %d ldc %d algo %d", p->kind, p->M, p->K,
                 p->N, G, ldc, q->algo);
        return -2;
    }
    // the one-row kernel loads the activations 16 bytes at a time: a row that is not 16-byte aligned (a caller's
    // device pointer) takes the panel-streaming kernel, as the plain GEMV falls back to whole panels
    if (q->algo == ORKH_ALGO_GEMV && ((uintptr_t)p->A & 15) == 0) {
        const int need = (q->kbw + 1) / 2, ni = need <= 1 ? 1 : need <= 2 ? 2 : need <= 4 ? 4 : 8;
        if (p->M != 1 || p->K / G > ORKH_GGEMV_SK_MAX || q->kbw < 1 || (q->wpg != 2 && q->wpg != 4 && q->wpg != 8) ||
            (q->kbw * q->wpg < p->KB)) {
            snprintf(g_lerr, sizeof g_lerr, "grouped gemv: M %d K/G %d wpg %d kbw %d", p->M, p->K / G, q->wpg, q->kbw);
            return -2;
        }
        const dim3 grid((unsigned)(p->N / 8)), block(q->wpg * 64);
#define ORKH_GG(KIND, W_, N_) hipLaunchKernelGGL((k_grouped_gemv<KIND, W_, N_>), grid, block, 0, s, *p, G, aS, bS, C, q->kbw)
#define ORKH_GGW(KIND, W_) do { if (ni == 1) ORKH_GG(KIND, W_, 1); else if (ni == 2) ORKH_GG(KIND, W_, 2); \
                                else if (ni == 4) ORKH_GG(KIND, W_, 4); else ORKH_GG(KIND, W_, 8); } while (0)
#define ORKH_GGK(KIND) do { if (q->wpg == 2) ORKH_GGW(KIND, 2); else if (q->wpg == 4) ORKH_GGW(KIND, 4); \
                            else ORKH_GGW(KIND, 8); } while (0)
        switch (p->kind) {
        case ORKH_I8: ORKH_GGK(ORKH_I8); break;
        case ORKH_I4U: ORKH_GGK(ORKH_I4U); break;
        default: ORKH_GGK(ORKH_NF4); break;
        }
#undef ORKH_GGK
#undef ORKH_GGW
#undef ORKH_GG
    } else if (q->algo == ORKH_ALGO_TILED2) {
        orkh_mm pc = *p;
        pc.C = C;
        pc.ldc = ldc;
        pc.c_wt = q->cwt;
        const T2Group gp = {G, aS, bS};
        const int rc = p->kind == ORKH_I8 ? launch_tiled2g<ORKH_I8>(&pc, q, gp, s) : launch_tiled2g<ORKH_I4U>(&pc, q, gp, s);
        if (rc) return rc;
    } else {
        const int MT = p->M > 16 ? 4 : 1;
        const dim3 grid((unsigned)(p->N / 16), (unsigned)((p->M + 16 * MT - 1) / (16 * MT))), block(256);
#define ORKH_GROUPED_CASE(KIND)                                                                              \
    if (MT == 1) hipLaunchKernelGGL((k_grouped<KIND, 1>), grid, block, 0, s, *p, G, aS, bS, C, ldc);          \
    else hipLaunchKernelGGL((k_grouped<KIND, 4>), grid, block, 0, s, *p, G, aS, bS, C, ldc);
        switch (p->kind) {
        case ORKH_I8: ORKH_GROUPED_CASE(ORKH_I8) break;
        case ORKH_I4U: ORKH_GROUPED_CASE(ORKH_I4U) break;
        default: ORKH_GROUPED_CASE(ORKH_NF4) break;
        }
#undef ORKH_GROUPED_CASE
    }
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
    if (q->algo == ORKH_ALGO_GEMV)
        snprintf(b, sizeof b, "%s_%s_w%d_kbw%d_ks%d", q->half ? "gemvh" : "gemv", k, q->wpg, q->kbw, q->ksplit);
    else if (q->algo == ORKH_ALGO_STREAM)
        snprintf(b, sizeof b, "stream_%s_mt%d_w%d_kbw%d_ks%d%s", k, q->mt, q->wpg, q->kbw, q->ksplit,
                 q->np == 2 ? "_p2" : q->half ? "_h" : "");
    else if (q->ksplit > 1)
        snprintf(b, sizeof b, "%s_%s_%dx%d_ks%d%s%s", q->algo == ORKH_ALGO_TILED2 ? "tiled2" : "tiled", k, q->bm, q->bn,
                 q->ksplit, q->algo == ORKH_ALGO_TILED2 && q->aline ? "_al" : "",
                 q->algo == ORKH_ALGO_TILED2 && q->ring == 2 ? "_r2" : "");
    else
        snprintf(b, sizeof b, "%s_%s_%dx%d%s%s", q->algo == ORKH_ALGO_TILED2 ? "tiled2" : "tiled", k, q->bm, q->bn,
                 q->algo == ORKH_ALGO_TILED2 && q->aline ? "_al" : "", q->algo == ORKH_ALGO_TILED2 && q->ring == 2 ? "_r2" : "");
    return b;
}
