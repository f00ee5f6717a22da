// orkh_rowrun.hip -- the one-row run with a fused row prologue and column epilogue (orkh_row_launch, orkh.h), for
// gfx950. The library's counterpart of what a decode step does around each projection: the reference's harness
// prepares the activation row on the host, runs ork_i8_mm_run and uses the columns on the host
// (examples/bench.c:83-90 quantise / dequantise, :105-113 mm(), :128-145 the layer's norm, residual and SwiGLU).
// Here the row's RMSNorm and int8 quantisation run in every workgroup's prologue and the column's use in its
// epilogue, around the M = 1 GEMV on the resident panels (orkh.h layout), so one launch replaces three.
// Compiled with -ffp-contract=off: every product and sum rounds as written.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "orkh.h"
#include "orkh_rowops.h"

namespace {
using namespace orkr;

// k_gemv_row: one 16-column panel per workgroup (pair mode: the same columns of two weights), 8 waves splitting the
// panel's K-blocks, on the library's resident layout (lane l of a 1 KiB block holds 16 bytes of column l % 16,
// k-group l / 16); with H, half a panel per workgroup (8 columns, twice the workgroups: the bytes spread evenly
// over the CUs where whole panels would leave some CUs one panel and others two, or none). Around that GEMV:
//   prologue: the int8 row, built in LDS by every workgroup. RMSNORM: RMSNorm of the row, its sum of squares taken
//     as a 512-thread workgroup takes it (thread t holds elements t, t + 512, ...; block_sum), then the per-row
//     quant; elements past K add exact zeros, so any E >= K / 512 gives the same sums. QUANT: the per-row quant of
//     the row as orkr::quant_regs does it (the absmax is order-independent).
//     Each wave's weight blocks (PRE >= its share, no more: a load past the share would fetch another wave's
//     bytes again) are loaded once the row has arrived: their latency hides behind the reductions and the
//     quant, and the row's own loads do not queue behind them in the CU's memory pipeline (measured: issuing
//     them first delayed the row by 1-2 us).
//   epilogue on each column's exact int32 sum c: STORE C[n] = c; RESID x[n] += (c * s) * ws[n] (a residual add);
//     SWIGLU y[n] = silu(g) * u of the gate and up columns, silu(g) = g / (1 + exp(-g)).
// A separate kernel that prepares the row with orkh_rowops.h in the same element mapping gets the same row and scale,
// so such a sequence and this launch give the same results bit for bit.
typedef int v4i_t __attribute__((ext_vector_type(4)));

struct RowLut { uint32_t l0, l1, l2, l3; };
// One dword of NF4 codes -> the int8 codebook values of its low nibbles (lo) and of its high nibbles (hi):
// v_perm selects within the 8 bytes of two LUT words by the low 3 bits of each code, and a second v_perm takes
// that from the upper or the lower LUT half by the code's top bit.
__device__ inline void row_nf4_map8(uint32_t x, const RowLut &L, uint32_t &lo, uint32_t &hi) {
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
__device__ inline int row_dot(v4i_t raw, const int *__restrict__ a, int acc, const RowLut &L) {
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
                row_nf4_map8(xs[d], L, lo, hi);
            }
            acc = __builtin_amdgcn_sdot4(a[2 * d], (int)lo, acc, false);
            acc = __builtin_amdgcn_sdot4(a[2 * d + 1], (int)hi, acc, false);
        }
    }
    return acc;
}

constexpr int ROW_WAVES = 8; // 512 threads: the element mapping of the row operations

template <int PRO, int EPI, int KIND, int E, int PRE, int H>
__global__ __launch_bounds__(ROW_WAVES * 64) void k_gemv_row(orkh_row p) {
    __shared__ __align__(16) int8_t arow[ORKH_ROW_KMAX];
    __shared__ __align__(16) float red[16];
    __shared__ __align__(16) float redq[16];
    __shared__ int racc[ROW_WAVES][2][16];
    constexpr bool PAIR = EPI == ORKH_COL_SWIGLU;
    constexpr int KPB = KIND == 0 ? 64 : 128;
    // Every kernel argument in one batch of scalar loads behind one wait: left to itself the compiler issues them
    // where first used, three waits in a row before the first weight load (the Qwen3-shaped decoder's four row runs
    // per layer: 0.878 -> 0.851 ms per token, three alternations on one box)
    asm volatile("" ::"s"(p.K), "s"(p.KB), "s"(p.nt), "s"(p.nb[0]), "s"(p.nb[1]), "s"(p.nb[2]), "s"(p.B[0]),
                 "s"(p.B[1]), "s"(p.B[2]), "s"(p.row), "s"(p.nw), "s"(p.eps), "s"(p.ws0), "s"(p.ws1));
    asm volatile("" ::"s"(p.x), "s"(p.y), "s"(p.C[0]), "s"(p.C[1]), "s"(p.C[2]), "s"(p.as_out));
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
    const int kbw = (KB + ROW_WAVES - 1) / ROW_WAVES, kb0 = min(wv * kbw, KB), kb1 = min(kb0 + kbw, KB);
    const v4i_t *b0 = (const v4i_t *)p.B[t] + (size_t)pnl * KB * 64 + loff;
    const v4i_t *b1 = PAIR ? (const v4i_t *)p.B[1] + (size_t)pnl * KB * 64 + loff : b0;
    // ---- prologue: the int8 row in LDS
    float y[E], nw[E];
    load_row(y, p.row, K);
    if constexpr (PRO == ORKH_ROW_RMSNORM) load_row(nw, p.nw, K);
    float mx = 0.f, ss = 0.f;
    if constexpr (PRO == ORKH_ROW_RMSNORM) {
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
    if constexpr (PRO == ORKH_ROW_RMSNORM) {
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
            if (i < K) arow[i] = quant_elem(y[k], inv, as);
        }
        for (int i = K + (int)threadIdx.x; i < KB * KPB; i += (int)blockDim.x) arow[i] = 0;
    }
    if (blockIdx.x == 0 && threadIdx.x == 0 && p.as_out) *p.as_out = as;
    __syncthreads();

    // ---- the GEMV: the preloaded blocks, then any further ones of this wave
    const RowLut L = {p.lut[0], p.lut[1], p.lut[2], p.lut[3]};
    const int aoff = grp * (KPB / 4);
    int acc0 = 0, acc1 = 0;
    if constexpr (H) {
        // a lane whose block lies past the run (the second half of an odd run's last instruction) adds nothing
#pragma unroll
        for (int u = 0; u < PRE; u++) {
            const int blk = kb0 + 2 * u + sub;
            const bool ok = blk < kb1;
            const int *a = (const int *)(arow + min(blk, kb1 - 1) * KPB + aoff);
            const int d0 = row_dot<KIND>(r0[u], a, 0, L);
            acc0 += ok ? d0 : 0;
            if constexpr (PAIR) {
                const int d1 = row_dot<KIND>(r1[u], a, 0, L);
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
            const int d0 = row_dot<KIND>(s0, a, 0, L);
            acc0 += ok ? d0 : 0;
            if constexpr (PAIR) {
                const int d1 = row_dot<KIND>(s1, a, 0, L);
                acc1 += ok ? d1 : 0;
            }
        }
    } else {
#pragma unroll
        for (int u = 0; u < PRE; u++) {
            if (kb0 + u < kb1) {
                const int *a = (const int *)(arow + (kb0 + u) * KPB + aoff);
                acc0 = row_dot<KIND>(r0[u], a, acc0, L);
                if constexpr (PAIR) acc1 = row_dot<KIND>(r1[u], a, acc1, L);
            }
        }
        for (int kb = kb0 + PRE; kb < kb1; kb++) {
            const v4i_t s0 = __builtin_nontemporal_load(b0 + (size_t)kb * 64);
            v4i_t s1 = s0;
            if constexpr (PAIR) s1 = __builtin_nontemporal_load(b1 + (size_t)kb * 64);
            const int *a = (const int *)(arow + kb * KPB + aoff);
            acc0 = row_dot<KIND>(s0, a, acc0, L);
            if constexpr (PAIR) acc1 = row_dot<KIND>(s1, a, acc1, L);
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
    for (int w = 0; w < ROW_WAVES; w++) {
        c0 += racc[w][0][j];
        if constexpr (PAIR) c1 += racc[w][1][j];
    }
    if constexpr (KIND == 1) { // every block's partial is 16 x an integer
        c0 >>= 4;
        c1 >>= 4;
    }
    const int n = pnl * 16 + hh * 8 + j;
    if constexpr (EPI == ORKH_COL_STORE) {
        p.C[t][n] = c0;
    } else if constexpr (EPI == ORKH_COL_RESID) {
        p.x[n] = p.x[n] + ((float)c0 * as) * p.ws0[n];
    } else {
        const float gv = ((float)c0 * as) * p.ws0[n];
        const float uv = ((float)c1 * as) * p.ws1[n];
        p.y[n] = (gv / (1.0f + expf(-gv))) * uv;
    }
}

// The built combinations: RMSNORM + STORE (int8: a decoder's q/k/v), QUANT + RESID (int8 / uniform int4 / NF4: o and
// down), RMSNORM + SWIGLU (int8 / uniform int4 / NF4: gate/up pairs).
// E: row elements per thread, a bound of K / 512; PRE: the weight blocks per wave, a bound of its share (half panels,
// orkh_row.half: the load instructions of two half blocks each that cover it).
template <int PRO, int EPI, int KIND, int E>
void row_launch_pre(const orkh_row *p, int grid, int pre, hipStream_t s) {
    const dim3 b(ROW_WAVES * 64);
    if (p->half) {
        // load instructions (two half blocks each) covering the wave's share, every count up to ORKH_ROW_KMAX
        const int ni = (pre + 1) / 2, g2 = 2 * grid;
        if (ni <= 1) hipLaunchKernelGGL((k_gemv_row<PRO, EPI, KIND, E, 1, 1>), dim3(g2), b, 0, s, *p);
        else if (ni <= 2) hipLaunchKernelGGL((k_gemv_row<PRO, EPI, KIND, E, 2, 1>), dim3(g2), b, 0, s, *p);
        else if (ni <= 3) hipLaunchKernelGGL((k_gemv_row<PRO, EPI, KIND, E, 3, 1>), dim3(g2), b, 0, s, *p);
        else if (ni <= 4) hipLaunchKernelGGL((k_gemv_row<PRO, EPI, KIND, E, 4, 1>), dim3(g2), b, 0, s, *p);
        else if (ni <= 6) hipLaunchKernelGGL((k_gemv_row<PRO, EPI, KIND, E, 6, 1>), dim3(g2), b, 0, s, *p);
        else hipLaunchKernelGGL((k_gemv_row<PRO, EPI, KIND, E, 8, 1>), dim3(g2), b, 0, s, *p);
        return;
    }
    if (pre <= 4) hipLaunchKernelGGL((k_gemv_row<PRO, EPI, KIND, E, 4, 0>), dim3(grid), b, 0, s, *p);
    else if (pre <= 8) hipLaunchKernelGGL((k_gemv_row<PRO, EPI, KIND, E, 8, 0>), dim3(grid), b, 0, s, *p);
    else hipLaunchKernelGGL((k_gemv_row<PRO, EPI, KIND, E, 16, 0>), dim3(grid), b, 0, s, *p);
}
template <int PRO, int EPI, int KIND> int row_launch(const orkh_row *p, int grid, hipStream_t s) {
    const int e = (p->K + ROW_WAVES * 64 - 1) / (ROW_WAVES * 64), pre = (p->KB + ROW_WAVES - 1) / ROW_WAVES;
    if (e <= 4) row_launch_pre<PRO, EPI, KIND, 4>(p, grid, pre, s);
    else if (e <= 8) row_launch_pre<PRO, EPI, KIND, 8>(p, grid, pre, s);
    else if (e <= 12) row_launch_pre<PRO, EPI, KIND, 12>(p, grid, pre, s);
    else if (e <= 16) row_launch_pre<PRO, EPI, KIND, 16>(p, grid, pre, s);
    else return -2;
    return 0;
}

}  // namespace

extern "C" {

int orkh_row_launch(const orkh_row *p, void *stream) {
    const hipStream_t s_ = (hipStream_t)stream;
    if (p->kind < 0 || p->kind > 2 || p->epi < ORKH_COL_STORE || p->epi > ORKH_COL_SWIGLU) return -2;
    const int kpb = p->kind == 0 ? 64 : 128;
    const int pro = p->pro;
    if ((pro != ORKH_ROW_RMSNORM && pro != ORKH_ROW_QUANT) || (pro == ORKH_ROW_RMSNORM && !p->nw)) return -2;
    const int nt = p->epi == ORKH_COL_SWIGLU ? 2 : p->epi == ORKH_COL_RESID ? 1 : p->nt;
    if (p->K < 32 || p->KB < 1 || (long)p->KB * kpb < p->K || (long)p->KB * kpb > ORKH_ROW_KMAX || nt < 1 || nt > 3 ||
        !p->row)
        return -2;
    int grid = 0;
    for (int i = 0; i < nt; i++) {
        if (!p->B[i] || p->nb[i] < 1) return -2;
        grid += p->nb[i];
    }
    int rc = -2;
    switch (p->epi) {
    case ORKH_COL_STORE:
        for (int i = 0; i < nt; i++)
            if (!p->C[i]) return -2;
        if (pro != ORKH_ROW_RMSNORM || p->kind != 0) return -2;
        rc = row_launch<ORKH_ROW_RMSNORM, ORKH_COL_STORE, 0>(p, grid, s_);
        break;
    case ORKH_COL_RESID:
        if (pro != ORKH_ROW_QUANT || !p->x || !p->ws0) return -2;
        if (p->kind == 0) rc = row_launch<ORKH_ROW_QUANT, ORKH_COL_RESID, 0>(p, grid, s_);
        else if (p->kind == 1) rc = row_launch<ORKH_ROW_QUANT, ORKH_COL_RESID, 1>(p, grid, s_);
        else rc = row_launch<ORKH_ROW_QUANT, ORKH_COL_RESID, 2>(p, grid, s_);
        break;
    default:
        if (pro != ORKH_ROW_RMSNORM || !p->y || !p->ws0 || !p->ws1 || p->nb[1] != p->nb[0]) return -2;
        grid = p->nb[0];
        if (p->kind == 0) rc = row_launch<ORKH_ROW_RMSNORM, ORKH_COL_SWIGLU, 0>(p, grid, s_);
        else if (p->kind == 1) rc = row_launch<ORKH_ROW_RMSNORM, ORKH_COL_SWIGLU, 1>(p, grid, s_);
        else rc = row_launch<ORKH_ROW_RMSNORM, ORKH_COL_SWIGLU, 2>(p, grid, s_);
        break;
    }
    if (rc) return rc;
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : -1;
}

}  // extern "C"
