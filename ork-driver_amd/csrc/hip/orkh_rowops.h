// orkh_rowops.h -- row operations shared by the library's fused one-row run (orkh_rowrun.hip) and the decoder
// harness's glue kernels (csrc/qwen3/q3_ops.hip): wave and workgroup reductions, register rows, and the per-row
// int8 quantisation. Both sides include this one definition, so a row prepared inside a fused matmul launch and
// the same row prepared by a separate kernel go through the same float operations in the same order and agree
// bit for bit. Device code for gfx950; every file that includes it is compiled with -ffp-contract=off.
#ifndef ORKH_ROWOPS_H
#define ORKH_ROWOPS_H
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

namespace orkr {

// One element of a per-row int8 quantisation with scale s and inv = 1 / s (quant_regs below, and the fused
// run's prologue): q = clamp(rint(y / s), -127, 127), where y * inv stands in for y / s except within 1e-4 of a
// half-way point, where the exact quotient decides.
__device__ inline int8_t quant_elem(float y, float inv, float s) {
    float r = y * inv;
    if (fabsf(r - floorf(r) - 0.5f) < 1e-4f) r = y / s;
    r = fminf(fmaxf(rintf(r), -127.f), 127.f);
    return (int8_t)(int)r;
}

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
        if (i < n) q[i] = quant_elem(y[k], inv, s);
    }
    if (threadIdx.x == 0) *s_out = s;
}

}  // namespace orkr
#endif
