"""CPU restatement (numpy, float32) of the one-row run's row prologue and column epilogue (ork_i8_mm_run_row,
include/ork/hip.h), in the exact order of operations the library documents, so that its results can be compared
bit for bit.

TEST INFRASTRUCTURE ONLY: imported by tests/, never by the product.

  per-row int8 quantisation   examples/quant.c:34-37: s = max|y| / 127 (1 for a zero row), q = clamp(rint(y / s),
                              -127, 127) -- with the library's evaluation of y / s: y * (1 / s), except within 1e-4
                              of a half-way point, where the exact quotient decides
  RMSNorm                     examples/bench.c:75 (o = x * (1 / sqrt(mean(x^2) + eps)) * w), with the sum of squares
                              in the documented order: 512 threads, thread t summing elements t, t + 512, ... in
                              order; each 64-thread wave folded by a pairwise tree of adjacent lanes (l with l ^ 1,
                              then pairs of pairs, ... up to l ^ 32); the 8 wave sums added in wave order from 0
  epilogues                   C = c; x + (c * s) * ws; silu(g) * u with g = (c_g * s) * ws_g, u = (c_u * s) * ws_u

Every + - * / sqrt here is an IEEE float32 operation, as on the GPU (compiled without contraction, divisions and
square roots correctly rounded). The int32 products come from oracle.gemm_i32. Only silu's exp differs: numpy's
float32 exp and the GPU's expf may differ in the last place, so the SwiGLU epilogue agrees to a few ulp, not bits.
"""
import numpy as np

import oracle as O

F32 = np.float32
THREADS = 512


def _wave_tree(v):
    """The pairwise fold of 64 lane values: l with l ^ 1, then l with l ^ 2, ... l with l ^ 32."""
    v = np.asarray(v, F32)
    while v.size > 1:
        v = (v[0::2] + v[1::2]).astype(F32)
    return v[0]


def sum_squares(x):
    """The row's sum of squares in the library's order (see the module docstring)."""
    x = np.asarray(x, F32)
    K = x.size
    E = (K + THREADS - 1) // THREADS
    xp = np.zeros(E * THREADS, F32)
    xp[:K] = x
    per = np.zeros(THREADS, F32)
    for k in range(E):                                     # thread t: ss = ss + y[k] * y[k], k ascending
        y = xp[k * THREADS:(k + 1) * THREADS]
        per = (per + (y * y).astype(F32)).astype(F32)
    s = F32(0.0)
    for w in range(THREADS // 64):                         # the waves' partials, added in wave order
        s = F32(s + _wave_tree(per[64 * w:64 * (w + 1)]))
    return s


def rmsnorm(x, w, eps):
    x = np.asarray(x, F32)
    ss = sum_squares(x)
    r = F32(1.0) / np.sqrt(F32(ss / F32(x.size) + F32(eps)))
    return ((x * r).astype(F32) * np.asarray(w, F32)).astype(F32)


def quant_row(y):
    """(int8 row, scale s)"""
    y = np.asarray(y, F32)
    mx = F32(np.abs(y).max()) if y.size else F32(0)
    s = F32(mx / F32(127.0)) if mx > 0 else F32(1.0)
    inv = F32(F32(1.0) / s)
    r = (y * inv).astype(F32)
    near = np.abs(r - np.floor(r) - F32(0.5)) < F32(1e-4)
    r = np.where(near, (y / s).astype(F32), r)
    return np.clip(np.rint(r), -127, 127).astype(np.int8), s


def prologue(row, norm_w=None, eps=0.0):
    """ORK_ROW_RMSNORM when norm_w is given, else ORK_ROW_QUANT: (int8 row, scale)."""
    y = rmsnorm(row, norm_w, eps) if norm_w is not None else np.asarray(row, F32)
    return quant_row(y)


def resid(x, c, s, ws):
    return (np.asarray(x, F32) + ((c.astype(F32) * F32(s)).astype(F32) * np.asarray(ws, F32)).astype(F32)).astype(F32)


def swiglu(cg, cu, s, wsg, wsu):
    g = ((cg.astype(F32) * F32(s)).astype(F32) * np.asarray(wsg, F32)).astype(F32)
    u = ((cu.astype(F32) * F32(s)).astype(F32) * np.asarray(wsu, F32)).astype(F32)
    with np.errstate(over="ignore"):   # exp(-g) = inf for very negative g: silu(g) = g / inf = -0, as expf gives
        return ((g / (F32(1.0) + np.exp(-g).astype(F32))).astype(F32) * u).astype(F32)


def gemv(a, codes_kn):
    """The exact int32 columns of one int8 row against int8 codes [K][N]."""
    return O.gemm_i32(np.asarray(a, np.int8)[None, :], codes_kn)[0]
