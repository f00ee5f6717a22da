"""GPU parity over a seeded random sweep of shapes, every resident kind, default plans.

The fixed-shape tests pin each kernel and tile on purpose; this sweep draws (kind, M, K, N) from a fixed seed
so that the planner's own choices -- GEMV, streaming, LDS-ring tiles with either A layout, the older tiled
kernel for NF4, K splits -- are all reached on shapes nobody picked by hand. M leans on the boundaries
where a choice changes (1, 2, 16/17, 64/65, 128/129, 255-257); K and N are any multiple the pack accepts
(K % 32; N % 32, N % 64 for W4A4, N % 16 for fp16), so K-block, panel and tile tails all occur.
Bar: bit-exact int32 vs the oracle for the integer kinds, fp16 within 2e-3 of fp64 accumulation.
"""
import os

import numpy as np
import pytest

import oracle as O
import ork

pytestmark = pytest.mark.gpu
FP16_TOL = 2e-3
M_EDGES = [1, 2, 3, 15, 16, 17, 31, 48, 63, 64, 65, 96, 127, 128, 129, 192, 255, 256, 257, 320, 384, 511, 512, 600]


def _cases(n=60, seed=0x6F726B52):
    rng = np.random.default_rng(seed)
    kinds = ["i8", "i4a8", "nf4", "w4a4", "f16"]
    out = []
    # every kind at the few-row sizes (GEMV, streaming, the mid-M choice), then the general draw
    fixed = [(kind, m) for kind in kinds for m in (1, 2, 17, 64)]
    for i in range(n + len(fixed)):
        kind, M = fixed[i] if i < len(fixed) else (kinds[i % len(kinds)], None)
        if M is None:
            M = int(rng.choice(M_EDGES)) if rng.random() < 0.8 else int(rng.integers(1, 700))
        K = 32 * int(rng.integers(1, 129))                      # 32 .. 4096
        step = {"w4a4": 64, "f16": 16}.get(kind, 32)
        N = step * int(rng.integers(1, 4096 // step + 1))        # up to 4096
        # keep the CPU oracle and packing quick: K x N <= 4 Mi, M x K x N <= 400 M
        while N > step and (K * N > (1 << 22) or M * K * N > 400_000_000):
            N = max(step, (N // 2) // step * step)
        out.append((i, kind, M, K, N))
    # the streaming kernel's paired-panel range at default plans: cu < N/16 < 2*cu panels (cu = 256 on MI355X)
    # and 9 <= M <= 32; N is a multiple of 64 there, so every kind packs
    for j in range(8):
        kind = kinds[j % len(kinds)]
        M = int(rng.integers(9, 33))
        N = 64 * int(rng.integers(16 * 256 // 64 + 1, 32 * 256 // 64))
        K = 32 * int(rng.integers(1, 33))
        out.append((n + len(fixed) + j, kind, M, K, N))
    return out


@pytest.mark.parametrize("i,kind,M,K,N", _cases())
def test_random_shape(npu, i, kind, M, K, N):
    print(f"[case] random #{i}: {kind} M={M} K={K} N={N}", flush=True)
    rng = np.random.default_rng(1000 + i)
    if kind == "i8":
        B = rng.integers(-128, 128, size=(K, N), dtype=np.int8)
        A = rng.integers(-128, 128, size=(M, K), dtype=np.int8)
        w = npu.pack_i8(B)
        rc, C = npu.run_i8(w, A)
        ref = O.gemm_i32(A, B)
    elif kind in ("i4a8", "nf4"):
        W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
        im = rng.uniform(0.5, 2.0, K).astype(np.float32)
        if kind == "nf4":
            os.environ["ORK_NF4"] = "1"
        try:
            w, _ = npu.pack_i4a8(W, im)
        finally:
            os.environ.pop("ORK_NF4", None)
        _, _, codes = O.pack_i4a8(W, im, nf4=kind == "nf4")
        A = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
        rc, C = npu.run_i8(w, A)
        ref = O.gemm_i32(A, codes)
    elif kind == "w4a4":
        B = rng.integers(-8, 8, size=(K, N), dtype=np.int8)
        A = rng.integers(-8, 8, size=(M, K), dtype=np.int8)
        w = npu.pack_i4(B)
        rc, C = npu.run_i4(w, A)
        ref = O.gemm_i32(A, B)
    else:
        B = (rng.standard_normal((K, N)) * 0.02).astype(np.float16)
        A = rng.standard_normal((M, K)).astype(np.float16)
        w = npu.pack_f16(B)
        rc, C = npu.run_f16(w, A)
        ref = None
    assert w, "pack failed"
    plan = npu.plan_name(w, M)
    assert rc == 0, plan
    if ref is None:
        err = O.fp16_err(C, O.gemm_f16_f64acc(A, B))
        assert err <= FP16_TOL, (plan, err)
    else:
        assert np.array_equal(C, ref), plan
    ork.free(w)
