"""GPU parity of the grouped-scale runs (ork_i4_mm_run_grouped, ork_i8_mm_run_grouped).

The bar is bit-exact fp32 equality with oracle.gemm_grouped, itself pinned bit for bit to the reference's
own compiled orki_cpu_gemm_grouped (src/npu/core/buf.c:501-520): each K-group's int32 partial is exact,
and the scaled sums run in the same ascending order without fused multiply-adds on both sides.
Shapes: examples/i4.c gtest (grouped W4A4, G 128 and 64), examples/test_grouped_i8.c (grouped int8 through
ork_i4a8_mm_load_tiled, N up to 20480 -- the reference's Sn > 1 cases), G = 32, row tiles (M > 16),
int8 and NF4 weights with ork_w_set_group, host and device operands.
"""
import os

import numpy as np
import pytest

import oracle as O
import ork

pytestmark = pytest.mark.gpu


def _say(*a):
    print("[case]", *a, flush=True)


def _run(fn, npu, w, A, aS, bS):
    M, N = A.shape[0], ork.dims(w)[1]
    C = np.full((M, N), np.nan, np.float32)
    rc = fn(npu.h, w, M, ork.ptr(A), ork.ptr(aS), ork.ptr(bS), ork.ptr(C))
    return rc, C


def _gtest_inputs(M, K, N, G):
    """examples/i4.c gtest (:62-72): LCG values in [-1, 1] quantised to int4 per (row, group) and per
    (group, column) with scale absmax/7, rounding as the reference does (+-0.5f, truncate, clamp [-8, 7])."""
    Sk = K // G
    s = (7 + M + K + N + G) & 0xFFFFFFFF
    raw = np.empty(M * K + K * N, np.int64)
    for i in range(raw.size):
        s = (s * 1103515245 + 12345) & 0xFFFFFFFF
        raw[i] = (s >> 9) % 2001 - 1000
    vals = raw.astype(np.float32) / np.float32(1000.0)
    Af = vals[:M * K].reshape(M, K)
    Bf = vals[M * K:].reshape(K, N)

    def q(x, sc):
        t = (x / sc).astype(np.float32) + np.where(x >= 0, np.float32(0.5), np.float32(-0.5)).astype(np.float32)
        return np.clip(np.trunc(t), -8, 7).astype(np.int8)

    aS = np.maximum(np.abs(Af.reshape(M, Sk, G)).max(2), np.float32(1e-9)) / np.float32(7)
    Ai = q(Af.reshape(M, Sk, G), aS[:, :, None]).reshape(M, K)
    bS = np.maximum(np.abs(Bf.reshape(Sk, G, N)).max(1), np.float32(1e-9)) / np.float32(7)
    Bi = q(Bf.reshape(Sk, G, N), bS[:, None, :]).reshape(K, N)
    return Ai, Bi, aS.astype(np.float32), bS.astype(np.float32)


@pytest.mark.parametrize("M,K,N,G", [(1, 2048, 256, 128), (1, 4096, 512, 128), (4, 2048, 128, 64),
                                     (8, 1024, 256, 64), (3, 512, 128, 32), (100, 1024, 192, 256)])
def test_i4_grouped_exact(npu, M, K, N, G):
    _say("w4a4 grouped", M, K, N, G)
    L = ork.lib()
    A, B, aS, bS = _gtest_inputs(M, K, N, G)
    w = L.ork_i4_mm_pack_grouped(npu.h, K, N, ork.ptr(B), G)
    assert w
    rc, C = _run(L.ork_i4_mm_run_grouped, npu, w, A, aS, bS)
    assert rc == 0
    assert np.array_equal(C, O.gemm_grouped(A, B, aS, bS, G))
    L.ork_mm_free(npu.h, w)


def _grouped_i8_inputs(M, K, N, G):
    """examples/test_grouped_i8.c: int4-range weights, int8-range activations (r4 * 7), patterned scales."""
    rng = np.random.default_rng(M * 31 + K + N + G)
    B = rng.integers(-8, 8, size=(K, N), dtype=np.int8)
    A = (rng.integers(-8, 8, size=(M, K)) * 7).astype(np.int8)
    SG = K // G
    aS = (0.001 * ((np.arange(M * SG) % 13) + 1)).astype(np.float32).reshape(M, SG)
    bS = (0.002 * ((np.arange(SG * N) % 7) + 1)).astype(np.float32).reshape(SG, N)
    return A, B, aS, bS


@pytest.mark.parametrize("M,K,N,G", [(8, 2048, 4096, 512), (8, 2048, 16384, 512), (8, 4096, 20480, 1024),
                                     (4, 3072, 12288, 1024)])
def test_i8_grouped_tiled_load_exact(npu, M, K, N, G):
    _say("i8 grouped via load_tiled", M, K, N, G)
    L = ork.lib()
    A, B, aS, bS = _grouped_i8_inputs(M, K, N, G)
    blob = ork.dump_cpu(npu.h, B, w4a4=True)
    w = L.ork_i4a8_mm_load_tiled(npu.h, K, N, ork.ptr(blob), blob.nbytes, G)
    assert w
    rc, C = _run(L.ork_i8_mm_run_grouped, npu, w, A, aS, bS)
    assert rc == 0
    assert np.array_equal(C, O.gemm_grouped(A, B, aS, bS, G))
    # the same weight runs ungrouped through ork_i8_mm_run, exact int32
    rc, Ci = npu.run_i8(w, A)
    assert rc == 0 and np.array_equal(Ci, O.gemm_i32(A, B))
    L.ork_mm_free(npu.h, w)


@pytest.mark.parametrize("G,M", [(32, 1), (64, 20), (256, 1), (2048, 5)])
def test_i8_set_group_exact(npu, G, M):
    _say("i8 set_group", G, M)
    L = ork.lib()
    K, N = 2048, 384
    rng = np.random.default_rng(G + M)
    B = rng.integers(-128, 128, size=(K, N), dtype=np.int8)
    A = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
    aS = rng.uniform(1e-3, 1e-2, size=(M, K // G)).astype(np.float32)
    bS = rng.uniform(1e-3, 1e-2, size=(K // G, N)).astype(np.float32)
    w = npu.pack_i8(B)
    assert L.ork_w_set_group(w, G) == 0
    rc, C = _run(L.ork_i8_mm_run_grouped, npu, w, A, aS, bS)
    assert rc == 0 and np.array_equal(C, O.gemm_grouped(A, B, aS, bS, G))
    L.ork_mm_free(npu.h, w)


@pytest.mark.parametrize("nf4", [0, 1])
def test_i4a8_grouped_exact(npu, nf4):
    _say("i4a8 grouped", nf4)
    L = ork.lib()
    K, N, M, G = 1024, 256, 3, 128
    rng = np.random.default_rng(40 + nf4)
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    if nf4:
        os.environ["ORK_NF4"] = "1"
    try:
        w, _ = npu.pack_i4a8(W)
    finally:
        os.environ.pop("ORK_NF4", None)
    _, _, codes = O.pack_i4a8(W, nf4=bool(nf4))
    A = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
    aS = rng.uniform(1e-3, 1e-2, size=(M, K // G)).astype(np.float32)
    bS = rng.uniform(1e-3, 1e-2, size=(K // G, N)).astype(np.float32)
    assert L.ork_w_set_group(w, G) == 0
    rc, C = _run(L.ork_i8_mm_run_grouped, npu, w, A, aS, bS)
    assert rc == 0 and np.array_equal(C, O.gemm_grouped(A, codes, aS, bS, G))
    L.ork_mm_free(npu.h, w)


def test_grouped_device_operands_async(npu):
    _say("grouped device operands")
    L = ork.lib()
    M, K, N, G = 16, 1024, 256, 128
    A, B, aS, bS = _gtest_inputs(M, K, N, G)
    w = L.ork_i4_mm_pack_grouped(npu.h, K, N, ork.ptr(B), G)
    bufs = []
    for arr in (A, aS, bS):
        d = L.ork_dev_alloc(npu.h, arr.nbytes)
        assert d and L.ork_dev_upload(npu.h, d, ork.ptr(arr), arr.nbytes) == 0
        bufs.append(d)
    dC = L.ork_dev_alloc(npu.h, M * N * 4)
    L.ork_npu_set_async(npu.h, 1)
    try:
        assert L.ork_i4_mm_run_grouped(npu.h, w, M, bufs[0], bufs[1], bufs[2], dC) == 0
        assert L.ork_npu_sync(npu.h) == 0
    finally:
        L.ork_npu_set_async(npu.h, 0)
    C = np.empty((M, N), np.float32)
    assert L.ork_dev_download(npu.h, ork.ptr(C), dC, C.nbytes) == 0
    assert np.array_equal(C, O.gemm_grouped(A, B, aS, bS, G))
    for d in bufs + [dC]:
        L.ork_dev_free(npu.h, d)
    L.ork_mm_free(npu.h, w)


def test_grouped_errors(npu):
    _say("grouped errors")
    L = ork.lib()
    K, N = 512, 128
    B = np.zeros((K, N), np.int8)
    A = np.zeros((2, K), np.int8)
    aS = np.ones((2, K // 64), np.float32)
    bS = np.ones((K // 64, N), np.float32)
    w = npu.pack_i8(B)
    assert _run(L.ork_i8_mm_run_grouped, npu, w, A, aS, bS)[0] == -1          # no group size
    assert L.ork_w_set_group(w, 96) == -1                                      # K % G
    assert L.ork_w_set_group(w, 16) == 0
    assert _run(L.ork_i8_mm_run_grouped, npu, w, A, aS, bS)[0] == -3          # G % 32
    assert L.ork_w_set_group(w, 64) == 0
    assert _run(L.ork_i4_mm_run_grouped, npu, w, A, aS, bS)[0] == -1          # int8 weight, int4 run
    assert _run(L.ork_i8_mm_run_grouped, npu, w, A, aS, bS)[0] == 0
    wf = npu.pack_f16(np.zeros((K, N), np.float16))
    assert L.ork_w_set_group(wf, 64) == -1                                     # fp16 has no groups
    assert L.ork_i4_mm_pack_grouped(npu.h, K, N, ork.ptr(B), 48) is None        # G % 32
    assert L.ork_i4_mm_pack_grouped(npu.h, K, 96, ork.ptr(np.zeros((K, 96), np.int8)), 64) is None  # N % 64
    L.ork_mm_free(npu.h, w)
    L.ork_mm_free(npu.h, wf)


def _env_run(env, fn, npu, w, A, aS, bS):
    old = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    try:
        return _run(fn, npu, w, A, aS, bS)
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


@pytest.mark.parametrize("tile", [None, "64x64", "64x192"])
@pytest.mark.parametrize("kind,M,K,N,G", [
    ("i8", 64, 2048, 256, 128),     # groups of one 128-k stage
    ("i8", 100, 2080, 224, 160),    # groups end inside stages and K-blocks; K tail mid-block; partial tiles
    ("i8", 33, 1024, 192, 32),      # two groups per K-block
    ("i8", 256, 2048, 384, 2048),   # one group
    ("i8", 70, 2048, 224, 512),     # groups of four stages; partial tiles
    ("w4a4", 256, 2048, 512, 128),  # one group per K-block (examples/i4.c gtest shape family)
    ("w4a4", 70, 1056, 320, 96),    # groups straddle the 128-k blocks; K tail; partial tiles
    ("w4a4", 48, 1024, 128, 32),    # four groups per K-block
])
def test_grouped_tiled_exact(npu, tile, kind, M, K, N, G):
    """The LDS-ring grouped kernel (k_tiled2g; ORK_PLAN=tiled, and ORK_TILE when given) against the oracle bit
    for bit, and against the panel-streaming k_grouped forced on the same inputs. G % 128 == 0 runs the
    whole-stage variant, the other group sizes the K-block walk."""
    _say("grouped tiled", kind, M, K, N, G, tile)
    L = ork.lib()
    if kind == "i8":
        rng = np.random.default_rng(M + K + N + G)
        B = rng.integers(-128, 128, size=(K, N), dtype=np.int8)
        A = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
        aS = rng.uniform(1e-3, 1e-2, size=(M, K // G)).astype(np.float32)
        bS = rng.uniform(1e-3, 1e-2, size=(K // G, N)).astype(np.float32)
        w = npu.pack_i8(B)
        assert L.ork_w_set_group(w, G) == 0
        fn = L.ork_i8_mm_run_grouped
    else:
        A, B, aS, bS = _gtest_inputs(M, K, N, G)
        w = L.ork_i4_mm_pack_grouped(npu.h, K, N, ork.ptr(B), G)
        assert w
        fn = L.ork_i4_mm_run_grouped
    env = {"ORK_PLAN": "tiled", **({"ORK_TILE": tile} if tile else {})}
    rc, C = _env_run(env, fn, npu, w, A, aS, bS)
    os.environ.update(env)
    try:
        name = npu.grouped_plan_name(w, M)
    finally:
        for k in env:
            os.environ.pop(k, None)
    assert name.startswith("tiled2g_") and (tile is None or name.endswith(tile)), name
    assert rc == 0 and np.array_equal(C, O.gemm_grouped(A, B, aS, bS, G)), name
    rc2, C2 = _env_run({"ORK_PLAN": "stream"}, fn, npu, w, A, aS, bS)
    assert rc2 == 0 and np.array_equal(C, C2)
    L.ork_mm_free(npu.h, w)


def test_grouped_plan_names(npu):
    """Default plans: one row runs the half-panel VALU kernel (k_grouped_gemv), a few rows stream panels
    (k_grouped); int8 / uniform int4 take the LDS-ring kernel from 32 rows when G % 128 == 0 and from 128 rows
    otherwise; NF4 always streams."""
    L = ork.lib()
    B = np.zeros((1024, 256), np.int8)
    w = npu.pack_i8(B)
    assert npu.grouped_plan_name(w, 8) == "none"  # no group size yet
    assert L.ork_w_set_group(w, 128) == 0
    assert npu.grouped_plan_name(w, 1).startswith("grouped_i8_gemvh_")  # one row: the half-panel VALU kernel
    assert npu.grouped_plan_name(w, 8).startswith("grouped_i8_mt")
    assert npu.grouped_plan_name(w, 31).startswith("grouped_i8_")
    assert npu.grouped_plan_name(w, 32).startswith("tiled2g_i8_")
    assert L.ork_w_set_group(w, 64) == 0
    assert npu.grouped_plan_name(w, 127).startswith("grouped_i8_")
    assert npu.grouped_plan_name(w, 128).startswith("tiled2g_i8_")
    L.ork_mm_free(npu.h, w)
    W = (np.random.default_rng(1).standard_normal((256, 1024)) * 0.02).astype(np.float32)
    os.environ["ORK_NF4"] = "1"
    try:
        w, _ = npu.pack_i4a8(W)
    finally:
        os.environ.pop("ORK_NF4", None)
    assert L.ork_w_set_group(w, 128) == 0
    assert npu.grouped_plan_name(w, 256).startswith("grouped_nf4_")
    L.ork_mm_free(npu.h, w)


def test_grouped_default_plan_exact(npu):
    """The default plan at M = 256 (the LDS-ring kernel) on a grouped W4A4 shape, bit for bit."""
    _say("grouped default plan W4A4 M=256")
    L = ork.lib()
    M, K, N, G = 256, 1024, 512, 128
    A, B, aS, bS = _gtest_inputs(M, K, N, G)
    w = L.ork_i4_mm_pack_grouped(npu.h, K, N, ork.ptr(B), G)
    assert npu.grouped_plan_name(w, M).startswith("tiled2g_i4u_")
    rc, C = _run(L.ork_i4_mm_run_grouped, npu, w, A, aS, bS)
    assert rc == 0 and np.array_equal(C, O.gemm_grouped(A, B, aS, bS, G))
    L.ork_mm_free(npu.h, w)


@pytest.mark.parametrize("kind", ["w4a4", "i8", "i4a8", "nf4"])
def test_grouped_one_row_exact(npu, kind):
    """One row (k_grouped_gemv: half panels, int32 group partials summed in LDS, scaled terms added in ascending
    group order) bit for bit against the oracle and against the panel-streaming kernel (ORK_PLAN=stream), over
    group sizes below, equal to and above a K-block, K tails inside a group and up to 512 groups."""
    _say("grouped one row", kind)
    L = ork.lib()
    rng = np.random.default_rng(77 + len(kind))
    for K, N, G in [(2048, 256, 32), (4096, 512, 128), (1024, 1024, 64), (1056, 256, 96), (2048, 384, 512),
                    (16384, 128, 32)]:
        if kind == "w4a4":
            A, B, aS, bS = _gtest_inputs(1, K, N, G)
            w = L.ork_i4_mm_pack_grouped(npu.h, K, N, ork.ptr(B), G)
            fn = L.ork_i4_mm_run_grouped
            codes = B
        else:
            A = rng.integers(-127, 128, size=(1, K), dtype=np.int8)
            aS = rng.uniform(1e-3, 1e-2, size=(1, K // G)).astype(np.float32)
            bS = rng.uniform(1e-3, 1e-2, size=(K // G, N)).astype(np.float32)
            if kind == "i8":
                codes = rng.integers(-128, 128, size=(K, N), dtype=np.int8)
                w = npu.pack_i8(codes)
            else:
                W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
                if kind == "nf4":
                    os.environ["ORK_NF4"] = "1"
                try:
                    w, _ = npu.pack_i4a8(W)
                finally:
                    os.environ.pop("ORK_NF4", None)
                _, _, codes = O.pack_i4a8(W, nf4=kind == "nf4")
            assert L.ork_w_set_group(w, G) == 0
            fn = L.ork_i8_mm_run_grouped
        assert w, (kind, K, N, G)
        name = npu.grouped_plan_name(w, 1)
        assert name.startswith("grouped_") and "_gemvh_" in name, name
        rc, C = _run(fn, npu, w, A, aS, bS)
        assert rc == 0 and np.array_equal(C, O.gemm_grouped(A, codes, aS, bS, G)), (kind, K, N, G, name)
        rc2, C2 = _env_run({"ORK_PLAN": "stream"}, fn, npu, w, A, aS, bS)
        assert rc2 == 0 and np.array_equal(C2, C), (kind, K, N, G)
        L.ork_mm_free(npu.h, w)


def _random_grouped(n=40, seed=0x67727073):
    rng = np.random.default_rng(seed)
    out = []
    for c in range(n):
        kind = ["i8", "w4a4", "u4", "nf4"][c % 4]
        G = int(rng.choice([32, 64, 96, 128, 256, 512]))
        K = G * int(rng.integers(1, max(2, 4096 // G) + 1))
        step = 64 if kind == "w4a4" else 32
        N = step * int(rng.integers(1, 2048 // step + 1))
        M = int(rng.choice([1, 2, 8, 17, 31, 32, 64, 100, 128, 129, 256]))
        while N > step and M * K * N > 300_000_000:
            N = max(step, (N // 2) // step * step)
        out.append((c, kind, M, K, N, G))
    return out


@pytest.mark.parametrize("c,kind,M,K,N,G", _random_grouped())
def test_grouped_random(npu, c, kind, M, K, N, G):
    """Seeded random grouped-scale runs at default plans (one-row kernel, panel streaming, grouped LDS-ring tiles;
    group sizes below, at and above a K-block), bit for bit against the oracle's ascending-group accumulate."""
    _say("random grouped", c, kind, M, K, N, G)
    L = ork.lib()
    rng = np.random.default_rng(700 + c)
    aS = rng.uniform(1e-3, 1e-2, size=(M, K // G)).astype(np.float32)
    bS = rng.uniform(1e-3, 1e-2, size=(K // G, N)).astype(np.float32)
    if kind == "w4a4":
        A = rng.integers(-8, 8, size=(M, K), dtype=np.int8)
        codes = rng.integers(-8, 8, size=(K, N), dtype=np.int8)
        w = L.ork_i4_mm_pack_grouped(npu.h, K, N, ork.ptr(codes), G)
        fn = L.ork_i4_mm_run_grouped
    else:
        A = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
        if kind == "i8":
            codes = rng.integers(-128, 128, size=(K, N), dtype=np.int8)
            w = npu.pack_i8(codes)
        else:
            W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
            if kind == "nf4":
                os.environ["ORK_NF4"] = "1"
            try:
                w, _ = npu.pack_i4a8(W)
            finally:
                os.environ.pop("ORK_NF4", None)
            _, _, codes = O.pack_i4a8(W, nf4=kind == "nf4")
        assert L.ork_w_set_group(w, G) == 0
        fn = L.ork_i8_mm_run_grouped
    assert w
    rc, C = _run(fn, npu, w, A, aS, bS)
    assert rc == 0 and np.array_equal(C, O.gemm_grouped(A, codes, aS, bS, G)), npu.grouped_plan_name(w, M)
    L.ork_mm_free(npu.h, w)
