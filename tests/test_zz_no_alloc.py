"""ork_i8_mm_run_noalloc (include/ork/hip.h): ork_i8_mm_run for callers that cannot allocate. Device A and C; a
split-K plan keeps its partials in the library's static per-GPU scratch array. Checked against the existing entry
point ork_i8_mm_run and the oracle, bit for bit, on two calls in a row (the second smaller, so it runs over the
first call's leftover partials), at forced split-K plans of the streaming, GEMV and LDS-ring kernels and at a
default plan; a plan whose partials exceed the array, and host operands, are refused (-1).
"""
import os

import numpy as np
import pytest

import oracle as O
import ork

pytestmark = pytest.mark.gpu


class _env:
    def __init__(self, **kv):
        self.kv = {k: str(v) for k, v in kv.items()}

    def __enter__(self):
        self.old = {k: os.environ.get(k) for k in self.kv}
        os.environ.update(self.kv)

    def __exit__(self, *a):
        for k, v in self.old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


def _dev(npu, a):
    L = ork.lib()
    d = L.ork_dev_alloc(npu.h, a.nbytes)
    assert d and L.ork_dev_upload(npu.h, d, ork.ptr(a), a.nbytes) == 0
    return d


def _run_both(npu, w, A, N, env):
    """(C from ork_i8_mm_run_noalloc, C from ork_i8_mm_run, plan name), both on device A and C."""
    L = ork.lib()
    M = A.shape[0]
    dA = _dev(npu, A)
    dC1 = L.ork_dev_alloc(npu.h, M * N * 4)
    dC2 = L.ork_dev_alloc(npu.h, M * N * 4)
    assert dC1 and dC2
    with _env(**env):
        name = npu.plan_name(w, M)
        assert L.ork_i8_mm_run_noalloc(npu.h, w, M, dA, dC1) == 0, name
        assert L.ork_i8_mm_run(npu.h, w, M, dA, dC2) == 0, name
    C1 = np.empty((M, N), np.int32)
    C2 = np.empty((M, N), np.int32)
    assert L.ork_dev_download(npu.h, ork.ptr(C1), dC1, C1.nbytes) == 0
    assert L.ork_dev_download(npu.h, ork.ptr(C2), dC2, C2.nbytes) == 0
    for d in (dA, dC1, dC2):
        L.ork_dev_free(npu.h, d)
    return C1, C2, name


# (first call, second smaller call): (M, K, N, plan env) -- split plans put their partials in the scratch array
PAIRS = [
    ((16, 4096, 1024, dict(ORK_PLAN="stream", ORK_KSPLIT=4)), (5, 2048, 512, dict(ORK_PLAN="stream", ORK_KSPLIT=2))),
    ((1, 12288, 2048, dict(ORK_KSPLIT=8)), (1, 4096, 256, dict(ORK_KSPLIT=4))),
    ((256, 4096, 768, dict(ORK_TILE="64x64", ORK_KSPLIT=4)), (96, 2048, 384, dict(ORK_TILE="64x64", ORK_KSPLIT=2))),
    ((1, 12288, 64, {}), (1, 2048, 64, {})),
]


@pytest.mark.parametrize("i", range(len(PAIRS)))
def test_noalloc_matches_run_twice(npu, i):
    rng = np.random.default_rng(300 + i)
    for j, (M, K, N, env) in enumerate(PAIRS[i]):
        print(f"[case] noalloc pair {i} call {j}: M={M} K={K} N={N} {env}", flush=True)
        B = rng.integers(-128, 128, size=(K, N), dtype=np.int8)
        A = rng.integers(-128, 128, size=(M, K), dtype=np.int8)
        w = npu.pack_i8(B)
        assert w
        C1, C2, name = _run_both(npu, w, A, N, env)
        if env:
            assert "_ks" in name and not name.endswith("_ks1"), name   # a split plan: partials in the scratch array
        assert np.array_equal(C1, C2), name
        assert np.array_equal(C1, O.gemm_i32(A, B)), name
        ork.free(w)


def test_noalloc_i4a8_weight(npu):
    """An i4a8 weight (nibbles resident) through the same entry point, split and unsplit."""
    rng = np.random.default_rng(310)
    K, N, M = 4096, 512, 8
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    w, _ = npu.pack_i4a8(W)
    _, _, codes = O.pack_i4a8(W)
    A = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
    for env in (dict(ORK_PLAN="stream", ORK_KSPLIT=4), {}):
        C1, C2, name = _run_both(npu, w, A, N, env)
        assert np.array_equal(C1, C2) and np.array_equal(C1, O.gemm_i32(A, codes)), name
    ork.free(w)


def test_noalloc_refusals(npu):
    """Partials above the scratch array (16 MiB at this forced split) and host operands are refused; the
    allocating entry point still runs that plan."""
    L = ork.lib()
    rng = np.random.default_rng(320)
    K, N, M = 8192, 8192, 64
    B = rng.integers(-128, 128, size=(K, N), dtype=np.int8)
    A = rng.integers(-128, 128, size=(M, K), dtype=np.int8)
    w = npu.pack_i8(B)
    dA = _dev(npu, A)
    dC = L.ork_dev_alloc(npu.h, M * N * 4)
    with _env(ORK_PLAN="stream", ORK_KSPLIT=8):
        assert L.ork_i8_mm_run_noalloc(npu.h, w, M, dA, dC) == -1
        assert L.ork_i8_mm_run(npu.h, w, M, dA, dC) == 0
    C = np.empty((M, N), np.int32)
    assert L.ork_dev_download(npu.h, ork.ptr(C), dC, C.nbytes) == 0
    assert np.array_equal(C[:4], O.gemm_i32(A[:4], B))
    Ch = np.zeros((M, N), np.int32)
    assert L.ork_i8_mm_run_noalloc(npu.h, w, M, ork.ptr(A), dC) == -1      # host A
    assert L.ork_i8_mm_run_noalloc(npu.h, w, M, dA, ork.ptr(Ch)) == -1     # host C
    assert L.ork_i8_mm_run_noalloc(npu.h, w, 0, dA, dC) == -1
    L.ork_dev_free(npu.h, dA)
    L.ork_dev_free(npu.h, dC)
    ork.free(w)


def test_noalloc_misaligned_a_refused(npu):
    """A device A that is not 16-byte aligned is refused (-1) by the no-allocation entry point, which cannot stage
    it; ork_i8_mm_run stages such an A and computes."""
    L = ork.lib()
    rng = np.random.default_rng(330)
    K, N, M = 256, 64, 2
    B = rng.integers(-128, 128, size=(K, N), dtype=np.int8)
    A = rng.integers(-128, 128, size=(M, K), dtype=np.int8)
    w = npu.pack_i8(B)
    raw = np.zeros(A.nbytes + 16, np.int8)
    raw[4:4 + A.nbytes] = A.reshape(-1)
    dA = _dev(npu, raw)
    dC = L.ork_dev_alloc(npu.h, M * N * 4)
    assert L.ork_i8_mm_run_noalloc(npu.h, w, M, dA + 4, dC) == -1
    assert L.ork_i8_mm_run(npu.h, w, M, dA + 4, dC) == 0
    C = np.empty((M, N), np.int32)
    assert L.ork_dev_download(npu.h, ork.ptr(C), dC, C.nbytes) == 0
    assert np.array_equal(C, O.gemm_i32(A, B))
    L.ork_dev_free(npu.h, dA)
    L.ork_dev_free(npu.h, dC)
    ork.free(w)


def test_noalloc_under_graph_capture(npu):
    """Under HIP graph capture: outside async mode the call is refused (-1) and enqueues nothing (the capture stays
    valid); in async mode a forced split-K call is captured, and its graph, replayed twice with an eager call that
    rewrites the scratch array in between, gives the oracle's C on every replay."""
    import hipgraph

    L = ork.lib()
    G = hipgraph.Graphs()
    stream = L.ork_npu_stream(npu.h)
    rng = np.random.default_rng(340)
    M, K, N = 16, 4096, 1024
    B = rng.integers(-128, 128, size=(K, N), dtype=np.int8)
    A = rng.integers(-128, 128, size=(M, K), dtype=np.int8)
    B2 = rng.integers(-128, 128, size=(2048, 512), dtype=np.int8)
    A2 = rng.integers(-128, 128, size=(5, 2048), dtype=np.int8)
    w, w2 = npu.pack_i8(B), npu.pack_i8(B2)
    dA, dA2 = _dev(npu, A), _dev(npu, A2)
    dC = L.ork_dev_alloc(npu.h, M * N * 4)
    dC2 = L.ork_dev_alloc(npu.h, 5 * 512 * 4)
    want = O.gemm_i32(A, B)
    zero = np.zeros((M, N), np.int32)
    try:
        with _env(ORK_PLAN="stream", ORK_KSPLIT=4):
            name = npu.plan_name(w, M)
            assert "_ks4" in name, name
            print("[case] noalloc under capture, sync mode (refused):", name, flush=True)
            rc, g, ex = G.capture(stream, lambda: L.ork_i8_mm_run_noalloc(npu.h, w, M, dA, dC), instantiate=False)
            assert rc == -1
            G.destroy(g, ex)
            print("[case] noalloc under capture, async mode:", name, flush=True)
            L.ork_npu_set_async(npu.h, 1)
            rc, g, ex = G.capture(stream, lambda: L.ork_i8_mm_run_noalloc(npu.h, w, M, dA, dC))
            assert rc == 0
        try:
            for rep in range(2):
                assert L.ork_dev_upload(npu.h, dC, ork.ptr(zero), zero.nbytes) == 0
                G.replay(ex, stream)
                C = np.empty((M, N), np.int32)
                assert L.ork_dev_download(npu.h, ork.ptr(C), dC, C.nbytes) == 0
                assert np.array_equal(C, want), rep
                # eager work between replays: another split call through the same scratch array
                with _env(ORK_PLAN="stream", ORK_KSPLIT=2):
                    assert L.ork_i8_mm_run_noalloc(npu.h, w2, 5, dA2, dC2) == 0
                assert L.ork_npu_sync(npu.h) == 0
                C2 = np.empty((5, 512), np.int32)
                assert L.ork_dev_download(npu.h, ork.ptr(C2), dC2, C2.nbytes) == 0
                assert np.array_equal(C2, O.gemm_i32(A2, B2)), rep
        finally:
            G.destroy(g, ex)
    finally:
        L.ork_npu_set_async(npu.h, 0)
        for d in (dA, dA2, dC, dC2):
            L.ork_dev_free(npu.h, d)
        ork.free(w)
        ork.free(w2)
