"""GPU parity of the multi-matmul submit (ork_{i8,i4}_mm_run_chain / _stream, ork_f16_mm_run_stream).

Each task of a chain must give exactly what its single run gives: bit-exact int32 against the oracle
for the integer kinds, within the fp16 bar for fp16. Chains mix grouped M = 1 tasks of several
resident kinds (more than one grouped launch's worth), MFMA-stream and tiled tasks, host and
device-resident operands, and a C row stride.
"""
import os

import numpy as np
import pytest

import oracle as O
import ork

pytestmark = pytest.mark.gpu
FP16_TOL = 2e-3


def _say(*a):
    print("[case]", *a, flush=True)


def _i4a8(npu, rng, K, N, nf4):
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    im = rng.uniform(0.5, 2.0, K).astype(np.float32)
    if nf4:
        os.environ["ORK_NF4"] = "1"
    try:
        w, _ = npu.pack_i4a8(W, im)
    finally:
        os.environ.pop("ORK_NF4", None)
    _, _, codes = O.pack_i4a8(W, im, nf4=nf4)
    return w, codes


@pytest.mark.parametrize("entry", ["ork_i8_mm_run_chain", "ork_i8_mm_run_stream"])
def test_i8_chain_mixed(npu, entry):
    _say(entry)
    rng = np.random.default_rng(71)
    specs = []  # (w, codes[K][N], M)
    for K, N in [(2048, 384), (96, 64), (2080, 96)] + [(256, 32)] * 18:  # > ORKH_GROUP_MAX M=1 int8 tasks
        B = rng.integers(-128, 128, size=(K, N), dtype=np.int8)
        specs.append((npu.pack_i8(B), B, 1))
    for nf4 in (0, 1):
        w, codes = _i4a8(npu, rng, 1024, 256, nf4)
        specs.append((w, codes, 1))
    B = rng.integers(-128, 128, size=(160, 96), dtype=np.int8)
    specs.append((npu.pack_i8(B), B, 5))        # MFMA stream
    B = rng.integers(-128, 128, size=(256, 128), dtype=np.int8)
    specs.append((npu.pack_i8(B), B, 100))      # tiled
    w, codes = _i4a8(npu, rng, 512, 96, 1)
    specs.append((w, codes, 7))                 # NF4 stream
    rows, refs, outs = [], [], []
    for w, codes, M in specs:
        K, N = codes.shape
        A = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
        Cb = np.full((M, N), -7, np.int32)
        rows.append((w, M, A, Cb, 0))
        refs.append(O.gemm_i32(A, codes))
        outs.append(Cb)
    t = ork.tasks(ork.TaskI8, rows)
    rc = getattr(ork.lib(), entry)(npu.h, len(rows), t)
    assert rc == 0
    for i, (Cb, R) in enumerate(zip(outs, refs)):
        assert np.array_equal(Cb, R), (i, npu.plan_name(specs[i][0], specs[i][2]))
    for w, _, _ in specs:
        ork.free(w)


def test_i8_chain_cstride_and_device_operands(npu):
    _say("chain cstride + device")
    L = ork.lib()
    rng = np.random.default_rng(72)
    K, N, Nw = 512, 64, 96  # C rows of 96 elements, 64 written
    B1 = rng.integers(-128, 128, size=(K, N), dtype=np.int8)
    B2 = rng.integers(-128, 128, size=(K, N), dtype=np.int8)
    w1, w2 = npu.pack_i8(B1), npu.pack_i8(B2)
    A1 = rng.integers(-127, 128, size=(1, K), dtype=np.int8)
    A2 = rng.integers(-127, 128, size=(3, K), dtype=np.int8)
    # host C with a row stride: columns N..Nw-1 must stay untouched
    Ch = np.full((3, Nw), 12345, np.int32)
    # device-resident operands for the M=1 task, async mode on
    dA = L.ork_dev_alloc(npu.h, K)
    dC = L.ork_dev_alloc(npu.h, Nw * 4)
    assert dA and dC and L.ork_dev_upload(npu.h, dA, ork.ptr(A1), K) == 0
    L.ork_npu_set_async(npu.h, 1)
    try:
        t = ork.tasks(ork.TaskI8, [(w1, 1, dA, dC, Nw), (w2, 3, A2, Ch, Nw)])
        assert L.ork_i8_mm_run_chain(npu.h, 2, t) == 0
        assert L.ork_npu_sync(npu.h) == 0
    finally:
        L.ork_npu_set_async(npu.h, 0)
    C1 = np.empty((1, N), np.int32)
    assert L.ork_dev_download(npu.h, ork.ptr(C1), dC, N * 4) == 0
    assert np.array_equal(C1, O.gemm_i32(A1, B1))
    assert np.array_equal(Ch[:, :N], O.gemm_i32(A2, B2)) and np.all(Ch[:, N:] == 12345)
    L.ork_dev_free(npu.h, dA)
    L.ork_dev_free(npu.h, dC)
    ork.free(w1)
    ork.free(w2)


@pytest.mark.parametrize("rows_big", [40, 300])
def test_i8_chain_host_c_staging(npu, rows_big):
    """Host C of a chain below and above the 1 MiB pinned-staging limit (kernels write pinned memory, or HBM
    staging with strided copies back), with a C row stride; a second call reuses the grown staging."""
    _say("chain host C", rows_big)
    rng = np.random.default_rng(73)
    K, N, Nw = 256, 1024, 1040
    Bs = [rng.integers(-128, 128, size=(K, N), dtype=np.int8) for _ in range(3)]
    ws = [npu.pack_i8(B) for B in Bs]
    for rep in range(2):
        Ms = [1, rows_big, 3 + rep]
        As = [rng.integers(-127, 128, size=(M, K), dtype=np.int8) for M in Ms]
        Cs = [np.full((M, Nw), 777, np.int32) for M in Ms]
        t = ork.tasks(ork.TaskI8, [(w, M, A, C, Nw) for w, M, A, C in zip(ws, Ms, As, Cs)])
        assert ork.lib().ork_i8_mm_run_chain(npu.h, 3, t) == 0
        for A, B, C in zip(As, Bs, Cs):
            assert np.array_equal(C[:, :N], O.gemm_i32(A, B)) and np.all(C[:, N:] == 777)
    for w in ws:
        ork.free(w)


@pytest.mark.parametrize("entry", ["ork_i8_mm_run_chain", "ork_i8_mm_run_stream"])
def test_i8_chain_grouped_tiled(npu, entry):
    """Tasks of one kind, M > 1 and K run as one grouped tiled launch (up to 8 per launch, under the tile planned for
    their summed columns): every result exact against the oracle, as its single run. A prefill's q/k/v shapes, N tails,
    more tasks of one shape than a launch holds, uniform-int4 and NF4 pairs, a C row stride, and tasks of other
    shapes between them."""
    _say(entry, "grouped tiled")
    rng = np.random.default_rng(74)
    specs = []  # (w, codes[K][N], M, cstride)
    for M, K, N in [(128, 2048, 2048), (128, 2048, 1024), (40, 512, 96), (128, 2048, 1024), (96, 512, 416),
                    (96, 512, 32), (96, 512, 96), (130, 1056, 64)] + [(70, 256, 160)] * 9:
        B = rng.integers(-128, 128, size=(K, N), dtype=np.int8)
        specs.append((npu.pack_i8(B), B, M, N + (16 if M == 96 else 0)))
    for nf4 in (0, 1):
        for N in (256, 512):
            w, codes = _i4a8(npu, rng, 1024, N, nf4)
            specs.append((w, codes, 200, N))
    rows, refs, outs = [], [], []
    for w, codes, M, ldc in specs:
        assert w
        K, N = codes.shape
        A = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
        Cb = np.full((M, ldc), -7, np.int32)
        rows.append((w, M, A, Cb, ldc))
        refs.append(O.gemm_i32(A, codes))
        outs.append(Cb)
    t = ork.tasks(ork.TaskI8, rows)
    assert getattr(ork.lib(), entry)(npu.h, len(rows), t) == 0
    for i, (Cb, R) in enumerate(zip(outs, refs)):
        N = R.shape[1]
        assert np.array_equal(Cb[:, :N], R), (i, specs[i][2], R.shape)
        assert np.all(Cb[:, N:] == -7), i
    for w, *_ in specs:
        ork.free(w)


@pytest.mark.parametrize("entry", ["ork_i4_mm_run_chain", "ork_i4_mm_run_stream"])
def test_i4_chain(npu, entry):
    _say(entry)
    rows, refs, ws = [], [], []
    for M, K, N in [(1, 2048, 256), (1, 64, 64), (3, 512, 128), (1, 12288, 64), (128, 512, 256), (128, 512, 512),
                    (128, 512, 64)]:
        A, B = O.gen_i4_test(M, K, N)
        w = npu.pack_i4(B)
        assert w
        Cb = np.zeros((M, N), np.int32)
        rows.append((w, M, A, Cb))
        refs.append(O.gemm_i32(A, B))
        ws.append(w)
    t = ork.tasks(ork.TaskI4, rows)
    assert getattr(ork.lib(), entry)(npu.h, len(rows), t) == 0
    for (w, M, A, Cb), R in zip(rows, refs):
        assert np.array_equal(Cb, R), (M, A.shape)
    for w in ws:
        ork.free(w)


def test_f16_stream(npu):
    _say("f16 stream")
    rng = np.random.default_rng(73)
    rows, refs, ws = [], [], []
    for M, K, N in [(1, 2048, 512), (1, 96, 48), (1, 4096, 16), (16, 1024, 256), (130, 512, 128)]:
        A = rng.standard_normal((M, K)).astype(np.float16)
        B = (rng.standard_normal((K, N)) * 0.02).astype(np.float16)
        w = npu.pack_f16(B)
        Cb = np.zeros((M, N), np.float32)
        rows.append((w, M, A, Cb))
        refs.append(O.gemm_f16_f64acc(A, B))
        ws.append(w)
    t = ork.tasks(ork.TaskF16, rows)
    assert ork.lib().ork_f16_mm_run_stream(npu.h, len(rows), t) == 0
    for (w, M, A, Cb), R in zip(rows, refs):
        assert O.fp16_err(Cb, R) <= FP16_TOL, (M, A.shape)
    for w in ws:
        ork.free(w)


def test_f16_stream_equals_single_runs(npu):
    """An fp16 stream gives each task exactly its single run's result (include/ork/chain.h: results identical to S
    single runs): fp32 sums in the same order, whether the task's own M = 1 plan is the half-panel GEMV (which the
    grouped whole-panel launch would sum in another order, so such tasks launch with their own plans) or whole
    panels (which group). Bit for bit, not to a tolerance."""
    _say("f16 stream = single runs, bit for bit")
    rng = np.random.default_rng(77)
    shapes = [(1, 2048, 512), (1, 2048, 6144), (1, 2048, 4096), (1, 6144, 2048), (1, 96, 48), (1, 4096, 16),
              (16, 1024, 256), (1, 2048, 2048)]
    rows, singles, ws = [], [], []
    for M, K, N in shapes:
        A = rng.standard_normal((M, K)).astype(np.float16)
        B = (rng.standard_normal((K, N)) * 0.02).astype(np.float16)
        w = npu.pack_f16(B)
        rc, Cs = npu.run_f16(w, A)
        assert rc == 0
        rows.append((w, M, A, np.zeros((M, N), np.float32)))
        singles.append((Cs, npu.plan_name(w, M)))
        ws.append(w)
    assert ork.lib().ork_f16_mm_run_stream(npu.h, len(rows), ork.tasks(ork.TaskF16, rows)) == 0
    for (w, M, A, Cb), (Cs, name) in zip(rows, singles):
        assert np.array_equal(Cb.view(np.uint32), Cs.view(np.uint32)), (A.shape, name)
    for w in ws:
        ork.free(w)


def test_chain_errors(npu):
    _say("chain errors")
    L = ork.lib()
    rng = np.random.default_rng(74)
    B = rng.integers(-128, 128, size=(64, 64), dtype=np.int8)
    w = npu.pack_i8(B)
    wf = npu.pack_f16(np.zeros((64, 64), np.float16))
    A = np.zeros((2, 64), np.int8)
    Cb = np.zeros((2, 64), np.int32)
    assert L.ork_i8_mm_run_chain(npu.h, 1, ork.tasks(ork.TaskI8, [(None, 1, A, Cb)])) == -2
    assert L.ork_i8_mm_run_chain(npu.h, 1, ork.tasks(ork.TaskI8, [(w, 0, A, Cb)])) == -2
    assert L.ork_i8_mm_run_chain(npu.h, 1, ork.tasks(ork.TaskI8, [(wf, 1, A, Cb)])) == -2   # dtype
    assert L.ork_i8_mm_run_chain(npu.h, 1, ork.tasks(ork.TaskI8, [(w, 1, A, Cb, 32)])) == -2  # cstride < N
    assert L.ork_i8_mm_run_chain(npu.h, 0, ork.tasks(ork.TaskI8, [(w, 1, A, Cb)])) == -2
    buf = np.zeros(64 * 4 * 4, np.int8)   # C overlapping A
    assert L.ork_i8_mm_run_chain(npu.h, 1, ork.tasks(ork.TaskI8, [(w, 1, buf[:64], buf.ctypes.data)])) == -1
    ork.free(w)
    ork.free(wf)


def _random_chains(n=24, seed=0x63686E):
    rng = np.random.default_rng(seed)
    out = []
    for c in range(n):
        S = int(rng.integers(1, 9))
        M = int(rng.choice([1, 3, 16, 33, 64, 65, 100, 128, 200, 256]))
        K = 32 * int(rng.integers(1, 65))
        kind = ["i8", "u4", "nf4"][c % 3]
        tasks = [(int(rng.choice([1, 5, 70])) if rng.random() < 0.2 else M, 32 * int(rng.integers(1, 97)))
                 for _ in range(S)]
        out.append((c, kind, K, tasks))
    return out


@pytest.mark.parametrize("c,kind,K,tasks", _random_chains())
def test_i8_chain_random(npu, c, kind, K, tasks):
    """Seeded random chains at default plans: runs of tasks sharing M and K (one grouped tiled launch when their
    summed columns plan to the LDS-ring kernel), M = 1 tasks (one grouped GEMV launch), odd ones out; every task
    bit-exact against the oracle."""
    _say("random chain", c, kind, K, tasks)
    rng = np.random.default_rng(500 + c)
    rows, refs, outs, ws = [], [], [], []
    for M, N in tasks:
        if kind == "i8":
            codes = rng.integers(-128, 128, size=(K, N), dtype=np.int8)
            w = npu.pack_i8(codes)
        else:
            w, codes = _i4a8(npu, rng, K, N, kind == "nf4")
        assert w
        A = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
        Cb = np.full((M, N), -7, np.int32)
        rows.append((w, M, A, Cb, 0))
        refs.append(O.gemm_i32(A, codes))
        outs.append(Cb)
        ws.append((w, M))
    assert ork.lib().ork_i8_mm_run_chain(npu.h, len(rows), ork.tasks(ork.TaskI8, rows)) == 0
    for i, (Cb, R) in enumerate(zip(outs, refs)):
        assert np.array_equal(Cb, R), (i, npu.plan_name(*ws[i]))
    for w, _ in ws:
        ork.free(w)
