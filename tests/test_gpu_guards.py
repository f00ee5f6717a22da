"""Guard bands around every device write of the run path.

An off-by-one store past C, past an edge tile or past a split-K partial would pass every exact-C comparison, so
here C lives in a device buffer with GUARD bytes of a fixed pattern on each side (and, for a C row stride, between
the rows), and the pattern must come back untouched. The reference checks the same property with its extent guard
(src/npu/internal.h:302-307). The split-K partials live in the library's own workspace, so these runs use a context
made with ORK_WS_GUARD (a test knob honoured only with ORK_PLAN_DEBUG): it stages the partials between two guard
bands and fails the run (-1) when a kernel wrote into them.

Covered: the M = 1 GEMV (half and whole panels, split K), the streaming MFMA kernel (one panel and paired panels,
row tails, split K), the LDS-ring tiles with M and N tails (every tile on offer, split K), the older LDS kernel,
fp16 / uniform int4 / NF4 / W4A4 panels, the grouped-scale kernels (one row, streaming, LDS ring), the multi-matmul
submit with a C row stride, and the no-allocation entry point. Results are checked against the oracle as well.
"""
import os

import numpy as np
import pytest

import oracle as O
import ork

pytestmark = pytest.mark.gpu

GUARD = 4096                               # bytes each side
PAT = np.frombuffer(bytes((0x5A ^ (i * 37)) & 0xFF for i in range(251)), np.uint8)


def _say(*a):
    print("[case]", *a, flush=True)


class _env:
    def __init__(self, kv):
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


@pytest.fixture(scope="module")
def gnpu():
    """A context whose split-K workspace is guarded (ORK_WS_GUARD is read when the context is made)."""
    with _env({"ORK_PLAN_DEBUG": 1, "ORK_WS_GUARD": 1}):
        ctx = ork.Npu()
    yield ctx
    ctx.close()


def _pattern(n):
    return np.resize(PAT, n)


class Guarded:
    """A device buffer [GUARD | body | GUARD] filled with the pattern; .c is the body's device address."""

    def __init__(self, npu, body_bytes):
        self.npu, self.n = npu, body_bytes
        self.L = ork.lib()
        self.total = GUARD + body_bytes + GUARD
        self.base = self.L.ork_dev_alloc(npu.h, self.total)
        assert self.base
        self.init = _pattern(self.total)
        assert self.L.ork_dev_upload(npu.h, self.base, ork.ptr(self.init), self.total) == 0
        self.c = self.base + GUARD

    def read(self):
        out = np.empty(self.total, np.uint8)
        assert self.L.ork_dev_download(self.npu.h, ork.ptr(out), self.base, self.total) == 0
        return out

    def check(self, got, what):
        assert np.array_equal(got[:GUARD], self.init[:GUARD]), f"{what}: guard before C written"
        assert np.array_equal(got[-GUARD:], self.init[-GUARD:]), f"{what}: guard after C written"

    def free(self):
        self.L.ork_dev_free(self.npu.h, self.base)


def _dev(npu, a):
    L = ork.lib()
    d = L.ork_dev_alloc(npu.h, max(a.nbytes, 16))
    assert d and L.ork_dev_upload(npu.h, d, ork.ptr(a), a.nbytes) == 0
    return d


def _weight(npu, kind, K, N, rng):
    """(weight, run entry, A generator, oracle C(A))"""
    L = ork.lib()
    if kind == "i8":
        B = rng.integers(-128, 128, size=(K, N), dtype=np.int8)
        return npu.pack_i8(B), L.ork_i8_mm_run, lambda M: rng.integers(-128, 128, size=(M, K), dtype=np.int8), \
            lambda A: O.gemm_i32(A, B)
    if kind == "w4a4":
        B = rng.integers(-8, 8, size=(K, N), dtype=np.int8)
        return npu.pack_i4(B), L.ork_i4_mm_run, lambda M: rng.integers(-8, 8, size=(M, K), dtype=np.int8), \
            lambda A: O.gemm_i32(A, B)
    if kind in ("i4u", "nf4"):
        W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
        with _env({"ORK_NF4": 1} if kind == "nf4" else {}):
            w, _ = npu.pack_i4a8(W)
        _, _, codes = O.pack_i4a8(W, nf4=kind == "nf4")
        return w, L.ork_i8_mm_run, lambda M: rng.integers(-127, 128, size=(M, K), dtype=np.int8), \
            lambda A: O.gemm_i32(A, codes)
    assert kind == "f16"
    B = (rng.standard_normal((K, N)) * 0.02).astype(np.float16)
    return npu.pack_f16(B), L.ork_f16_mm_run, lambda M: rng.standard_normal((M, K)).astype(np.float16), \
        lambda A: O.gemm_f16_f64acc(A, B)


# (kind, M, K, N, plan knobs, what the plan name must contain)
CASES = [
    ("i8", 1, 2048, 6144, {}, "gemvh_"),
    ("i8", 1, 2048, 6144, {"ORK_GEMV_HALF": 0}, "gemv_"),
    ("i8", 1, 4096, 96, {"ORK_KSPLIT": 4}, "_ks4"),
    ("f16", 1, 2048, 48, {}, "gemv"),
    ("f16", 1, 4096, 80, {"ORK_KSPLIT": 2}, "_ks2"),
    ("i4u", 1, 2048, 160, {}, "gemv"),
    ("nf4", 1, 4096, 96, {"ORK_KSPLIT": 2}, "_ks2"),
    ("w4a4", 1, 4096, 128, {}, "gemv"),
    ("i8", 16, 2048, 6144, {"ORK_PLAN": "stream"}, "_p2"),
    ("i8", 16, 2048, 6144, {"ORK_PLAN": "stream", "ORK_STREAM_NP": 1}, "stream_"),
    ("i8", 37, 2048, 96, {"ORK_PLAN": "stream", "ORK_KSPLIT": 2}, "stream_i8_mt3"),
    ("f16", 9, 1024, 80, {"ORK_PLAN": "stream"}, "stream_f16"),
    ("nf4", 20, 2048, 160, {"ORK_PLAN": "stream"}, "stream_nf4"),
    ("f16", 16, 2048, 768, {}, "stream_f16_mt1_w8_kbw8_ks1_h"),
    ("i8", 37, 2048, 96, {"ORK_PLAN": "stream", "ORK_STREAM_HALF": 1, "ORK_KSPLIT": 2}, "_ks2_h"),
    ("w4a4", 21, 1024, 128, {"ORK_PLAN": "stream", "ORK_STREAM_HALF": 1}, "_h"),
    ("i8", 130, 2048, 4128, {"ORK_TILE": "64x192"}, "64x192"),
    ("i8", 200, 1024, 4128, {"ORK_TILE": "128x128"}, "128x128"),
    ("i8", 300, 1024, 544, {"ORK_TILE": "256x256"}, "256x256"),
    ("i8", 1100, 1056, 3072, {"ORK_TILE": "64x192"}, "64x192_al_r2"),
    ("i8", 300, 1024, 4128, {"ORK_TILE": "64x192", "ORK_CWT": 0}, "64x192"),
    ("f16", 130, 1024, 80, {"ORK_TILE": "64x64", "ORK_CWT": 0}, "tiled2_f16_64x64"),
    ("w4a4", 150, 1024, 320, {"ORK_TILE": "64x64", "ORK_CWT": 0}, "tiled2_i4u_64x64"),
    ("f16", 300, 1024, 544, {"ORK_TILE": "128x128", "ORK_RING": 2}, "128x128_al_r2"),
    ("i8", 70, 2048, 96, {"ORK_TILE": "64x64", "ORK_KSPLIT": 4}, "64x64_ks4"),
    ("i8", 40, 2048, 96, {"ORK_TILE": "32x64"}, "32x64"),
    ("i8", 40, 1024, 96, {"ORK_TILE": "32x32", "ORK_KSPLIT": 2}, "32x32_ks2"),
    ("i8", 21, 1024, 96, {"ORK_TILE": "16x64"}, "16x64"),
    ("i8", 21, 1024, 96, {"ORK_TILE": "16x32"}, "16x32"),
    ("i8", 100, 1024, 96, {"ORK_TILE": "128x96"}, "128x96"),
    ("f16", 130, 1024, 80, {"ORK_TILE": "64x64"}, "tiled2_f16_64x64"),
    ("f16", 70, 1024, 80, {"ORK_TILE": "32x32", "ORK_KSPLIT": 2}, "tiled2_f16_32x32_ks2"),
    ("i4u", 100, 2048, 160, {"ORK_TILE": "64x192"}, "tiled2_i4u_64x192"),
    ("w4a4", 100, 1024, 192, {"ORK_TILE": "64x64"}, "tiled2_i4u_64x64"),
    ("nf4", 150, 1024, 96, {"ORK_TILE": "64x64"}, "tiled2_nf4_64x64"),
    ("nf4", 60, 2048, 96, {"ORK_TILE": "32x64"}, "tiled2_nf4_32x64"),
    ("nf4", 60, 2048, 96, {}, "_nf4_"),
    ("nf4", 100, 1024, 96, {"ORK_PLAN": "tiled"}, "tiled_nf4"),
    ("nf4", 100, 1024, 96, {"ORK_PLAN": "tiled", "ORK_TILE": "128x96"}, "tiled_nf4_128x96"),
    ("i8", 100, 1024, 96, {"ORK_PLAN": "tiled"}, "tiled_i8"),
]


@pytest.mark.parametrize("i", range(len(CASES)))
def test_run_guards(gnpu, i):
    kind, M, K, N, env, want = CASES[i]
    rng = np.random.default_rng(900 + i)
    w, run, gen_a, ref = _weight(gnpu, kind, K, N, rng)
    assert w
    with _env(env):
        name = gnpu.plan_name(w, M)
    _say("guards", kind, M, K, N, env, name)
    assert want in name, (name, want)
    A = gen_a(M)
    esz = 4
    g = Guarded(gnpu, M * N * esz)
    dA = _dev(gnpu, A)
    try:
        with _env(env):
            assert run(gnpu.h, w, M, dA, g.c) == 0, name     # -1 would also mean a split-K guard band was written
        got = g.read()
        g.check(got, name)
        C = got[GUARD:GUARD + M * N * esz].view(np.float32 if kind == "f16" else np.int32).reshape(M, N)
        if kind == "f16":
            assert O.fp16_err(C, ref(A)) <= 2e-3, name
        else:
            assert np.array_equal(C, ref(A)), name
    finally:
        g.free()
        ork.lib().ork_dev_free(gnpu.h, dA)
        ork.free(w)


def test_host_c_guards(gnpu):
    """A host C (pinned staging up to 1 MiB, HBM staging and a D2H copy above) comes back into exactly its bytes."""
    rng = np.random.default_rng(950)
    for M, K, N in [(3, 1024, 160), (130, 1024, 4128)]:
        w, run, gen_a, ref = _weight(gnpu, "i8", K, N, rng)
        A = gen_a(M)
        body = M * N * 4
        buf = _pattern(GUARD + body + GUARD).copy()
        Cv = buf[GUARD:GUARD + body].view(np.int32)
        _say("host C guards", M, K, N, gnpu.plan_name(w, M))
        assert run(gnpu.h, w, M, ork.ptr(A), Cv.ctypes.data) == 0
        init = _pattern(GUARD + body + GUARD)
        assert np.array_equal(buf[:GUARD], init[:GUARD]) and np.array_equal(buf[-GUARD:], init[-GUARD:])
        assert np.array_equal(Cv.reshape(M, N), ref(A))
        ork.free(w)


@pytest.mark.parametrize("M,K,N,G,env,want", [
    (1, 2048, 160, 128, {}, "gemvh"),
    (8, 2048, 160, 64, {}, "grouped_i8_mt"),
    (100, 2080, 224, 160, {"ORK_PLAN": "tiled", "ORK_TILE": "64x64"}, "tiled2g_i8_64x64"),
    (70, 2048, 224, 512, {"ORK_PLAN": "tiled", "ORK_TILE": "64x192"}, "tiled2g_i8_64x192"),
])
def test_grouped_guards(gnpu, M, K, N, G, env, want):
    L = ork.lib()
    rng = np.random.default_rng(M + K + N + G)
    B = rng.integers(-128, 128, size=(K, N), dtype=np.int8)
    A = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
    aS = rng.uniform(1e-3, 1e-2, size=(M, K // G)).astype(np.float32)
    bS = rng.uniform(1e-3, 1e-2, size=(K // G, N)).astype(np.float32)
    w = gnpu.pack_i8(B)
    assert L.ork_w_set_group(w, G) == 0
    with _env(env):
        name = gnpu.grouped_plan_name(w, M)
    _say("grouped guards", M, K, N, G, name)
    assert want in name, name
    g = Guarded(gnpu, M * N * 4)
    dA, daS, dbS = _dev(gnpu, A), _dev(gnpu, aS), _dev(gnpu, bS)
    try:
        with _env(env):
            assert L.ork_i8_mm_run_grouped(gnpu.h, w, M, dA, daS, dbS, g.c) == 0
        got = g.read()
        g.check(got, name)
        C = got[GUARD:GUARD + M * N * 4].view(np.float32).reshape(M, N)
        assert np.array_equal(C, O.gemm_grouped(A, B, aS, bS, G)), name
    finally:
        g.free()
        for d in (dA, daS, dbS):
            L.ork_dev_free(gnpu.h, d)
        L.ork_mm_free(gnpu.h, w)


@pytest.mark.parametrize("shift", [0, 4, 8])
@pytest.mark.parametrize("M", [150, 64])
@pytest.mark.parametrize("kind,tile", [("w4a4", "64x64"), ("f16", "32x32")])
def test_allwave_epilogue_c_alignment_guards(gnpu, shift, M, kind, tile):
    """The tiles whose 16 waves all store C (W4A4 64 x 64, fp16 32 x 32: 16 bytes a thread where C is 16-byte
    aligned, else a word at a time) into a C that starts 0, 4 or 8 bytes past a 16-byte boundary: exact (fp16:
    within its bar), and the bytes either side untouched. M = 150 leaves a partial row tile; N = 320 five panels
    of 64."""
    rng = np.random.default_rng(980 + shift + M + len(kind))
    K, N = 1024, 320
    w, run, gen_a, ref = _weight(gnpu, kind, K, N, rng)
    A = gen_a(M)
    g = Guarded(gnpu, M * N * 4 + 16)
    dA = _dev(gnpu, A)
    try:
        with _env({"ORK_TILE": tile}):
            name = gnpu.plan_name(w, M)
            _say("all-wave epilogue C alignment", kind, M, shift, name)
            base = ("tiled2_i4u_" if kind == "w4a4" else "tiled2_f16_") + tile
            assert name in (base, base + "_al"), name   # either A-stage layout: the C stores are the same
            assert run(gnpu.h, w, M, dA, g.c + shift) == 0
        got = g.read()
        g.check(got, name)
        body = got[GUARD:GUARD + M * N * 4 + 16]
        init = g.init[GUARD:GUARD + M * N * 4 + 16]
        assert np.array_equal(body[:shift], init[:shift]) and np.array_equal(body[shift + M * N * 4:],
                                                                               init[shift + M * N * 4:])
        if kind == "f16":
            assert O.fp16_err(body[shift:shift + M * N * 4].view(np.float32).reshape(M, N), ref(A)) <= 2e-3
        else:
            assert np.array_equal(body[shift:shift + M * N * 4].view(np.int32).reshape(M, N), ref(A))
    finally:
        g.free()
        ork.lib().ork_dev_free(gnpu.h, dA)
        ork.free(w)


@pytest.mark.parametrize("ld", [1024 + 96, 1024 + 97])
def test_chain_cstride_guards(gnpu, ld):
    """Three int8 tasks writing into one device C at row stride `ld` (the reference's cstride): a grouped one-row
    launch, a grouped LDS-ring launch of two M = 64 tasks sharing K, and a split-K task launched on its own (its
    partials between the workspace's guard bands); a row stride that keeps every row 16-byte aligned and one that
    does not (the tile epilogue's vector and scalar stores). Every
    byte of the buffer outside each task's M x N block (the guards, the gaps at the end of each row, the columns of
    the other tasks) keeps the pattern."""
    L = ork.lib()
    rng = np.random.default_rng(960)
    specs = [(1, 2048, 512, 0), (64, 2048, 384, 512), (64, 2048, 160, 512 + 384), (40, 4096, 64, 0)]
    rows = sum(m for m, _, _, _ in specs)
    g = Guarded(gnpu, rows * ld * 4)
    tasks, refs, devs, ws = [], [], [], []
    r0 = 0
    try:
        for M, K, N, col in specs:
            B = rng.integers(-128, 128, size=(K, N), dtype=np.int8)
            A = rng.integers(-128, 128, size=(M, K), dtype=np.int8)
            w = gnpu.pack_i8(B)
            dA = _dev(gnpu, A)
            devs.append(dA)
            ws.append(w)
            tasks.append((w, M, dA, g.c + (r0 * ld + col) * 4, ld))
            refs.append((r0, col, M, N, O.gemm_i32(A, B)))
            r0 += M
        names = [gnpu.plan_name(t[0], t[1]) for t in tasks]
        _say("chain cstride guards", names)
        assert "_ks1" not in names[-1] and "_ks" in names[-1], names    # the last task's partials are guarded
        assert L.ork_i8_mm_run_chain(gnpu.h, len(tasks), ork.tasks(ork.TaskI8, tasks)) == 0
        got = g.read()
        g.check(got, "chain")
        body = got[GUARD:GUARD + rows * ld * 4].view(np.int32).reshape(rows, ld).copy()
        init = g.init[GUARD:GUARD + rows * ld * 4].view(np.int32).reshape(rows, ld)
        touched = np.zeros_like(body, bool)
        for r0, col, M, N, R in refs:
            assert np.array_equal(body[r0:r0 + M, col:col + N], R), (r0, col, M, N)
            touched[r0:r0 + M, col:col + N] = True
        assert np.array_equal(body[~touched], init[~touched]), "a chain task wrote outside its block"
    finally:
        g.free()
        for d in devs:
            L.ork_dev_free(gnpu.h, d)
        for w in ws:
            ork.free(w)


def test_noalloc_guards(gnpu):
    """The no-allocation entry point at a forced split: C guard bands, and the scratch array's partials between
    guard bands (the context's ORK_WS_GUARD applies there too)."""
    L = ork.lib()
    rng = np.random.default_rng(970)
    M, K, N = 37, 4096, 96
    B = rng.integers(-128, 128, size=(K, N), dtype=np.int8)
    A = rng.integers(-128, 128, size=(M, K), dtype=np.int8)
    w = gnpu.pack_i8(B)
    g = Guarded(gnpu, M * N * 4)
    dA = _dev(gnpu, A)
    try:
        for env in ({"ORK_PLAN": "stream", "ORK_KSPLIT": 4}, {"ORK_TILE": "32x32", "ORK_KSPLIT": 2}):
            with _env(env):
                name = gnpu.plan_name(w, M)
                _say("noalloc guards", name)
                assert L.ork_i8_mm_run_noalloc(gnpu.h, w, M, dA, g.c) == 0, name
            got = g.read()
            g.check(got, name)
            assert np.array_equal(got[GUARD:GUARD + M * N * 4].view(np.int32).reshape(M, N), O.gemm_i32(A, B)), name
    finally:
        g.free()
        L.ork_dev_free(gnpu.h, dA)
        ork.free(w)
