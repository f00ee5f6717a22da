"""GPU parity of the one-row run with a fused prologue and epilogue (ork_i8_mm_run_row, include/ork/hip.h).

Against oracle/rowops_ref.py, a numpy float32 restatement of the documented row operations in their documented
order (RMSNorm's sum of squares over 512 threads, the per-row int8 quantisation of examples/quant.c:34-37) and of
the epilogues, with the int32 columns from the oracle's exact GEMM: the row scale and every int32 column bit for
bit, the residual add bit for bit, SwiGLU within a few ulp (numpy's float32 exp is not the GPU's expf). Every
built combination over int8, uniform int4 and NF4 weights, whole and half panels, K tails inside a block, a HIP
graph replay of the async call, and the refusals.
"""
import os

import numpy as np
import pytest

import oracle as O
import ork
import rowops_ref as R

pytestmark = pytest.mark.gpu
F32 = np.float32


def _say(*a):
    print("[case]", *a, flush=True)


class Dev:
    """Device buffers of one test, freed together."""

    def __init__(self, npu):
        self.npu, self.L, self.bufs = npu, ork.lib(), []

    def put(self, a):
        a = np.ascontiguousarray(a)
        d = self.L.ork_dev_alloc(self.npu.h, max(a.nbytes, 16))
        assert d and self.L.ork_dev_upload(self.npu.h, d, ork.ptr(a), a.nbytes) == 0
        self.bufs.append(d)
        return d

    def get(self, d, shape, dtype):
        out = np.empty(shape, dtype)
        assert self.L.ork_dev_download(self.npu.h, ork.ptr(out), d, out.nbytes) == 0
        return out

    def free(self):
        for d in self.bufs:
            self.L.ork_dev_free(self.npu.h, d)


def _weight(npu, kind, K, N, rng):
    """(weight, int8 codes [K][N])"""
    if kind == "i8":
        B = rng.integers(-127, 128, size=(K, N), dtype=np.int8)
        return npu.pack_i8(B), B
    W = (rng.standard_normal((N, K)) * 0.02).astype(F32)
    os.environ.pop("ORK_NF4", None)
    if kind == "nf4":
        os.environ["ORK_NF4"] = "1"
    try:
        w, _ = npu.pack_i4a8(W)
    finally:
        os.environ.pop("ORK_NF4", None)
    _, _, codes = O.pack_i4a8(W, nf4=kind == "nf4")
    return w, codes


def _row(rng, K):
    return (rng.standard_normal(K) * 0.7 + 0.05).astype(F32)


def _call(npu, ws, op):
    arr = (ork.C.c_void_p * len(ws))(*ws)
    return ork.lib().ork_i8_mm_run_row(npu.h, len(ws), arr, ork.C.byref(op))


@pytest.mark.parametrize("K,Ns", [(2048, (2048, 1024, 1024)), (1024, (4096,)), (1024, (6144,)), (1056, (96, 32)),
                                  (8192, (64,))])
def test_rmsnorm_store(npu, K, Ns):
    """RMSNORM + STORE (int8 weights: a decoder's q/k/v): row scale and int32 columns bit for bit."""
    rng = np.random.default_rng(K + sum(Ns))
    D = Dev(npu)
    ws, codes = zip(*[_weight(npu, "i8", K, N, rng) for N in Ns])
    try:
        row, nw = _row(rng, K), (1 + 0.02 * rng.standard_normal(K)).astype(F32)
        op = ork.RowOp()
        op.prologue, op.epilogue, op.eps = ork.ROW_RMSNORM, ork.COL_STORE, 1e-6
        op.row, op.norm_w, op.row_scale = D.put(row), D.put(nw), D.put(np.zeros(1, F32))
        for i, N in enumerate(Ns):
            op.C[i] = D.put(np.zeros(N, np.int32))
        _say("rmsnorm+store", K, Ns)
        assert _call(npu, ws, op) == 0
        a, s = R.prologue(row, nw, 1e-6)
        assert D.get(op.row_scale, 1, F32).view(np.uint32)[0] == np.array([s], F32).view(np.uint32)[0]
        for i, N in enumerate(Ns):
            assert np.array_equal(D.get(op.C[i], N, np.int32), R.gemv(a, codes[i])), (i, N)
    finally:
        D.free()
        for w in ws:
            ork.free(w)


@pytest.mark.parametrize("kind", ["i8", "i4u", "nf4"])
@pytest.mark.parametrize("K,N", [(2048, 2048), (6144, 2048), (2048, 4096), (4000, 160)])
def test_quant_resid(npu, kind, K, N):
    """QUANT + RESID (o and down of a decoder): x[n] += (c * s) * ws[n], bit for bit; the row is only read."""
    if kind != "i8" and K % 32:
        pytest.skip("w4a8 packs need K % 32")
    rng = np.random.default_rng(7 * K + N + len(kind))
    D = Dev(npu)
    w, codes = _weight(npu, kind, K, N, rng)
    try:
        row, x, wsc = _row(rng, K), rng.standard_normal(N).astype(F32), rng.uniform(1e-3, 2e-2, N).astype(F32)
        op = ork.RowOp()
        op.prologue, op.epilogue = ork.ROW_QUANT, ork.COL_RESID
        op.row, op.row_scale, op.out = D.put(row), D.put(np.zeros(1, F32)), D.put(x)
        op.w_scale[0] = D.put(wsc)
        _say("quant+resid", kind, K, N)
        assert _call(npu, [w], op) == 0
        a, s = R.prologue(row)
        want = R.resid(x, R.gemv(a, codes), s, wsc)
        assert np.array_equal(D.get(op.out, N, F32).view(np.uint32), want.view(np.uint32))
        assert np.array_equal(D.get(op.row, K, F32), row)
        assert D.get(op.row_scale, 1, F32)[0] == s
    finally:
        D.free()
        ork.free(w)


@pytest.mark.parametrize("kind", ["i8", "i4u", "nf4"])
@pytest.mark.parametrize("K,N", [(2048, 6144), (1024, 4096), (2048, 96)])
def test_rmsnorm_swiglu(npu, kind, K, N):
    """RMSNORM + SWIGLU (a gate/up pair): y = silu(g) * u within 4 ulp of the restatement (the exp differs)."""
    rng = np.random.default_rng(11 * K + N + len(kind))
    D = Dev(npu)
    (wg, cg), (wu, cu) = _weight(npu, kind, K, N, rng), _weight(npu, kind, K, N, rng)
    try:
        row, nw = _row(rng, K), (1 + 0.02 * rng.standard_normal(K)).astype(F32)
        wsg, wsu = rng.uniform(1e-3, 2e-2, N).astype(F32), rng.uniform(1e-3, 2e-2, N).astype(F32)
        op = ork.RowOp()
        op.prologue, op.epilogue, op.eps = ork.ROW_RMSNORM, ork.COL_SWIGLU, 1e-6
        op.row, op.norm_w, op.out = D.put(row), D.put(nw), D.put(np.zeros(N, F32))
        op.w_scale[0], op.w_scale[1] = D.put(wsg), D.put(wsu)
        _say("rmsnorm+swiglu", kind, K, N)
        assert _call(npu, [wg, wu], op) == 0
        a, s = R.prologue(row, nw, 1e-6)
        want = R.swiglu(R.gemv(a, cg), R.gemv(a, cu), s, wsg, wsu)
        got = D.get(op.out, N, F32)
        assert np.all(np.abs(got - want) <= 4 * np.spacing(np.abs(want)) + 1e-30), np.abs(got - want).max()
    finally:
        D.free()
        ork.free(wg)
        ork.free(wu)


def test_graph_replay_async(npu):
    """In async mode the call only enqueues: captured into a HIP graph and replayed twice, the residual row takes
    the add twice, bit for bit."""
    import hipgraph

    L = ork.lib()
    G = hipgraph.Graphs()
    rng = np.random.default_rng(5)
    K, N = 2048, 2048
    D = Dev(npu)
    w, codes = _weight(npu, "nf4", K, N, rng)
    row, x, wsc = _row(rng, K), rng.standard_normal(N).astype(F32), rng.uniform(1e-3, 2e-2, N).astype(F32)
    op = ork.RowOp()
    op.prologue, op.epilogue = ork.ROW_QUANT, ork.COL_RESID
    op.row, op.out = D.put(row), D.put(x)
    op.w_scale[0] = D.put(wsc)
    L.ork_npu_set_async(npu.h, 1)
    try:
        rc, g, ex = G.capture(L.ork_npu_stream(npu.h), lambda: _call(npu, [w], op))
        assert rc == 0
        try:
            stream = L.ork_npu_stream(npu.h)
            G.replay(ex, stream)
            G.replay(ex, stream)
        finally:
            G.destroy(g, ex)
        a, s = R.prologue(row)
        c = R.gemv(a, codes)
        want = R.resid(R.resid(x, c, s, wsc), c, s, wsc)
        assert np.array_equal(D.get(op.out, N, F32).view(np.uint32), want.view(np.uint32))
    finally:
        L.ork_npu_set_async(npu.h, 0)
        D.free()
        ork.free(w)


def test_refusals(npu):
    """-2 for what is not built or not allowed: STORE with nibble weights, an output overlapping the row, host
    operands, a weight count that does not fit the epilogue, K above the row bound, fp16 weights."""
    rng = np.random.default_rng(9)
    D = Dev(npu)
    w8, _ = _weight(npu, "i8", 1024, 256, rng)
    w4, _ = _weight(npu, "i4u", 1024, 256, rng)
    wbig = npu.pack_i8(np.zeros((8256, 64), np.int8))
    wf = npu.pack_f16(np.zeros((1024, 256), np.float16))
    try:
        row = D.put(_row(rng, 1024))
        buf = D.put(np.zeros(4096, F32))
        ws = D.put(np.ones(256, F32))
        st = ork.RowOp()
        st.prologue, st.epilogue, st.eps, st.row, st.norm_w = ork.ROW_RMSNORM, ork.COL_STORE, 1e-6, row, ws
        st.C[0] = buf
        assert _call(npu, [w4], st) == -2                       # STORE is built for int8 weights only
        assert _call(npu, [wf], st) == -2                       # fp16 weights
        assert _call(npu, [w8, w8, w8, w8], st) == -2           # S outside 1..3
        rs = ork.RowOp()
        rs.prologue, rs.epilogue, rs.row, rs.out = ork.ROW_QUANT, ork.COL_RESID, row, row   # out is the row
        rs.w_scale[0] = ws
        assert _call(npu, [w8], rs) == -2
        host = np.zeros(256, F32)
        rs.out = host.ctypes.data                               # host output
        assert _call(npu, [w8], rs) == -2
        rs.out = buf
        assert _call(npu, [w8, w8], rs) == -2                   # RESID takes one weight
        assert _call(npu, [w8], rs) == 0
        sw = ork.RowOp()
        sw.prologue, sw.epilogue, sw.eps, sw.row, sw.norm_w, sw.out = ork.ROW_RMSNORM, ork.COL_SWIGLU, 1e-6, row, ws, buf
        sw.w_scale[0] = sw.w_scale[1] = ws
        assert _call(npu, [w8, w4], sw) == -2                   # gate and up of different kinds
        assert _call(npu, [w8], sw) == -2                       # SWIGLU takes two
        big = ork.RowOp()
        big.prologue, big.epilogue, big.row, big.out = ork.ROW_QUANT, ork.COL_RESID, D.put(np.zeros(8256, F32)), buf
        big.w_scale[0] = D.put(np.ones(64, F32))
        assert _call(npu, [wbig], big) == -2                    # K above ORK_ROW_KMAX
    finally:
        D.free()
        for w in (w8, w4, wbig, wf):
            ork.free(w)
