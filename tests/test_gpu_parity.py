"""GPU parity: the HIP path through the C-ABI vs the CPU oracle and the reference's own goldens.

Bar: bit-exact int32 for every integer path (int8, i4a8 uniform/NF4, W4A4); fp16 within 2e-3 relative
error (per element, floored at 0.1% of the output range) of an fp64-accumulated reference, and
bit-exact where the reference's known-answer inputs make every fp32 partial sum exact.
"""
import os

import numpy as np
import pytest

import goldens as G
import oracle as O
import ork

pytestmark = pytest.mark.gpu

FP16_TOL = 2e-3  # north_star: max relative error of fp16 -> fp32 results vs fp64 accumulation


def _say(*a):
    print("[case]", *a, flush=True)


def _rng(seed):
    return np.random.default_rng(seed)


# ---------------------------------------------------------------------------------------------- int8
I8_SHAPES = [  # (M, K, N): stream and tiled paths, K tails (K%64 == 32), N tails vs the tile width
    (1, 32, 32), (1, 96, 64), (1, 2048, 6144), (2, 2048, 6144), (15, 160, 96), (16, 2048, 6144),
    (17, 1024, 128), (33, 2080, 224), (64, 4096, 512), (65, 512, 96), (100, 96, 1568), (128, 2048, 2048),
    (200, 1056, 416), (512, 2048, 6144), (300, 3072, 4096), (1, 12288, 64), (7, 10752, 160)]


@pytest.mark.parametrize("M,K,N", I8_SHAPES)
def test_i8_random_vs_oracle(npu, M, K, N):
    _say("i8", M, K, N)
    rng = _rng(M * 7 + K + N)
    B = rng.integers(-128, 128, size=(K, N), dtype=np.int8)
    A = rng.integers(-128, 128, size=(M, K), dtype=np.int8)
    w = npu.pack_i8(B)
    assert w
    rc, C = npu.run_i8(w, A)
    assert rc == 0
    assert np.array_equal(C, O.gemm_i32(A, B)), npu.plan_name(w, M)
    ork.free(w)


@pytest.mark.parametrize("M", [1, 16, 64, 512])
def test_i8_forced_algorithms_agree(npu, M):
    """The stream and tiled kernels give the same exact result on the same weight."""
    _say("i8 forced", M)
    rng = _rng(M)
    K, N = 1024, 768
    B = rng.integers(-127, 128, size=(K, N), dtype=np.int8)
    A = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
    w = npu.pack_i8(B)
    ref = O.gemm_i32(A, B)
    for algo in (["stream", "tiled"] if M <= 64 else ["tiled"]):
        os.environ["ORK_PLAN"] = algo
        try:
            rc, C = npu.run_i8(w, A)
        finally:
            del os.environ["ORK_PLAN"]
        assert rc == 0 and np.array_equal(C, ref), algo
    ork.free(w)


class _env:
    """Sets environment variables for the duration of a with-block (the planner reads them per call)."""

    def __init__(self, **kv):
        self.kv = kv

    def __enter__(self):
        for k, v in self.kv.items():
            os.environ[k] = str(v)

    def __exit__(self, *a):
        for k in self.kv:
            os.environ.pop(k, None)


@pytest.mark.parametrize("ks", [2, 3, 7, 64])
def test_forced_split_k_all_kinds(npu, ks):
    """K split across workgroups + the fixed-order reduce: exact for int8 / int4 (uniform and W4A4),
    within tolerance and run-to-run bit-identical for fp16. ks=64 exceeds the K-blocks of the int4
    shape and is clamped to one block per workgroup."""
    _say("split-k", ks)
    rng = _rng(ks)
    K, N = 2080, 128  # K % 64 == 32: a K tail in every kind; N % 64 == 0 for the W4A4 pack gate
    for M in (1, 13, 40):
        A = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
        B = rng.integers(-128, 128, size=(K, N), dtype=np.int8)
        w = npu.pack_i8(B)
        with _env(ORK_PLAN="stream", ORK_KSPLIT=ks):
            rc, C = npu.run_i8(w, A)
            KB = -(-K // 64)
            kbs = -(-KB // min(ks, KB))
            assert npu.plan_name(w, M).endswith(f"_ks{-(-KB // kbs)}"), npu.plan_name(w, M)
        assert rc == 0 and np.array_equal(C, O.gemm_i32(A, B)), ("i8", M, npu.plan_name(w, M))
        ork.free(w)

        A4, B4 = O.gen_i4_test(M, K, N)
        w = npu.pack_i4(B4)
        assert w
        with _env(ORK_PLAN="stream", ORK_KSPLIT=ks):
            rc, C = npu.run_i4(w, A4)
        assert rc == 0 and np.array_equal(C, O.gemm_i32(A4, B4)), ("w4a4", M)
        ork.free(w)

        Ah = rng.standard_normal((M, K)).astype(np.float16)
        Bh = (rng.standard_normal((K, N)) * 0.02).astype(np.float16)
        w = npu.pack_f16(Bh)
        with _env(ORK_PLAN="stream", ORK_KSPLIT=ks):
            rc, C1 = npu.run_f16(w, Ah)
            rc2, C2 = npu.run_f16(w, Ah)
        assert rc == 0 and rc2 == 0 and np.array_equal(C1, C2), ("f16 determinism", M)
        assert O.fp16_err(C1, O.gemm_f16_f64acc(Ah, Bh)) <= FP16_TOL, ("f16", M)
        ork.free(w)


@pytest.mark.parametrize("ks", [2, 3, 8])
def test_forced_tiled_split_k(npu, ks):
    """The tiled kernel with K split across workgroups (partials + fixed-order reduce): exact for int8 and
    int4, within tolerance and run-to-run identical for fp16; M and N tails included."""
    _say("tiled split-k", ks)
    rng = _rng(50 + ks)
    M, K, N = 200, 2080, 192
    A = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
    B = rng.integers(-128, 128, size=(K, N), dtype=np.int8)
    w = npu.pack_i8(B)
    with _env(ORK_PLAN="tiled", ORK_KSPLIT=ks):
        rc, C = npu.run_i8(w, A)
        assert "_ks" in npu.plan_name(w, M), npu.plan_name(w, M)
    assert rc == 0 and np.array_equal(C, O.gemm_i32(A, B)), ("i8", npu.plan_name(w, M))
    ork.free(w)
    A4, B4 = O.gen_i4_test(M, K, N)
    w = npu.pack_i4(B4)
    with _env(ORK_PLAN="tiled", ORK_KSPLIT=ks):
        rc, C = npu.run_i4(w, A4)
    assert rc == 0 and np.array_equal(C, O.gemm_i32(A4, B4)), "w4a4"
    ork.free(w)
    Ah = rng.standard_normal((M, K)).astype(np.float16)
    Bh = (rng.standard_normal((K, N)) * 0.02).astype(np.float16)
    w = npu.pack_f16(Bh)
    with _env(ORK_PLAN="tiled", ORK_KSPLIT=ks):
        rc, C1 = npu.run_f16(w, Ah)
        rc2, C2 = npu.run_f16(w, Ah)
    assert rc == 0 and rc2 == 0 and np.array_equal(C1, C2)
    assert O.fp16_err(C1, O.gemm_f16_f64acc(Ah, Bh)) <= FP16_TOL
    ork.free(w)


@pytest.mark.parametrize("idx", range(7))
def test_quant_c_goldens_on_gpu(npu, idx):
    """examples/quant.c end to end: ork_i8_mm_pack + ork_i8_mm_run, FNV-64 of C == the reference golden."""
    for M, K, N, Aq, Bq, gold, hm in G.quant_c_cases(select={idx}):
        _say("quant.c", M, K, N)
        w = npu.pack_i8(Bq)
        rc, C = npu.run_i8(w, Aq)
        assert rc == 0 and G.chained_hash(C, hm) == gold, (M, K, N)
        ork.free(w)


@pytest.mark.parametrize("shape", range(7))
def test_chain_prefill_goldens_on_gpu(npu, shape):
    for M, K, N, A, B, gold, hm in G.tm_chain_cases({shape}):
        _say("chain_prefill", M, K, N)
        w = npu.pack_i8(B)
        rc, C = npu.run_i8(w, A)
        assert rc == 0 and G.chained_hash(C, hm) == gold, (M, K, N)
        ork.free(w)


def test_check_i8_goldens_on_gpu(npu):
    for M, K, N, A, B, gold, hm in G.tm_check_i8_cases():
        _say("check_i8", M, K, N)
        w = npu.pack_i8(B)
        h = O.FNV_OFFSET
        for m in hm:  # the same resident weight run at M = 1, 1, 4, M (test_matmul.c:53-56)
            rc, C = npu.run_i8(w, A[:m])
            assert rc == 0
            h = O.fnv64(C, h)
        assert h == gold, (M, K, N)
        ork.free(w)


def test_i8_pack_f32_bscale_and_codes(npu):
    """ork_i8_mm_pack_f32: bscale bit-exact and the resident codes equal the oracle's (via C = I x B)."""
    rng = _rng(5)
    K, N = 2048, 512
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    W[3, :] = 0.0  # all-zero channel: mx = 1e-9 floor, codes all 0
    w, bs = npu.pack_i8_f32(W)
    codes, bs_ref = O.pack_i8_f32(W)
    assert np.array_equal(bs, bs_ref)
    A = np.zeros((64, K), np.int8)
    for i in range(64):
        A[i, i * 32] = 1  # row i selects k = 32*i
    rc, C = npu.run_i8(w, A)
    assert rc == 0 and np.array_equal(C, codes[::32, :].astype(np.int32))
    A2 = rng.integers(-127, 128, size=(8, K), dtype=np.int8)
    rc, C2 = npu.run_i8(w, A2)
    assert rc == 0 and np.array_equal(C2, O.gemm_i32(A2, codes))
    ork.free(w)


# -------------------------------------------------------------------------------------------- W4A8
def _i4a8_case(npu, K, N, M, nf4, imatrix, sr, seed):
    rng = _rng(seed)
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    im = rng.uniform(0.5, 2.0, K).astype(np.float32) if imatrix else None
    env = {"ORK_NF4": nf4, "ORK_SR": sr}
    for k, v in env.items():
        if v:
            os.environ[k] = "1"
    try:
        w, bs = npu.pack_i4a8(W, im)
    finally:
        for k in env:
            os.environ.pop(k, None)
    bs_ref, nib_ref, codes = O.pack_i4a8(W, im, nf4=nf4, sr=sr)
    return W, im, w, bs, bs_ref, codes, rng


@pytest.mark.parametrize("nf4", [0, 1])
@pytest.mark.parametrize("imatrix", [0, 1])
@pytest.mark.parametrize("M", [1, 5, 16, 64, 130])
def test_i4a8_vs_oracle(npu, nf4, imatrix, M):
    _say("i4a8", nf4, imatrix, M)
    K, N = 1024, 256
    W, im, w, bs, bs_ref, codes, rng = _i4a8_case(npu, K, N, M, nf4, imatrix, 0, 100 + M)
    assert w and np.array_equal(bs, bs_ref)
    assert ork.lib().ork_w_quant_kind(w) == (1 if nf4 else 0)
    A = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
    rc, C = npu.run_i8(w, A)
    assert rc == 0 and np.array_equal(C, O.gemm_i32(A, codes)), npu.plan_name(w, M)
    # O4N1 round trip: dump == the oracle's blob bytes, load runs bit-identically, re-dump identical
    blob = ork.dump_i4a8(w)
    assert np.array_equal(blob, O.i4a8_blob(W, im, nf4=nf4))
    w2 = npu.load_i4a8(K, N, blob)
    rc2, C2 = npu.run_i8(w2, A)
    assert rc2 == 0 and np.array_equal(C2, C)
    assert np.array_equal(ork.dump_i4a8(w2), blob)
    ork.free(w)
    ork.free(w2)


@pytest.mark.parametrize("nf4", [0, 1])
@pytest.mark.parametrize("imatrix", [0, 1])
def test_i4a8_stochastic_rounding(npu, nf4, imatrix):
    """ORK_SR (src/npu/i4/pack.c:32, quant.c:32-33 / :82-83): one xorshift32 stream across the channels in order;
    the device pack's bscale, nibble store (O4N1 bytes) and results equal the oracle's, uniform and NF4."""
    _say("i4a8 SR", nf4, imatrix)
    K, N, M = 512, 128, 8
    W, im, w, bs, bs_ref, codes, rng = _i4a8_case(npu, K, N, M, nf4, imatrix, 1, 9 + nf4 + 2 * imatrix)
    assert np.array_equal(bs, bs_ref)
    assert np.array_equal(ork.dump_i4a8(w), O.i4a8_blob(W, im, nf4=bool(nf4), sr=True))
    A = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
    rc, C = npu.run_i8(w, A)
    assert rc == 0 and np.array_equal(C, O.gemm_i32(A, codes))
    ork.free(w)


# -------------------------------------------------------------------------------------------- W4A4
I4_SHAPES = [  # examples/i4.c:95-136
    (1, 64, 64), (4, 128, 128), (2, 256, 64), (1, 12288, 64), (3, 2048, 256), (8, 512, 256), (16, 512, 64),
    (16, 2048, 64), (16, 2048, 256), (128, 512, 256), (256, 512, 256), (128, 512, 512), (20, 2048, 256),
    (100, 512, 512), (4, 2048, 256), (32, 1024, 128), (64, 512, 256)]


@pytest.mark.parametrize("M,K,N", I4_SHAPES)
def test_w4a4_i4c_shapes(npu, M, K, N):
    _say("w4a4", M, K, N)
    A, B = O.gen_i4_test(M, K, N)
    w = npu.pack_i4(B)
    assert w
    rc, C = npu.run_i4(w, A)
    assert rc == 0 and np.array_equal(C, O.gemm_i32(A, B)), npu.plan_name(w, M)
    ork.free(w)


def test_w4a4_sattest(npu):
    """examples/i4.c:37-58: one output cell is exactly 32767, reached without saturation."""
    M, K, N = 16, 2048, 256
    A, B = O.gen_i4_sattest(M, K, N)
    w = npu.pack_i4(B)
    rc, C = npu.run_i4(w, A)
    assert rc == 0 and C[0, 0] == 32767 and np.array_equal(C, O.gemm_i32(A, B))
    ork.free(w)


def test_w4a4_extremes(npu):
    """-8 x -8 everywhere: 64*K exactly (int4 range edges, the x16 widening at its limit)."""
    M, K, N = 70, 4096, 128
    A = np.full((M, K), -8, np.int8)
    B = np.full((K, N), -8, np.int8)
    w = npu.pack_i4(B)
    rc, C = npu.run_i4(w, A)
    assert rc == 0 and np.all(C == 64 * K)
    ork.free(w)


# -------------------------------------------------------------------------------------------- fp16
def test_fp16_goldens_on_gpu(npu):
    for M, K, N, A, B, gold, hm in G.tm_fp16_cases():
        _say("fp16 golden", M, K, N)
        w = npu.pack_f16(B)
        h = O.FNV_OFFSET
        for m in hm:
            rc, C = npu.run_f16(w, A[:m])
            assert rc == 0
            h = O.fnv64(C, h)
        assert h == gold, (M, K, N)
        ork.free(w)


@pytest.mark.parametrize("M", [1, 16, 128, 512])
def test_fp16_config_tolerance(npu, M):
    """A ~ N(0,1), B ~ N(0,0.02), K = N = 2048."""
    _say("fp16", M)
    rng = _rng(1000 + M)
    K = N = 2048
    A = rng.standard_normal((M, K)).astype(np.float16)
    B = (rng.standard_normal((K, N)) * 0.02).astype(np.float16)
    w = npu.pack_f16(B)
    rc, C = npu.run_f16(w, A)
    assert rc == 0
    err = O.fp16_err(C, O.gemm_f16_f64acc(A, B))
    assert err <= FP16_TOL, (err, npu.plan_name(w, M))
    ork.free(w)


@pytest.mark.parametrize("M,K,N", [(3, 96, 48), (65, 160, 112), (1, 4096, 16)])
def test_fp16_odd_shapes(npu, M, K, N):
    rng = _rng(M + K + N)
    A = rng.standard_normal((M, K)).astype(np.float16)
    B = rng.standard_normal((K, N)).astype(np.float16)
    w = npu.pack_f16(B)
    rc, C = npu.run_f16(w, A)
    assert rc == 0 and O.fp16_err(C, O.gemm_f16_f64acc(A, B)) <= FP16_TOL
    ork.free(w)


# ------------------------------------------------------------------------------ full-size properties
def test_m512_full_size_properties(npu):
    """The metric's M=512 int8 GEMM at full size: exact on sampled rows, and the column checksum
    sum_m C[m][n] == (sum_m A[m]) . B[:, n] (exact in int64) over every column."""
    rng = _rng(512)
    K, N, M = 2048, 6144, 512
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    w, _ = npu.pack_i8_f32(W)
    codes, _ = O.pack_i8_f32(W)
    A = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
    rc, C = npu.run_i8(w, A)
    assert rc == 0
    rows = np.r_[0:8, 250:262, 504:512]
    assert np.array_equal(C[rows], O.gemm_i32(A[rows], codes))
    colsum = A.astype(np.int64).sum(axis=0) @ codes.astype(np.int64)
    assert np.array_equal(C.astype(np.int64).sum(axis=0), colsum)
    ork.free(w)


def test_w4a4_config4_full(npu):
    """A int4[256,4096] x B int4[4096,4096], exact."""
    rng = _rng(44)
    M, K, N = 256, 4096, 4096
    A = rng.integers(-8, 8, size=(M, K), dtype=np.int8)
    B = rng.integers(-8, 8, size=(K, N), dtype=np.int8)
    w = npu.pack_i4(B)
    rc, C = npu.run_i4(w, A)
    assert rc == 0
    rows = np.r_[0:16, 120:136, 240:256]
    assert np.array_equal(C[rows], O.gemm_i32(A[rows], B))
    colsum = A.astype(np.int64).sum(axis=0) @ B.astype(np.int64)
    assert np.array_equal(C.astype(np.int64).sum(axis=0), colsum)
    ork.free(w)


# ---------------------------------------------------------------------------- residency / errors
def test_device_resident_operands_async(npu):
    L = ork.lib()
    rng = _rng(77)
    K, N, M = 2048, 6144, 1
    B = rng.integers(-127, 128, size=(K, N), dtype=np.int8)
    A = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
    w = npu.pack_i8(B)
    dA = L.ork_dev_alloc(npu.h, A.nbytes)
    dC = L.ork_dev_alloc(npu.h, M * N * 4)
    assert dA and dC
    assert L.ork_dev_upload(npu.h, dA, ork.ptr(A), A.nbytes) == 0
    L.ork_npu_set_async(npu.h, 1)
    for _ in range(3):
        assert L.ork_i8_mm_run(npu.h, w, M, dA, dC) == 0
    assert L.ork_npu_sync(npu.h) == 0
    L.ork_npu_set_async(npu.h, 0)
    C = np.empty((M, N), np.int32)
    assert L.ork_dev_download(npu.h, ork.ptr(C), dC, C.nbytes) == 0
    assert np.array_equal(C, O.gemm_i32(A, B))
    L.ork_dev_free(npu.h, dA)
    L.ork_dev_free(npu.h, dC)
    ork.free(w)


@pytest.mark.parametrize("nbytes", [16, 8192, 1_000_016, 12_582_912])
def test_read_probe_reads_every_byte(npu, nbytes):
    """ork_npu_read_probe (the benchmark's plain read of a weight's bytes): the XOR of its per-workgroup words
    equals the XOR of every 32-bit word of the buffer, at sizes with and without a partial last workgroup."""
    L = ork.lib()
    rng = _rng(nbytes % 997)
    host = rng.integers(0, 256, size=nbytes, dtype=np.uint8)
    dev = L.ork_dev_alloc(npu.h, nbytes)
    sink = L.ork_dev_alloc(npu.h, 4 * ((nbytes + 8191) // 8192))
    assert dev and sink
    assert L.ork_dev_upload(npu.h, dev, ork.ptr(host), nbytes) == 0
    n = L.ork_npu_read_probe(npu.h, dev, nbytes, sink)
    assert n == (nbytes + 8191) // 8192
    words = np.empty(n, np.uint32)
    assert L.ork_dev_download(npu.h, ork.ptr(words), sink, 4 * n) == 0
    assert np.bitwise_xor.reduce(words) == np.bitwise_xor.reduce(host.view(np.uint32))
    # refusals: a size that is not a multiple of 16, a misaligned start, host memory
    assert L.ork_npu_read_probe(npu.h, dev, 24, sink) == -1
    assert L.ork_npu_read_probe(npu.h, dev + 8, 16, sink) == -1
    assert L.ork_npu_read_probe(npu.h, ork.ptr(host), 16, sink) == -1
    L.ork_dev_free(npu.h, dev)
    L.ork_dev_free(npu.h, sink)


def test_dma_buffers(npu):
    import ctypes as Ct

    L = ork.lib()
    rng = _rng(78)
    K, N, M = 512, 256, 4
    B = rng.integers(-127, 128, size=(K, N), dtype=np.int8)
    A = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
    w = npu.pack_i8(B)
    pa = L.ork_dma_alloc(npu.h, A.nbytes)
    pc = L.ork_dma_alloc(npu.h, M * N * 4)
    Ct.memmove(pa, A.ctypes.data, A.nbytes)
    assert L.ork_i8_mm_run(npu.h, w, M, pa, pc) == 0
    C = np.ctypeslib.as_array(Ct.cast(pc, Ct.POINTER(Ct.c_int32)), shape=(M, N)).copy()
    assert np.array_equal(C, O.gemm_i32(A, B))
    L.ork_dma_free(npu.h, pa)
    L.ork_dma_free(npu.h, pc)
    ork.free(w)


@pytest.mark.parametrize("kind", ["i8", "f16"])
def test_host_operand_modes(npu, kind):
    """Host C on either side of the 1 MiB pinned-staging limit (written by the kernels into pinned memory, or
    staged in HBM and copied back), in both orders so the staging is grown and reused, and C / A placed at
    offsets inside ork_dma_alloc buffers (written and read in place)."""
    import ctypes as Ct

    L = ork.lib()
    rng = _rng(79)
    K, N = 256, 2048  # one C row is 8 KiB: M=128 is exactly 1 MiB
    if kind == "i8":
        B = rng.integers(-127, 128, size=(K, N), dtype=np.int8)
        w = npu.pack_i8(B)
        mk = lambda M: rng.integers(-127, 128, size=(M, K), dtype=np.int8)
        run, ref, ct = npu.run_i8, (lambda A: O.gemm_i32(A, B)), Ct.c_int32
    else:
        B = rng.integers(-3, 4, size=(K, N)).astype(np.float16)
        w = npu.pack_f16(B)
        mk = lambda M: rng.integers(-3, 4, size=(M, K)).astype(np.float16)  # integer-valued: exact in fp32
        run, ref, ct = npu.run_f16, (lambda A: (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32)), Ct.c_float
    for M in (1, 128, 129, 7, 300, 3):
        print(f"[case] host C {kind} M={M} ({M * N * 4} bytes)", flush=True)
        A = mk(M)
        rc, C = run(w, A)
        assert rc == 0
        assert np.array_equal(C, ref(A)), f"M={M}"
    M = 5
    A = mk(M)
    pa = L.ork_dma_alloc(npu.h, A.nbytes + 256)
    pc = L.ork_dma_alloc(npu.h, M * N * 4 + 4096)
    Ct.memmove(pa + 256, A.ctypes.data, A.nbytes)
    fn = L.ork_i8_mm_run if kind == "i8" else L.ork_f16_mm_run
    assert fn(npu.h, w, M, pa + 256, pc + 4096) == 0
    C = np.ctypeslib.as_array(Ct.cast(pc + 4096, Ct.POINTER(ct)), shape=(M, N)).copy()
    assert np.array_equal(C, ref(A))
    L.ork_dma_free(npu.h, pa)
    L.ork_dma_free(npu.h, pc)
    ork.free(w)


def test_run_errors(npu):
    import ctypes as Ct

    L = ork.lib()
    B = np.ones((64, 64), np.int8)
    wi8 = npu.pack_i8(B)
    wi4 = npu.pack_i4(B)
    A = np.ones((1, 64), np.int8)
    C = np.empty((1, 64), np.int32)
    assert L.ork_i4_mm_run(npu.h, wi8, 1, ork.ptr(A), ork.ptr(C)) == -1   # dtype mismatch
    assert L.ork_i8_mm_run(npu.h, wi4, 1, ork.ptr(A), ork.ptr(C)) == -1
    buf = (Ct.c_int8 * 512)()
    base = Ct.addressof(buf)
    assert L.ork_i8_mm_run(npu.h, wi8, 1, base, base + 16) == -1          # A/C overlap (test_matmul.c:559-589)
    assert L.ork_i8_mm_run(npu.h, wi8, 0, ork.ptr(A), ork.ptr(C)) == -1
    ork.free(wi8)
    ork.free(wi4)
    assert L.ork_io_failures() == 0


@pytest.mark.parametrize("kind,tile", [("i8", "64x192"), ("i8", "128x128"), ("i8", "128x96"), ("f16", "64x192"),
                                       ("f16", "128x128"), ("f16", "128x96"), ("i4a8", "128x128"), ("w4a4", "128x128")])
def test_lds_ring_two_slots(npu, kind, tile):
    """The LDS-ring kernel's two-slot ring (two workgroups per CU), forced (ORK_RING=2) on every tile it is built
    for: rows and columns with tails, K tails (one stage, a few, many), a K split, and a grid of several rounds of
    the CUs (M=1100, N=1536). Exact for the integer kinds, within the fp16 bar for fp16."""
    _say("lds ring two slots", kind, tile)
    rng = np.random.default_rng(151 + len(kind) + int(tile.split("x")[1]))
    for (M, K, N, ks) in [(70, 1056, 224, 1), (300, 160, 224, 1), (130, 2080, 320, 2), (1100, 1056, 1536, 1)]:
        if kind == "w4a4":
            N = (N + 63) // 64 * 64
            B = rng.integers(-8, 8, size=(K, N), dtype=np.int8)
            A = rng.integers(-8, 8, size=(M, K), dtype=np.int8)
            w, run, ref = npu.pack_i4(B), npu.run_i4, O.gemm_i32(A, B)
        elif kind == "f16":
            B = (rng.standard_normal((K, N)) * 0.02).astype(np.float16)
            A = rng.standard_normal((M, K)).astype(np.float16)
            w, run, ref = npu.pack_f16(B), npu.run_f16, O.gemm_f16_f64acc(A, B)
        elif kind == "i8":
            B = rng.integers(-128, 128, size=(K, N), dtype=np.int8)
            A = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
            w, run, ref = npu.pack_i8(B), npu.run_i8, O.gemm_i32(A, B)
        else:
            W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
            w, _ = npu.pack_i4a8(W)
            A = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
            run, ref = npu.run_i8, O.gemm_i32(A, O.pack_i4a8(W)[2])
        with _env(ORK_TILE=tile, ORK_RING=2, ORK_KSPLIT=ks):
            rc, C = run(w, A)
            name = npu.plan_name(w, M)
        assert rc == 0 and name.endswith("_r2") and tile in name, name
        if kind == "f16":
            assert O.fp16_err(C, ref) <= FP16_TOL, (name, M, K, N)
        else:
            assert np.array_equal(C, ref), (name, M, K, N)
        ork.free(w)


@pytest.mark.parametrize("tile", ["256x256", "128x128", "128x96", "64x192", "64x64", "32x64", "32x32", "16x64", "16x32"])
def test_nf4_ring_short_k(npu, tile):
    """NF4 on every LDS-ring tile with rings of one to three stages (K = 32, 128, 160, 288: one K-block, one, two and
    three, the last ones ending mid-block): the stage decode runs a stage ahead where the tile has room for two decode
    buffers, so the first and last stages are its edges. Exact against the oracle, M = 70 and 5 (row tails)."""
    _say("nf4 short-K ring", tile)
    rng = np.random.default_rng(141 + int(tile.split("x")[0]) + int(tile.split("x")[1]))
    N = 224
    for K in (32, 128, 160, 288):
        W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
        with _env(ORK_NF4=1):
            w, _ = npu.pack_i4a8(W)
        _, _, codes = O.pack_i4a8(W, nf4=True)
        for M in (70, 5):
            A = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
            with _env(ORK_TILE=tile):
                rc, C = npu.run_i8(w, A)
                name = npu.plan_name(w, M)
            assert name.startswith("tiled2_nf4_" + tile), name
            assert rc == 0 and np.array_equal(C, O.gemm_i32(A, codes)), (name, K, M)
        ork.free(w)


@pytest.mark.parametrize("tile", ["256x256", "128x128", "128x96", "64x192", "64x64", "32x64", "32x32", "16x64", "16x32"])
@pytest.mark.parametrize("ks", [1, 3])
@pytest.mark.parametrize("aline", [0, 1])
def test_lds_ring_tiles_all_kinds(npu, tile, ks, aline):
    """The LDS-ring tiled kernel at every tile shape the planner can choose (32- and 16-row tiles, and 128x96 whose six
    block columns take two waves, split each stage's K-blocks over groups of waves and sum their partial tiles in
    LDS), unsplit and K-split, with A stages
    in fragment order and as whole row lines (ORK_ALINE; 256x256 has 64-byte stage rows and always uses
    fragment order): exact for int8, uniform-int4 and NF4 i4a8 and W4A4, within the fp16 bar (and run-to-run
    identical) for fp16. M, N and K tails: M = 300 and 70 are no tile multiple, N = 224 (14 panels) leaves a
    partial tile for every tile width, K = 2080 ends mid K-block for int8 (K % 64 = 32) and the nibble kinds
    (K % 128 = 32)."""
    _say("lds-ring tile", tile, "ks", ks, "aline", aline)
    os.environ["ORK_ALINE"] = str(aline)
    try:
        _lds_ring_tiles_all_kinds(npu, tile, ks)
    finally:
        os.environ.pop("ORK_ALINE", None)


def _lds_ring_tiles_all_kinds(npu, tile, ks):
    bm, bn = map(int, tile.split("x"))
    rng = np.random.default_rng(bm * 1000 + bn * 10 + ks)  # fixed per case (str hash() is salted per process)
    K, N = 2080, 224
    for M in (300, 70):
        B = rng.integers(-128, 128, size=(K, N), dtype=np.int8)
        A = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
        w = npu.pack_i8(B)
        assert w
        with _env(ORK_TILE=tile, ORK_KSPLIT=ks):
            rc, C = npu.run_i8(w, A)
            name = npu.plan_name(w, M)
        assert name.startswith("tiled2_i8_" + tile), name
        assert rc == 0 and np.array_equal(C, O.gemm_i32(A, B)), ("i8", name)
        ork.free(w)
        W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
        w, _ = npu.pack_i4a8(W)
        _, _, codes = O.pack_i4a8(W)
        with _env(ORK_TILE=tile, ORK_KSPLIT=ks):
            rc, C = npu.run_i8(w, A)
        assert rc == 0 and np.array_equal(C, O.gemm_i32(A, codes)), ("i4a8 uniform", M)
        ork.free(w)
        with _env(ORK_NF4=1):  # NF4: the stage's blocks decoded once into LDS
            w, _ = npu.pack_i4a8(W)
        _, _, codes = O.pack_i4a8(W, nf4=True)
        with _env(ORK_TILE=tile, ORK_KSPLIT=ks):
            rc, C = npu.run_i8(w, A)
            name = npu.plan_name(w, M)
        assert name.startswith("tiled2_nf4_" + tile), name
        assert rc == 0 and np.array_equal(C, O.gemm_i32(A, codes)), ("i4a8 nf4", M)
        ork.free(w)
    A4, B4 = O.gen_i4_test(150, 1056, 256)   # W4A4 needs N % 64
    w = npu.pack_i4(B4)
    with _env(ORK_TILE=tile, ORK_KSPLIT=ks):
        rc, C = npu.run_i4(w, A4)
    assert rc == 0 and np.array_equal(C, O.gemm_i32(A4, B4)), "w4a4"
    ork.free(w)
    Ah = rng.standard_normal((130, 1056)).astype(np.float16)
    Bh = (rng.standard_normal((1056, 224)) * 0.02).astype(np.float16)
    w = npu.pack_f16(Bh)
    with _env(ORK_TILE=tile, ORK_KSPLIT=ks):
        rc, C1 = npu.run_f16(w, Ah)
        rc2, C2 = npu.run_f16(w, Ah)
    assert rc == 0 and rc2 == 0 and np.array_equal(C1, C2)
    assert O.fp16_err(C1, O.gemm_f16_f64acc(Ah, Bh)) <= FP16_TOL
    ork.free(w)


@pytest.mark.parametrize("tile", ["128x96", "64x192", "64x64", "32x64", "32x32", "16x64", "16x32"])
@pytest.mark.parametrize("M", [1, 5, 17, 48, 64])
def test_lds_ring_small_m(npu, tile, M):
    """The LDS-ring kernel below one tile height (the planner takes it from M = 24 on wide or long-K
    shapes): rows past M are zero-filled loads and unwritten C rows. int8 exact, unsplit and split; fp16
    within the bar."""
    _say("lds-ring small M", tile, M)
    rng = np.random.default_rng(M * 7 + len(tile))
    K, N = 2080, 224
    A = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
    B = rng.integers(-128, 128, size=(K, N), dtype=np.int8)
    w = npu.pack_i8(B)
    for ks in (1, 2):
        with _env(ORK_TILE=tile, ORK_KSPLIT=ks):
            rc, C = npu.run_i8(w, A)
            name = npu.plan_name(w, M)
        assert name.startswith("tiled2_i8_" + tile), name
        assert rc == 0 and np.array_equal(C, O.gemm_i32(A, B)), name
    ork.free(w)
    Ah = rng.standard_normal((M, 1056)).astype(np.float16)
    Bh = (rng.standard_normal((1056, 224)) * 0.02).astype(np.float16)
    w = npu.pack_f16(Bh)
    with _env(ORK_TILE=tile):
        rc, C = npu.run_f16(w, Ah)
    assert rc == 0 and O.fp16_err(C, O.gemm_f16_f64acc(Ah, Bh)) <= FP16_TOL
    ork.free(w)


@pytest.mark.parametrize("np_", [1, 2])
@pytest.mark.parametrize("kind", ["i8", "i4a8", "nf4", "f16", "w4a4"])
def test_stream_paired_panels(npu, kind, np_):
    """The streaming kernel with paired panels (one round of as many workgroups as CUs, the first N/16 - CUs
    owning two adjacent panels and sharing each A chunk between them) and without (ORK_STREAM_NP): exact for
    the integer kinds, within the fp16 bar for fp16. N is derived from the device's CU count so that
    cu < N/16 < 2*cu (the range where pairing applies; 260 and 400 panels on 256 CUs, both pairings uneven), M
    from 2 to 32 (one and two row tiles), K tails."""
    _say("stream paired", kind, np_)
    rng = np.random.default_rng(91 + np_)
    cu = ork.lib().ork_npu_cores(npu.h)
    n1 = (16 * cu // 64 + 1) * 64        # just above cu panels (a multiple of 64 for W4A4)
    n2 = (25 * cu // 64) * 64            # ~1.56 cu panels
    assert cu < n1 // 16 < 2 * cu and cu < n2 // 16 < 2 * cu
    for (K, N, M) in [(1056, n1, 2), (2080, n1, 17), (512, n2, 32), (2048, n2, 9)]:
        if kind == "w4a4":
            B = rng.integers(-8, 8, size=(K, N), dtype=np.int8)
            A = rng.integers(-8, 8, size=(M, K), dtype=np.int8)
            w = npu.pack_i4(B)
            ref = O.gemm_i32(A, B)
            run = npu.run_i4
        elif kind == "f16":
            B = (rng.standard_normal((K, N)) * 0.02).astype(np.float16)
            A = rng.standard_normal((M, K)).astype(np.float16)
            w = npu.pack_f16(B)
            ref = O.gemm_f16_f64acc(A, B)
            run = npu.run_f16
        elif kind == "i8":
            B = rng.integers(-128, 128, size=(K, N), dtype=np.int8)
            A = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
            w = npu.pack_i8(B)
            ref = O.gemm_i32(A, B)
            run = npu.run_i8
        else:
            W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
            with _env(**({"ORK_NF4": 1} if kind == "nf4" else {})):
                w, _ = npu.pack_i4a8(W)
            _, _, codes = O.pack_i4a8(W, nf4=kind == "nf4")
            A = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
            ref = O.gemm_i32(A, codes)
            run = npu.run_i8
        with _env(ORK_PLAN="stream", ORK_STREAM_NP=np_):
            rc, C = run(w, A)
            name = npu.plan_name(w, M)
        assert rc == 0 and name.startswith("stream_") and name.endswith("_p2") == (np_ == 2), name
        if kind == "f16":
            assert O.fp16_err(C, ref) <= FP16_TOL, name
        else:
            assert np.array_equal(C, ref), (name, K, N, M)
        ork.free(w)


@pytest.mark.parametrize("ks", [1, 2])
@pytest.mark.parametrize("kind", ["i8", "i4a8", "nf4", "f16", "w4a4"])
def test_stream_half_panels(npu, kind, ks):
    """The streaming kernel with half panels (ORK_STREAM_HALF: each workgroup loads and stores 8 of a panel's 16
    columns, twice the workgroups), every kind the kernel is built for, whole K and split K: exact for the integer
    kinds, within the fp16 bar for fp16, and every column of C written by its own half (N = 128 and 320: 16 and 40
    half panels; M = 1 row tile to 4, with tails; K tails)."""
    _say("stream half", kind, ks)
    rng = np.random.default_rng(131 + ks)
    for (K, N, M) in [(1056, 128, 2), (2080, 320, 17), (512, 320, 64), (4096, 128, 37)]:
        if kind == "w4a4":
            B = rng.integers(-8, 8, size=(K, N), dtype=np.int8)
            A = rng.integers(-8, 8, size=(M, K), dtype=np.int8)
            w = npu.pack_i4(B)
            ref = O.gemm_i32(A, B)
            run = npu.run_i4
        elif kind == "f16":
            B = (rng.standard_normal((K, N)) * 0.02).astype(np.float16)
            A = rng.standard_normal((M, K)).astype(np.float16)
            w = npu.pack_f16(B)
            ref = O.gemm_f16_f64acc(A, B)
            run = npu.run_f16
        elif kind == "i8":
            B = rng.integers(-128, 128, size=(K, N), dtype=np.int8)
            A = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
            w = npu.pack_i8(B)
            ref = O.gemm_i32(A, B)
            run = npu.run_i8
        else:
            W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
            with _env(**({"ORK_NF4": 1} if kind == "nf4" else {})):
                w, _ = npu.pack_i4a8(W)
            _, _, codes = O.pack_i4a8(W, nf4=kind == "nf4")
            A = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
            ref = O.gemm_i32(A, codes)
            run = npu.run_i8
        with _env(ORK_PLAN="stream", ORK_STREAM_HALF=1, ORK_KSPLIT=ks):
            rc, C = run(w, A)
            name = npu.plan_name(w, M)
        assert rc == 0 and name.startswith("stream_") and name.endswith("_h") and f"_ks{ks}_" in name, name
        if kind == "f16":
            assert O.fp16_err(C, ref) <= FP16_TOL, name
        else:
            assert np.array_equal(C, ref), (name, K, N, M)
        ork.free(w)


@pytest.mark.parametrize("kind,K,N,M", [("i8", 2048, 6144, 48), ("i8", 6144, 2048, 64), ("i4a8", 2048, 6144, 64),
                                        ("f16", 2048, 6144, 32), ("i8", 2048, 22016, 24)])
def test_planner_mid_m_default(npu, kind, K, N, M):
    """Default plans at 17 <= M <= 64 where the time model prefers the LDS-ring kernel (possibly K-split):
    results as exact as every other route."""
    _say("planner mid-M", kind, K, N, M)
    rng = np.random.default_rng(K + N + M)
    if kind == "f16":
        Ah = rng.standard_normal((M, K)).astype(np.float16)
        Bh = (rng.standard_normal((K, N)) * 0.02).astype(np.float16)
        w = npu.pack_f16(Bh)
        rc, C = npu.run_f16(w, Ah)
        assert npu.plan_name(w, M).startswith("tiled2_"), npu.plan_name(w, M)
        assert rc == 0 and O.fp16_err(C, O.gemm_f16_f64acc(Ah, Bh)) <= FP16_TOL
        ork.free(w)
        return
    A = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
    if kind == "i8":
        B = rng.integers(-128, 128, size=(K, N), dtype=np.int8)
        w = npu.pack_i8(B)
    else:
        W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
        w, _ = npu.pack_i4a8(W)
        _, _, B = O.pack_i4a8(W)
    rc, C = npu.run_i8(w, A)
    assert npu.plan_name(w, M).startswith("tiled2_"), npu.plan_name(w, M)
    assert rc == 0 and np.array_equal(C, O.gemm_i32(A, B)), npu.plan_name(w, M)
    ork.free(w)


# ------------------------------------------------------------------------ M = 1: half panels and whole panels
GEMV_HALF_SHAPES = [  # (K, N): K tails (K % 64 == 32; K % 128 == 32 for the nibble kinds), odd runs per wave, one panel
    (32, 64), (96, 64), (2080, 64), (1056, 4160), (2048, 6144), (6144, 2048)]


def _gemv_weight(npu, kind, K, N, rng):
    """A packed weight of one kind and the B operand its oracle product takes (the codes for the W4A8 kinds)."""
    if kind == "f16":
        Bh = (rng.standard_normal((K, N)) * 0.02).astype(np.float16)
        return npu.pack_f16(Bh), Bh
    if kind == "w4a4":
        B = rng.integers(-8, 8, size=(K, N), dtype=np.int8)
        return npu.pack_i4(B), B
    if kind == "i8":
        B = rng.integers(-128, 128, size=(K, N), dtype=np.int8)
        return npu.pack_i8(B), B
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    if kind == "nf4":
        os.environ["ORK_NF4"] = "1"
    try:
        w, _ = npu.pack_i4a8(W)
    finally:
        os.environ.pop("ORK_NF4", None)
    _, _, codes = O.pack_i4a8(W, nf4=kind == "nf4")
    return w, codes


def _gemv_run(npu, kind, w, B, A):
    if kind == "f16":
        rc, C = npu.run_f16(w, A)
        return rc == 0 and O.fp16_err(C, O.gemm_f16_f64acc(A, B)) <= FP16_TOL
    rc, C = (npu.run_i4 if kind == "w4a4" else npu.run_i8)(w, A)
    return rc == 0 and np.array_equal(C, O.gemm_i32(A, B))


@pytest.mark.parametrize("kind", ["i8", "f16", "i4a8", "nf4", "w4a4"])
def test_gemv_half_panels(npu, kind):
    """M = 1 runs on half panels by default (8 columns per workgroup): exact against the oracle for the integer
    kinds and within tolerance for fp16, like whole panels (ORK_GEMV_HALF=0), at every wave count (ORK_WPG) and
    with forced K splits, over K tails and runs with an odd number of blocks."""
    _say("gemv half", kind)
    rng = _rng(77)
    for K, N in GEMV_HALF_SHAPES:
        w, B = _gemv_weight(npu, kind, K, N, rng)
        assert w, (kind, K, N)
        if kind == "f16":
            A = rng.standard_normal((1, K)).astype(np.float16)
        elif kind == "w4a4":
            A = rng.integers(-8, 8, size=(1, K), dtype=np.int8)
        else:
            A = rng.integers(-127, 128, size=(1, K), dtype=np.int8)
        assert _gemv_run(npu, kind, w, B, A), (kind, K, N, npu.plan_name(w, 1))
        for env in (dict(ORK_GEMV_HALF=0), dict(ORK_GEMV_HALF=1), dict(ORK_GEMV_HALF=1, ORK_WPG=2),
                    dict(ORK_GEMV_HALF=1, ORK_WPG=4), dict(ORK_GEMV_HALF=1, ORK_WPG=8), dict(ORK_GEMV_HALF=1, ORK_KSPLIT=3),
                    dict(ORK_GEMV_HALF=1, ORK_KSPLIT=2, ORK_WPG=8), dict(ORK_GEMV_HALF=0, ORK_KSPLIT=2)):
            with _env(**env):
                name = npu.plan_name(w, 1)
                assert name.startswith("gemvh_" if env["ORK_GEMV_HALF"] else "gemv_"), (env, name)
                assert _gemv_run(npu, kind, w, B, A), (kind, K, N, env, name)
        ork.free(w)


def test_gemv_half_panel_rule(npu):
    """The planner keeps whole panels where they already spread evenly (N/16 a multiple of the CU count) and takes
    half panels otherwise: fewer panels than CUs, or a remainder that would put two panels on some CUs only."""
    cu = ork.lib().ork_npu_cores(npu.h)
    rng = _rng(79)
    for N, half in ((16 * cu, False), (32 * cu, False), (24 * cu, True), (8 * cu, True), (16 * cu + 32, True)):
        B = rng.integers(-128, 128, size=(256, N), dtype=np.int8)
        w = npu.pack_i8(B)
        assert npu.plan_name(w, 1).startswith("gemvh_" if half else "gemv_"), (N, cu, npu.plan_name(w, 1))
        A = rng.integers(-127, 128, size=(1, 256), dtype=np.int8)
        rc, C = npu.run_i8(w, A)
        assert rc == 0 and np.array_equal(C, O.gemm_i32(A, B)), N
        ork.free(w)


def test_gemv_half_unaligned_activations(npu):
    """A device activation row that is not 16-byte aligned runs on whole panels (the half-panel kernel loads
    16 bytes at a time): same exact result."""
    _say("gemv half unaligned A")
    L = ork.lib()
    rng = _rng(78)
    K, N = 2080, 1056
    B = rng.integers(-128, 128, size=(K, N), dtype=np.int8)
    A = rng.integers(-127, 128, size=(1, K), dtype=np.int8)
    w = npu.pack_i8(B)
    dA = L.ork_dev_alloc(npu.h, K + 64)
    dC = L.ork_dev_alloc(npu.h, N * 4)
    assert w and dA and dC
    for off in (0, 4, 8, 20):
        assert L.ork_dev_upload(npu.h, dA + off, ork.ptr(A), K) == 0
        assert L.ork_i8_mm_run(npu.h, w, 1, dA + off, dC) == 0
        C = np.zeros((1, N), np.int32)
        assert L.ork_dev_download(npu.h, ork.ptr(C), dC, N * 4) == 0
        assert np.array_equal(C, O.gemm_i32(A, B)), off
    L.ork_dev_free(npu.h, dA)
    L.ork_dev_free(npu.h, dC)
    ork.free(w)
