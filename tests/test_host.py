"""Host-side tests of the product library (CPU only, no compute calls on a GPU).

- libork_npu.so loads and exports every function include/*.h declares
- offline-context surfaces: ork_i4a8_pack_cpu_blob(_qerr) byte-identical to the oracle, offline
  pack / load keep the oracle's codes, and runs on an offline context compute the exact result on the CPU
  as the reference's offline branches do (int8 / int4 / grouped runs, int8 chain, int4 chain and stream)
- dims gates, O4N1 validation cases, ork_i8_mm_run_cpu vs the oracle
- bench.py refuses more than one GPU
"""
import ctypes as C
import os
import re

import numpy as np
import pytest

import oracle as O
import ork

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_functions():
    names = set()
    for dirpath, _, files in os.walk(os.path.join(ROOT, "include")):
        for f in files:
            if f.endswith(".h"):
                text = open(os.path.join(dirpath, f)).read()
                text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
                names |= set(re.findall(r"\b(ork_[a-z0-9_]+)\s*\(", text))
    return names


def test_exports_every_declared_symbol():
    declared = _declared_functions()
    assert len(declared) >= 40
    L = ork.lib()
    missing = [n for n in sorted(declared) if not hasattr(L, n)]
    assert not missing, missing
    assert set(ork.API) == declared  # the binding covers exactly the declared API


def test_version_strings():
    L = ork.lib()
    assert L.ork_npu_version().decode() == "1.0.190+mi355x"
    assert L.ork_pack_format_version() == 1


@pytest.fixture
def off():
    c = ork.Npu(offline="gfx950")
    yield c
    c.close()


def test_offline_unknown_soc():
    assert not ork.lib().ork_npu_init_offline(b"nope")


@pytest.mark.parametrize("nf4", [0, 1])
@pytest.mark.parametrize("imatrix", [0, 1])
@pytest.mark.parametrize("K,N", [(1024, 256), (1536, 128), (96, 64)])
def test_cpu_blob_matches_oracle(off, nf4, imatrix, K, N):
    rng = np.random.default_rng(K + N + nf4 + 10 * imatrix)
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    W[0, :5] = [0.0, 1e-12, -1e-12, 0.5, -0.5]
    im = rng.uniform(0.5, 2.0, K).astype(np.float32) if imatrix else None
    blob, q = ork.cpu_blob(K, N, W, im, nf4=nf4, ctx=off.h, qerr=True)
    ref, qref = O.i4a8_blob(W, im, nf4=nf4, want_qerr=True)
    assert np.array_equal(blob, ref)
    assert q == qref and 0.0 < q < 1.0


def test_cpu_blob_stochastic_rounding(off):
    rng = np.random.default_rng(3)
    K, N = 512, 64
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    os.environ["ORK_SR"] = "1"
    try:
        for nf4 in (0, 1):
            blob = ork.cpu_blob(K, N, W, None, nf4=nf4, ctx=off.h)
            assert np.array_equal(blob, O.i4a8_blob(W, None, nf4=nf4, sr=True))
            assert not np.array_equal(blob, O.i4a8_blob(W, None, nf4=nf4, sr=False))
    finally:
        del os.environ["ORK_SR"]


def test_cpu_blob_dims_and_cap(off):
    W = np.zeros((64, 100), np.float32)
    assert ork.lib().ork_i4a8_pack_cpu_blob(off.h, 100, 64, ork.ptr(W), None, 0, None, 0) == 0
    W = np.ones((64, 64), np.float32)
    need = ork.lib().ork_i4a8_pack_cpu_blob(off.h, 64, 64, ork.ptr(W), None, 0, None, 0)
    assert need == 20 + 64 * 4 + 64 * 64 // 2  # examples/test_matmul.c:528
    small = np.zeros(need - 1, np.uint8)
    assert ork.lib().ork_i4a8_pack_cpu_blob(off.h, 64, 64, ork.ptr(W), None, 0, ork.ptr(small), need - 1) == 0


@pytest.mark.parametrize("nf4", [0, 1])
def test_offline_pack_i4a8_codes_and_dump(off, nf4):
    rng = np.random.default_rng(21 + nf4)
    K, N = 512, 96
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    im = rng.uniform(0.5, 2.0, K).astype(np.float32)
    if nf4:
        os.environ["ORK_NF4"] = "1"
    try:
        w, bs = off.pack_i4a8(W, im)
    finally:
        os.environ.pop("ORK_NF4", None)
    bs_ref, nib_ref, codes_ref = O.pack_i4a8(W, im, nf4=nf4)
    assert w and np.array_equal(bs, bs_ref)
    assert np.array_equal(ork.bscale(w, N), bs_ref)
    assert np.array_equal(ork.codes(w, K, N), codes_ref)
    assert ork.lib().ork_w_quant_kind(w) == nf4
    blob = ork.dump_i4a8(w)
    assert np.array_equal(blob, O.i4a8_blob(W, im, nf4=nf4))
    # offline load of that blob recovers exactly the same codes (examples/test_offline_load.c:44-77)
    w2 = off.load_i4a8(K, N, blob)
    assert np.array_equal(ork.codes(w2, K, N), codes_ref)
    assert np.array_equal(ork.dump_i4a8(w2), blob)
    # and a run on an offline context is the exact CPU MAC on those codes (src/npu/i8/run.c:140)
    A = np.random.default_rng(5).integers(-127, 128, size=(3, K), dtype=np.int8)
    rc, Cg = off.run_i8(w, A)
    assert rc == 0 and np.array_equal(Cg, O.gemm_i32(A, codes_ref))
    ork.free(w)
    ork.free(w2)


def test_offline_i4a8_identity_roundtrip(off):
    """examples/test_offline_load.c:44-77: codes in [-7,7] with one +7 per channel pack to themselves."""
    rng = np.random.default_rng(4)
    K, N = 1536, 256
    codes = rng.integers(-7, 8, size=(K, N), dtype=np.int8)
    codes[0, :] = 7
    W = codes.T.astype(np.float32).copy()
    blob = ork.cpu_blob(K, N, W, None, nf4=0, ctx=off.h)
    w = off.load_i4a8(K, N, blob)
    assert np.array_equal(ork.codes(w, K, N), codes)
    assert np.all(ork.bscale(w, N) == np.float32(1.0))
    ork.free(w)


def test_o4n1_rejections(off):
    rng = np.random.default_rng(5)
    K, N = 64, 32
    W = rng.standard_normal((N, K)).astype(np.float32)
    blob = ork.cpu_blob(K, N, W, None, ctx=off.h)
    assert off.load_i4a8(K, N, blob)
    bad = []
    b = blob.copy(); b[0] ^= 1; bad.append(("magic", K, N, b))
    b = blob.copy(); b[4] = 2; bad.append(("version", K, N, b))
    b = blob.copy(); b[16] = 2; bad.append(("kind", K, N, b))
    bad.append(("K", 96, N, blob))
    bad.append(("N", K, 64, blob))
    bad.append(("short", K, N, blob[:-1]))
    bad.append(("long", K, N, np.concatenate([blob, np.zeros(1, np.uint8)])))
    for name, k, n, b in bad:
        assert not off.load_i4a8(k, n, b), name
    assert O.o4n1_decode(K, N, blob) is not None


def test_offline_pack_i8_f32_codes(off):
    rng = np.random.default_rng(6)
    K, N = 2048, 512
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    w, bs = off.pack_i8_f32(W)
    codes, bs_ref = O.pack_i8_f32(W)
    assert np.array_equal(bs, bs_ref)
    assert np.array_equal(ork.codes(w, K, N), codes)
    ork.free(w)


def test_dims_gates(off):
    L = ork.lib()
    B = np.zeros(64 * 128, np.int8)
    F = np.zeros(64 * 128, np.float32)
    H = np.zeros(64 * 128, np.float16)
    assert not L.ork_i8_mm_pack(off.h, 48, 64, ork.ptr(B))       # K%32
    assert not L.ork_i8_mm_pack(off.h, 64, 48, ork.ptr(B))       # N%32
    assert not L.ork_i8_mm_pack_f32(off.h, 64, 16, ork.ptr(F), None)
    assert not L.ork_i4a8_mm_pack(off.h, 64, 16, ork.ptr(F), None)
    assert not L.ork_i4_mm_pack(off.h, 64, 32, ork.ptr(B))       # N%64
    assert not L.ork_f16_mm_pack(off.h, 64, 8, ork.ptr(H))       # N%16
    w = L.ork_i4_mm_pack(off.h, 64, 64, ork.ptr(B))
    assert w
    L.ork_w_free(w)


def test_offline_runs_compute_exactly(off):
    """The reference's offline branches (src/npu/i8/run.c:140, src/npu/i4/run.c:236, grouped :48-49 and
    src/npu/i4/run.c:368-369): an offline weight's runs are the exact CPU result, here checked against the
    oracle. The product computes them with its own cpu_gemm.c, never the oracle."""
    L = ork.lib()
    rng = np.random.default_rng(12)
    K, N, M = 256, 96, 5
    B = rng.integers(-128, 128, size=(K, N), dtype=np.int8)
    A = rng.integers(-128, 128, size=(M, K), dtype=np.int8)
    w = off.pack_i8(B)
    rc, Cm = off.run_i8(w, A)
    assert rc == 0 and np.array_equal(Cm, O.gemm_i32(A, B))
    # W4A4 (int4 values in int8 containers), N % 64
    B4 = rng.integers(-8, 8, size=(K, 128), dtype=np.int8)
    A4 = rng.integers(-8, 8, size=(M, K), dtype=np.int8)
    w4 = off.pack_i4(B4)
    rc, C4 = off.run_i4(w4, A4)
    assert rc == 0 and np.array_equal(C4, O.gemm_i32(A4, B4))
    # grouped: per-group exact partials scaled and summed in group order, bit for bit
    G = 64
    aS = rng.uniform(1e-3, 2e-2, size=(M, K // G)).astype(np.float32)
    bS = rng.uniform(1e-3, 2e-2, size=(K // G, 128)).astype(np.float32)
    assert L.ork_w_set_group(w4, G) == 0
    Cg = np.zeros((M, 128), np.float32)
    assert L.ork_i4_mm_run_grouped(off.h, w4, M, ork.ptr(A4), ork.ptr(aS), ork.ptr(bS), ork.ptr(Cg)) == 0
    assert np.array_equal(Cg, O.gemm_grouped(A4, B4, aS, bS, G))
    if O.ref_available():
        assert np.array_equal(Cg, O.ref_gemm_grouped(A4, B4, aS, bS, G))
    # an offline context still has no device memory and no fp16 weights
    assert L.ork_dma_alloc(off.h, 64) is None
    assert L.ork_dev_alloc(off.h, 64) is None
    assert not L.ork_f16_mm_pack(off.h, 64, 64, ork.ptr(np.zeros(64 * 64, np.float16)))
    ork.free(w)
    ork.free(w4)


def test_cpu_gemm_api_matches_oracle():
    st = O.LCGState(7777)
    for M, K, N, lo, hi in [(1, 1024, 1024, -8, 7), (32, 1024, 1024, -8, 7), (4, 512, 256, -128, 127), (3, 130, 144, -8, 7)]:
        A = O.gen_cpu_gemm(st, lo, hi, M * K).reshape(M, K)
        B = O.gen_cpu_gemm(st, lo, hi, K * N).reshape(K, N)
        Cm = np.empty((M, N), np.int32)
        ork.lib().ork_i8_mm_run_cpu(M, K, N, ork.ptr(A), ork.ptr(B), ork.ptr(Cm))
        assert np.array_equal(Cm, O.gemm_i32(A, B))


def test_chain_offline(off):
    """ork/chain.h on an offline context, as the reference's CPU chains (src/npu/core/buf.c:483-487, :560-564,
    entered before any argument check): the int8 chain and the int4 chain / stream compute each task exactly
    (C rows at stride N), S <= 0 runs nothing and returns 0; the int8 and fp16 streams have no offline path."""
    L = ork.lib()
    rng = np.random.default_rng(44)
    K = 128
    B1 = rng.integers(-128, 128, size=(K, 64), dtype=np.int8)
    B2 = rng.integers(-8, 8, size=(K, 128), dtype=np.int8)
    w1 = off.pack_i8(B1)
    w2 = off.pack_i4(B2)
    A1 = rng.integers(-128, 128, size=(3, K), dtype=np.int8)
    A2 = rng.integers(-8, 8, size=(2, K), dtype=np.int8)
    C1 = np.zeros((3, 64), np.int32)
    C2 = np.zeros((2, 128), np.int32)
    t = ork.tasks(ork.TaskI8, [(w1, 3, A1, C1), (w2, 2, A2, C2)])
    assert L.ork_i8_mm_run_chain(off.h, 2, t) == 0
    assert np.array_equal(C1, O.gemm_i32(A1, B1)) and np.array_equal(C2, O.gemm_i32(A2, B2))
    C1[:] = 0
    C2[:] = 0
    t4 = ork.tasks(ork.TaskI4, [(w2, 2, A2, C2), (w1, 3, A1, C1)])
    for fn in (L.ork_i4_mm_run_chain, L.ork_i4_mm_run_stream):
        assert fn(off.h, 2, t4) == 0
        assert np.array_equal(C1, O.gemm_i32(A1, B1)) and np.array_equal(C2, O.gemm_i32(A2, B2))
    assert L.ork_i8_mm_run_chain(off.h, 0, t) == 0
    assert L.ork_i8_mm_run_chain(off.h, 1, None) == -2
    # the streams without an offline branch, and contexts that are NULL
    assert L.ork_i8_mm_run_stream(off.h, 1, t) == -1
    assert L.ork_i8_mm_run_chain(None, 1, t) == -1
    assert L.ork_i8_mm_run_stream(None, 1, t) == -2
    assert L.ork_f16_mm_run_stream(off.h, 0, ork.tasks(ork.TaskF16, [(w1, 1, A1, C1)])) == -2
    ork.free(w1)
    ork.free(w2)


def test_accessors_null_safe():
    L = ork.lib()
    K = C.c_int(5)
    N = C.c_int(5)
    L.ork_w_dims(None, C.byref(K), C.byref(N))
    assert (K.value, N.value) == (0, 0)
    assert L.ork_w_quant_kind(None) == -1
    assert L.ork_w_bscale(None) is None
    assert L.ork_i4a8_w_dump(None, None, 0) == 0


def test_reference_offline_load_example_runs_unmodified():
    """examples/test_offline_load.c from the reference, compiled unmodified against include/ and linked to
    libork_npu.so (oracle/ref.mk): offline packs and loads of i4a8 blobs recover the exact codes, and
    pack_cpu_blob(_qerr) is byte-identical to the device-context pack. Needs no GPU."""
    import subprocess

    exe = os.path.join(ROOT, "oracle", "_ref", "test_offline_load_on_mi355x")
    if not os.path.exists(exe):
        pytest.skip("oracle/_ref/test_offline_load_on_mi355x not built (needs the reference tree)")
    r = subprocess.run([exe], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "test_offline_load: PASS" in r.stdout
    assert "FAIL" not in r.stdout


def test_bench_refuses_more_than_one_gpu():
    """bench.py's contract: this build runs on one GPU, so --gpus N > 1 exits with status 2 and says why, before
    touching a device."""
    import subprocess
    import sys

    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_ork_profile_rows_printed_at_free(capfd, monkeypatch):
    """ORK_PROFILE (read when the context is made, src/npu/core/sched.c:53): ork_npu_free prints one
    "[ork PROFILE]" row per entry point and plan with the call count and host time, as the reference prints its
    run_i8 / run_i4 totals (src/npu/core/device.c:257-263). On an offline context the runs are the CPU's."""
    rng = np.random.default_rng(13)
    B = rng.integers(-128, 128, size=(128, 64), dtype=np.int8)
    A = rng.integers(-128, 128, size=(3, 128), dtype=np.int8)
    monkeypatch.setenv("ORK_PROFILE", "1")
    c = ork.Npu(offline="gfx950")
    monkeypatch.delenv("ORK_PROFILE")
    w = c.pack_i8(B)
    for _ in range(3):
        rc, Cm = c.run_i8(w, A)
        assert rc == 0 and np.array_equal(Cm, O.gemm_i32(A, B))
    w4 = c.pack_i4(rng.integers(-8, 8, size=(128, 64), dtype=np.int8))
    assert c.run_i4(w4, rng.integers(-8, 8, size=(2, 128), dtype=np.int8))[0] == 0
    ork.free(w)
    ork.free(w4)
    capfd.readouterr()
    c.close()
    err = capfd.readouterr().err
    rows = [l for l in err.splitlines() if l.startswith("[ork PROFILE]")]
    assert any(l.startswith("[ork PROFILE] ork_i8_mm_run cpu: 3 calls,") for l in rows), err
    assert any(l.startswith("[ork PROFILE] ork_i4_mm_run cpu: 1 calls,") for l in rows), err
    # without the switch nothing is printed
    c2 = ork.Npu(offline="gfx950")
    w2 = c2.pack_i8(B)
    assert c2.run_i8(w2, A)[0] == 0
    ork.free(w2)
    capfd.readouterr()
    c2.close()
    assert "[ork PROFILE]" not in capfd.readouterr().err
