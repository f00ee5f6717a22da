"""Persisted weights on the GPU: dump -> load round trips that run, and the load gate.

- pack + ork_w_dump is byte-identical to the CPU dumper (the reference's examples/test_i4_dump_cpu.c
  property, for int8 and W4A4);
- a loaded weight runs bit-exact against the oracle (int8, W4A4) or identically to the packed one
  (fp16: same panels, same kernel), and re-dumps byte-identically;
- an i4a8 weight dumps as the int8 codes it multiplies with (dtype I8, as the reference's inflated int8
  tiles), and the loaded int8 weight runs exactly as the i4a8 weight did;
- examples/test_pack_gate.c on the device loaders (int8 and fp16).
"""
import os
import struct

import numpy as np
import pytest

import oracle as O
import ork
from test_persist_host import HDR, _gate_cases, _load

pytestmark = pytest.mark.gpu


def _say(*a):
    print("[case]", *a, flush=True)


@pytest.mark.parametrize("K,N,M", [(2048, 6144, 1), (1536, 256, 16), (96, 64, 130)])
def test_i8_dump_load_run(npu, K, N, M):
    _say("i8", K, N, M)
    L = ork.lib()
    rng = np.random.default_rng(K + N + M)
    B = rng.integers(-128, 128, size=(K, N), dtype=np.int8)
    w = npu.pack_i8(B)
    blob = ork.dump(w)
    assert np.array_equal(blob, ork.dump_cpu(npu.h, B))
    ork.lib().ork_mm_free(npu.h, w)
    w2 = _load(L, L.ork_i8_mm_load, npu.h, K, N, blob)
    assert w2
    A = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
    rc, Cg = npu.run_i8(w2, A)
    assert rc == 0 and np.array_equal(Cg, O.gemm_i32(A, B))
    assert np.array_equal(ork.dump(w2), blob)
    L.ork_mm_free(npu.h, w2)


def test_i8_pack_f32_dump_load(npu):
    _say("i8 pack_f32")
    L = ork.lib()
    rng = np.random.default_rng(5)
    W = (rng.standard_normal((512, 1024)) * 0.02).astype(np.float32)
    w, bs = npu.pack_i8_f32(W)
    codes, bs_ref = O.pack_i8_f32(W)
    blob = ork.dump(w)
    assert np.array_equal(blob, ork.dump_cpu(npu.h, codes))
    w2 = _load(L, L.ork_i8_mm_load, npu.h, 1024, 512, blob)
    A = rng.integers(-127, 128, size=(3, 1024), dtype=np.int8)
    assert np.array_equal(npu.run_i8(w2, A)[1], O.gemm_i32(A, codes))
    L.ork_mm_free(npu.h, w)
    L.ork_mm_free(npu.h, w2)


@pytest.mark.parametrize("K,N,M", [(4096, 4096, 256), (1024, 128, 1), (96, 64, 7)])
def test_i4_dump_load_run(npu, K, N, M):
    _say("w4a4", K, N, M)
    L = ork.lib()
    A, B = O.gen_i4_test(M, K, N)
    w = npu.pack_i4(B)
    blob = ork.dump(w)
    assert np.array_equal(blob, ork.dump_cpu(npu.h, B, w4a4=True))
    w2 = _load(L, L.ork_i4_mm_load, npu.h, K, N, blob)
    assert w2
    rc, Cg = npu.run_i4(w2, A)
    assert rc == 0 and np.array_equal(Cg, O.gemm_i32(A, B))
    assert np.array_equal(ork.dump(w2), blob)
    L.ork_mm_free(npu.h, w)
    L.ork_mm_free(npu.h, w2)


def test_f16_dump_load_run(npu):
    _say("fp16")
    L = ork.lib()
    rng = np.random.default_rng(9)
    K, N = 2048, 2048
    B = (rng.standard_normal((K, N)) * 0.02).astype(np.float16)
    A = rng.standard_normal((16, K)).astype(np.float16)
    w = npu.pack_f16(B)
    blob = ork.dump(w)
    assert struct.unpack_from("<I", blob, 12)[0] == 0  # dtype F16
    w2 = _load(L, L.ork_f16_mm_load, npu.h, K, N, blob)
    assert w2
    _, C1 = npu.run_f16(w, A)
    _, C2 = npu.run_f16(w2, A)
    assert np.array_equal(C1, C2)
    assert O.fp16_err(C2, O.gemm_f16_f64acc(A, B)) <= 2e-3
    assert np.array_equal(ork.dump(w2), blob)
    L.ork_mm_free(npu.h, w)
    L.ork_mm_free(npu.h, w2)


@pytest.mark.parametrize("nf4", [0, 1])
def test_i4a8_dumps_as_int8(npu, nf4):
    _say("i4a8 -> i8", nf4)
    L = ork.lib()
    rng = np.random.default_rng(11 + nf4)
    K, N = 1024, 256
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    if nf4:
        os.environ["ORK_NF4"] = "1"
    try:
        w, _ = npu.pack_i4a8(W)
    finally:
        os.environ.pop("ORK_NF4", None)
    _, _, codes = O.pack_i4a8(W, nf4=bool(nf4))
    blob = ork.dump(w)
    assert struct.unpack_from("<I", blob, 12)[0] == 1  # dtype I8
    assert np.array_equal(blob, ork.dump_cpu(npu.h, codes))
    w2 = _load(L, L.ork_i8_mm_load, npu.h, K, N, blob)
    A = rng.integers(-127, 128, size=(5, K), dtype=np.int8)
    _, C1 = npu.run_i8(w, A)
    _, C2 = npu.run_i8(w2, A)
    assert np.array_equal(C1, C2) and np.array_equal(C2, O.gemm_i32(A, codes))
    L.ork_mm_free(npu.h, w)
    L.ork_mm_free(npu.h, w2)


@pytest.mark.parametrize("kind", ["i8", "f16"])
def test_pack_gate_on_device(npu, kind):
    """examples/test_pack_gate.c, int8 and fp16 loaders."""
    _say("gate", kind)
    L = ork.lib()
    K, N = 512, 256
    if kind == "i8":
        B = (np.array([(i * 37) & 0x7F for i in range(K * N)], np.int32).reshape(K, N) - 64).astype(np.int8)
        w = npu.pack_i8(B)
        fn = L.ork_i8_mm_load
    else:
        B = (((np.arange(K * N) % 17) - 8) * 0.01).astype(np.float16).reshape(K, N)
        w = npu.pack_f16(B)
        fn = L.ork_f16_mm_load
    good = ork.dump(w)
    L.ork_mm_free(npu.h, w)
    ok = _load(L, fn, npu.h, K, N, good)
    assert ok, "the honest pack must load"
    L.ork_mm_free(npu.h, ok)
    for what, blob, k, n in _gate_cases(good, K, N):
        assert not _load(L, fn, npu.h, k, n, blob), what
