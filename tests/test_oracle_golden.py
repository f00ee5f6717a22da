"""Pins the CPU oracle to the reference's own known answers (CPU only).

- every FNV-64 golden embedded in examples/quant.c and examples/test_matmul.c that is cheap enough
  on the CPU (the rest are checked on the GPU against the same goldens)
- the reference's own compiled CPU GEMM (oracle/_ref, src/npu/core/buf.c:428-477) on the shapes of
  examples/test_cpu_gemm.c:56-61, and against the naive triple loop
- the reference's own compiled uniform int4 channel quantiser (src/npu/i4/quant.c:28-40), RN and SR
"""
import numpy as np
import pytest

import goldens as G
import oracle as O


@pytest.mark.parametrize("idx", range(7))
def test_quant_c_goldens(idx):
    for M, K, N, Aq, Bq, gold, hm in G.quant_c_cases(select={idx}):
        assert G.chained_hash(O.gemm_i32(Aq, Bq), hm) == gold, (M, K, N)


def test_test_matmul_fp16_goldens():
    for M, K, N, A, B, gold, hm in G.tm_fp16_cases():
        C = O.gemm_f16_f32acc(A, B)
        assert G.chained_hash(C, hm) == gold, (M, K, N)
        # integer inputs 0..3: every partial sum is an exact integer < 2^24, so fp64 agrees bit for bit
        assert np.array_equal(C.astype(np.float64), O.gemm_f16_f64acc(A, B))


@pytest.mark.parametrize("shape", [2, 3, 4])
def test_chain_prefill_goldens(shape):
    for M, K, N, A, B, gold, hm in G.tm_chain_cases({shape}):
        assert G.chained_hash(O.gemm_i32(A, B), hm) == gold, (M, K, N)


def test_check_i8_goldens():
    for M, K, N, A, B, gold, hm in G.tm_check_i8_cases():
        assert G.chained_hash(O.gemm_i32(A, B), hm) == gold, (M, K, N)


def test_fnv64_variant():
    # The reference's offset basis is the decimal 1469598103934665603 (examples/quant.c:24), one digit
    # short of the published FNV-1a basis 14695981039346656037; its goldens only reproduce with it.
    assert O.FNV_OFFSET == 1469598103934665603 != 0xCBF29CE484222325
    assert O.fnv64(np.zeros(0, np.uint8)) == O.FNV_OFFSET
    for b in (0x00, 0x61, 0xFF):
        assert O.fnv64(np.array([b], np.uint8)) == ((O.FNV_OFFSET ^ b) * 1099511628211) % (1 << 64)


CPU_GEMM_CASES = [  # examples/test_cpu_gemm.c:56-61: (M, K, N, lo, hi, zero_row)
    (1, 1024, 1024, -8, 7, 0), (32, 1024, 1024, -8, 7, 0), (4, 512, 256, -128, 127, 0),
    (3, 130, 144, -8, 7, 0), (2, 256, 80, -8, 7, 1), (1, 32, 16, -8, 7, 0)]


def test_gemm_vs_naive_and_reference():
    st = O.LCGState(7777)
    for M, K, N, lo, hi, zr in CPU_GEMM_CASES:
        A = O.gen_cpu_gemm(st, lo, hi, M * K).reshape(M, K)
        B = O.gen_cpu_gemm(st, lo, hi, K * N).reshape(K, N)
        if zr:
            A[0, :] = 0
        C = O.gemm_i32(A, B)
        assert np.array_equal(C, O.gemm_i32(A, B, naive=True))
        assert np.array_equal(C, A.astype(np.int64) @ B.astype(np.int64))
        if O.ref_available():
            assert np.array_equal(C, O.ref_gemm_i32(A, B)), (M, K, N)
        if O.ref_omp_available():  # the -fopenmp build (the CPU baseline's all-cores leg): same integers
            assert np.array_equal(C, O.ref_gemm_i32(A, B, omp=True)), (M, K, N)


def test_gemm_int8_extremes_closed_form():
    # all -128 x all -128: every output is exactly 16384*K
    A = np.full((2, 96), -128, np.int8)
    B = np.full((96, 32), -128, np.int8)
    assert np.all(O.gemm_i32(A, B) == 16384 * 96)
    # a single non-zero: C[m][n] = a * b at one position
    A = np.zeros((3, 64), np.int8)
    B = np.zeros((64, 32), np.int8)
    A[1, 17] = -7
    B[17, 5] = 9
    C = O.gemm_i32(A, B)
    assert C[1, 5] == -63 and np.count_nonzero(C) == 1


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (no /root/reference here)")
@pytest.mark.parametrize("sr", [0, 1])
def test_i4_quant_chan_vs_reference(sr):
    import ctypes as C

    rng = np.random.default_rng(11 + sr)
    K = 512
    for trial in range(8):
        fr = (rng.standard_normal(K) * (0.02 + trial)).astype(np.float32)
        if trial == 3:
            fr[::7] = np.float32(3.5)  # exact .5 ties at scale 1 -> round half to even
        scale = np.float32(np.max(np.abs(fr)) / np.float32(7.0)) if trial != 3 else np.float32(1.0)
        seed_r = np.array([0x2545F491], np.uint32)
        seed_o = np.array([0x2545F491], np.uint32)
        nib_r = np.zeros(K // 2, np.uint8)
        nib_o = np.zeros(K // 2, np.uint8)
        qf = np.zeros(K, np.float32)
        codes = np.zeros(K, np.int8)
        O.ref().ref_i4_quant_chan(O._ptr(fr), K, C.c_float(scale), sr, O._ptr(seed_r), O._ptr(nib_r), O._ptr(qf))
        O.lib().oracle_i4_quant_chan(O._ptr(fr), K, C.c_float(scale), sr, O._ptr(seed_o), O._ptr(nib_o), O._ptr(codes))
        assert np.array_equal(nib_r, nib_o)
        assert np.array_equal(qf.astype(np.int8), codes)
        assert seed_r[0] == seed_o[0]
        # the reference's own sign-extending inflate recovers the same codes
        back = np.zeros(K, np.int8)
        O.ref().ref_i4_expand_chan_to_i8(O._ptr(nib_r), K, O._ptr(back))
        assert np.array_equal(back, codes)
