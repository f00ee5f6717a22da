"""Replays the inputs of the reference tests whose outputs are pinned by embedded FNV-64 goldens.

The golden values live in tests/golden/reference_goldens.json; the generators are the reference tests'
own LCG streams, restated in oracle/ork_oracle.c (oracle_gen_*). Each case is yielded as
(M, K, N, A, B, gold, hash_ms): hash the output of rows [:m] for m in hash_ms, chained.
"""
import json
import os

import numpy as np

import oracle as O

GOLD = json.load(open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "reference_goldens.json")))


def _i8_from_rnd(st, n):
    return (O.gen_tm_rnd(st, n).astype(np.int16) - 1).astype(np.int8)


def quant_c_cases(select=None):
    """examples/quant.c: int8 codes from the test's own per-channel quantisation, Ci = Aq x Bq."""
    st = O.LCGState(1)
    for i, (M, K, N, g) in enumerate(GOLD["quant_c"]["cases"]):
        A = O.gen_quant_frand(st, M * K).reshape(M, K)
        B = O.gen_quant_frand(st, K * N).reshape(K, N)
        if select is not None and i not in select:
            continue
        _, Bq = O.quant_test_weights(B)
        _, Aq = O.quant_test_acts(A)
        yield M, K, N, Aq, Bq, int(g, 16), (M,)


def tm_fp16_cases():
    st = O.LCGState(12345)
    for M, K, N, g in GOLD["test_matmul_fp16"]["cases"]:
        A = O.gen_tm_rnd(st, M * K).astype(np.float16).reshape(M, K)
        B = O.gen_tm_rnd(st, K * N).astype(np.float16).reshape(K, N)
        yield M, K, N, A, B, int(g, 16), (1, 1, 4, M)


def _after_fp16():
    st = O.LCGState(12345)
    for M, K, N, _ in GOLD["test_matmul_fp16"]["cases"]:
        O.lcg_skip(st, M * K + K * N)
    return st


def tm_chain_cases(select):
    """examples/test_matmul.c check_chain_prefill shapes (indices into the golden list)."""
    st = _after_fp16()
    shapes = GOLD["test_matmul_chain_prefill"]["shapes"]
    gold = GOLD["test_matmul_chain_prefill"]["gold"]
    for s, (M, K, N) in enumerate(shapes):
        if s not in select:
            O.lcg_skip(st, M * K + K * N)
            continue
        A = _i8_from_rnd(st, M * K).reshape(M, K)
        B = _i8_from_rnd(st, K * N).reshape(K, N)
        yield M, K, N, A, B, int(gold[s], 16), (M,)


def tm_check_i8_cases():
    st = _after_fp16()
    shapes = GOLD["test_matmul_chain_prefill"]["shapes"]
    for M, K, N in shapes[:5]:  # shapes 5 and 6 restore the stream position afterwards
        O.lcg_skip(st, M * K + K * N)
    O.lcg_skip(st, 4 * (512 + 512 * 64))                                   # check_chain_i8
    for m in (1, 8, 40, 96):                                               # check_chain_i8_bf
        O.lcg_skip(st, m * 2048 + 2048 * 768)
    for K, N, M in zip((2048, 512, 4096, 1536, 1024, 2048), (512, 256, 2048, 512, 512, 768), (64, 8, 1, 40, 128, 32)):
        O.lcg_skip(st, M * K + K * N)                                      # check_stream_i8
    O.lcg_skip(st, 768 * 512 + 8 * 768)                                    # check_chain_envelope (a)
    O.lcg_skip(st, 1536 * 256 + 33 * 1536)                                 # check_chain_envelope (b)
    O.lcg_skip(st, 512 * 2048 + 8 * 2048)                                  # check_pack_i8_f32
    O.lcg_skip(st, 512 * 2048 + 8 * 2048)                                  # check_pack_i4a8
    O.lcg_skip(st, 512 * (2048 + 5) + 8 * 2048)                            # check_pack_i4a8_imatrix
    for M, K, N, g in GOLD["test_matmul_check_i8"]["cases"]:
        A = _i8_from_rnd(st, M * K).reshape(M, K)
        B = _i8_from_rnd(st, K * N).reshape(K, N)
        yield M, K, N, A, B, int(g, 16), (1, 1, 4, M)


def chained_hash(C, hash_ms):
    h = O.FNV_OFFSET
    for m in hash_ms:
        h = O.fnv64(np.ascontiguousarray(C[:m]), h)
    return h
