"""ctypes wrapper over the CPU oracle (oracle/ork_oracle.c) and the reference-built library (oracle/_ref).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() as the checker, and by
bench.py's cpu_baseline leg. The product (ork-driver_amd/) never imports this module.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "_build", "libork_oracle.so")
REF_SO = os.path.join(HERE, "_ref", "libork_ref.so")
REF_OMP_SO = os.path.join(HERE, "_ref", "libork_ref_omp.so")

_P = C.c_void_p
_lib = None
_ref = None
_ref_omp = None


def _ptr(a):
    return a.ctypes.data_as(_P) if a is not None else None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE_SO):
            raise RuntimeError(f"oracle not built: {ORACLE_SO} (run `make -C oracle`)")
        L = C.CDLL(ORACLE_SO)
        L.oracle_fnv64.restype = C.c_uint64
        L.oracle_fnv64.argtypes = [C.c_uint64, _P, C.c_size_t]
        for name in ("oracle_gemm_i32", "oracle_gemm_i32_naive"):
            getattr(L, name).argtypes = [C.c_int, C.c_int, C.c_int, _P, _P, _P]
        L.oracle_chan_scales_f32.argtypes = [_P, C.c_int, C.c_int, _P, _P]
        L.oracle_quant_i8.argtypes = [_P, C.c_int, C.c_int, _P, _P]
        L.oracle_pack_i8_f32.argtypes = [C.c_int, C.c_int, _P, _P, _P]
        L.oracle_pack_i8_f32.restype = C.c_int
        L.oracle_nf4_lut.argtypes = [_P]
        L.oracle_i4_quant_chan.argtypes = [_P, C.c_int, C.c_float, C.c_int, _P, _P, _P]
        L.oracle_nf4_quant_chan.argtypes = [_P, C.c_int, C.c_float, C.c_int, _P, _P, _P]
        L.oracle_wq_err_chan.argtypes = [_P, C.c_int, C.c_float, C.c_int, _P, _P]
        L.oracle_wq_err_chan.restype = C.c_float
        L.oracle_wq_best_absmax.argtypes = [_P, C.c_int, C.c_float, C.c_int, _P, _P]
        L.oracle_wq_best_absmax.restype = C.c_float
        L.oracle_pack_i4a8.argtypes = [C.c_int, C.c_int, _P, _P, C.c_int, C.c_int, _P, _P, _P]
        L.oracle_pack_i4a8.restype = C.c_int
        L.oracle_i4a8_blob.argtypes = [C.c_int, C.c_int, _P, _P, C.c_int, C.c_int, _P, C.c_size_t, _P]
        L.oracle_i4a8_blob.restype = C.c_size_t
        L.oracle_o4n1_decode.argtypes = [C.c_int, C.c_int, _P, C.c_size_t, _P, _P]
        L.oracle_o4n1_decode.restype = C.c_int
        L.oracle_h2f.argtypes = [C.c_uint16]
        L.oracle_h2f.restype = C.c_float
        L.oracle_gemm_f16_f32acc.argtypes = [C.c_int, C.c_int, C.c_int, _P, _P, _P]
        L.oracle_gemm_f16_f64acc.argtypes = [C.c_int, C.c_int, C.c_int, _P, _P, _P]
        L.oracle_gen_quant_frand.argtypes = [_P, _P, C.c_size_t]
        L.oracle_quant_test_weights.argtypes = [C.c_int, C.c_int, _P, _P, _P]
        L.oracle_quant_test_acts.argtypes = [C.c_int, C.c_int, _P, _P, _P]
        L.oracle_gen_tm_rnd.argtypes = [_P, _P, C.c_size_t]
        L.oracle_lcg_skip.argtypes = [C.c_uint32, C.c_uint64]
        L.oracle_lcg_skip.restype = C.c_uint32
        L.oracle_gen_i4_test.argtypes = [C.c_int, C.c_int, C.c_int, _P, _P]
        L.oracle_gen_i4_sattest.argtypes = [C.c_int, C.c_int, C.c_int, _P, _P]
        L.oracle_gen_cpu_gemm.argtypes = [_P, C.c_int, C.c_int, _P, C.c_size_t]
        L.oracle_gen_tm_gauss.argtypes = [_P, _P, C.c_size_t]
        L.oracle_gemm_grouped.argtypes = [C.c_int] * 4 + [_P] * 5
        L.oracle_gemm_grouped.restype = C.c_int
        _lib = L
    return _lib


def ref_available():
    return os.path.exists(REF_SO)


def _load_ref(path):
    R = C.CDLL(path)
    R.ref_gemm_i32.argtypes = [C.c_int, C.c_int, C.c_int, _P, _P, _P]
    R.ref_i4_quant_chan.argtypes = [_P, C.c_int, C.c_float, C.c_int, _P, _P, _P]
    R.ref_i4_expand_chan_to_i8.argtypes = [_P, C.c_int, _P]
    R.ref_gemm_grouped.argtypes = [C.c_int] * 4 + [_P] * 5
    R.ref_gemm_grouped.restype = C.c_int
    R.ref_threads.restype = C.c_int
    return R


def ref():
    """The reference's own CPU functions, compiled from its sources (oracle/ref.mk), single-threaded as the
    reference library is built."""
    global _ref
    if _ref is None:
        if not ref_available():
            raise RuntimeError(f"reference library not built: {REF_SO}")
        _ref = _load_ref(REF_SO)
    return _ref


def ref_omp_available():
    return os.path.exists(REF_OMP_SO)


def ref_omp():
    """The same functions built with -fopenmp: orki_cpu_gemm_i32's row-parallel pragma
    (src/npu/core/buf.c:438) runs on ref_omp().ref_threads() host threads."""
    global _ref_omp
    if _ref_omp is None:
        if not ref_omp_available():
            raise RuntimeError(f"reference OpenMP library not built: {REF_OMP_SO}")
        _ref_omp = _load_ref(REF_OMP_SO)
    return _ref_omp


FNV_OFFSET = 1469598103934665603


def fnv64(arr, h=FNV_OFFSET):
    a = np.ascontiguousarray(arr)
    return lib().oracle_fnv64(h, _ptr(a), a.nbytes)


def gemm_i32(A, B, naive=False):
    """C[M,N] int32 = A[M,K] int8 x B[K,N] int8 (src/npu/core/buf.c:428-477)."""
    A = np.ascontiguousarray(A, dtype=np.int8)
    B = np.ascontiguousarray(B, dtype=np.int8)
    M, K = A.shape
    K2, N = B.shape
    assert K == K2
    Cm = np.empty((M, N), dtype=np.int32)
    fn = lib().oracle_gemm_i32_naive if naive else lib().oracle_gemm_i32
    fn(M, K, N, _ptr(A), _ptr(B), _ptr(Cm))
    return Cm


def ref_gemm_i32(A, B, omp=False):
    """orki_cpu_gemm_i32 as the reference builds it (omp=False: one thread) or with its OpenMP pragma live."""
    A = np.ascontiguousarray(A, dtype=np.int8)
    B = np.ascontiguousarray(B, dtype=np.int8)
    M, K = A.shape
    N = B.shape[1]
    Cm = np.empty((M, N), dtype=np.int32)
    (ref_omp() if omp else ref()).ref_gemm_i32(M, K, N, _ptr(A), _ptr(B), _ptr(Cm))
    return Cm


def _grouped(fn, A, codes, aS, bS, G):
    A = np.ascontiguousarray(A, np.int8)
    B = np.ascontiguousarray(codes, np.int8)
    aS = np.ascontiguousarray(aS, np.float32)
    bS = np.ascontiguousarray(bS, np.float32)
    M, K = A.shape
    N = B.shape[1]
    Cm = np.empty((M, N), np.float32)
    assert fn(M, K, N, G, _ptr(A), _ptr(B), _ptr(aS), _ptr(bS), _ptr(Cm)) == 0
    return Cm


def gemm_grouped(A, codes_kn, aScale, bScale, G):
    """ork_{i4,i8}_mm_run_grouped arithmetic (src/npu/core/buf.c:501-520): C f32 [M][N]; aScale [M][K/G],
    bScale [K/G][N]."""
    return _grouped(lib().oracle_gemm_grouped, A, codes_kn, aScale, bScale, G)


def ref_gemm_grouped(A, codes_kn, aScale, bScale, G):
    return _grouped(ref().ref_gemm_grouped, A, codes_kn, aScale, bScale, G)


def chan_scales_f32(f32_nk):
    f = np.ascontiguousarray(f32_nk, dtype=np.float32)
    N, K = f.shape
    inv = np.empty(N, np.float32)
    bs = np.empty(N, np.float32)
    lib().oracle_chan_scales_f32(_ptr(f), K, N, _ptr(inv), _ptr(bs))
    return inv, bs


def pack_i8_f32(f32_nk):
    """ork_i8_mm_pack_f32 arithmetic: returns (codes[K][N] int8, bscale[N]) or None on bad dims."""
    f = np.ascontiguousarray(f32_nk, dtype=np.float32)
    N, K = f.shape
    codes = np.empty((K, N), np.int8)
    bs = np.empty(N, np.float32)
    if lib().oracle_pack_i8_f32(K, N, _ptr(f), _ptr(bs), _ptr(codes)) != 0:
        return None
    return codes, bs


def nf4_lut():
    lut = np.empty(16, np.int8)
    lib().oracle_nf4_lut(_ptr(lut))
    return lut


def pack_i4a8(f32_nk, imatrix=None, nf4=False, sr=False):
    """ork_i4a8_mm_pack_im arithmetic: returns (bscale[N], nib[N][K/2], codes[K][N])."""
    f = np.ascontiguousarray(f32_nk, dtype=np.float32)
    N, K = f.shape
    im = None if imatrix is None else np.ascontiguousarray(imatrix, dtype=np.float32)
    bs = np.empty(N, np.float32)
    nib = np.zeros((N, K // 2), np.uint8)
    codes = np.empty((K, N), np.int8)
    rc = lib().oracle_pack_i4a8(K, N, _ptr(f), _ptr(im), int(nf4), int(sr), _ptr(bs), _ptr(nib), _ptr(codes))
    if rc != 0:
        return None
    return bs, nib, codes


def i4a8_blob(f32_nk, imatrix=None, nf4=False, sr=False, want_qerr=False):
    """ork_i4a8_pack_cpu_blob(_qerr) bytes (and qerr)."""
    f = np.ascontiguousarray(f32_nk, dtype=np.float32)
    N, K = f.shape
    im = None if imatrix is None else np.ascontiguousarray(imatrix, dtype=np.float32)
    need = lib().oracle_i4a8_blob(K, N, _ptr(f), _ptr(im), int(nf4), int(sr), None, 0, None)
    if need == 0:
        return None
    out = np.zeros(need, np.uint8)
    q = np.zeros(1, np.float32)
    got = lib().oracle_i4a8_blob(K, N, _ptr(f), _ptr(im), int(nf4), int(sr), _ptr(out), need,
                                 _ptr(q) if want_qerr else None)
    assert got == need
    return (out, float(q[0])) if want_qerr else out


def o4n1_decode(K, N, blob):
    b = np.ascontiguousarray(blob, dtype=np.uint8)
    bs = np.empty(N, np.float32)
    codes = np.empty((K, N), np.int8)
    if lib().oracle_o4n1_decode(K, N, _ptr(b), b.nbytes, _ptr(bs), _ptr(codes)) != 0:
        return None
    return bs, codes


def gemm_f16_f32acc(A16, B16):
    A = np.ascontiguousarray(A16, dtype=np.float16)
    B = np.ascontiguousarray(B16, dtype=np.float16)
    M, K = A.shape
    N = B.shape[1]
    Cm = np.empty((M, N), np.float32)
    lib().oracle_gemm_f16_f32acc(M, K, N, _ptr(A), _ptr(B), _ptr(Cm))
    return Cm


def gemm_f16_f64acc(A16, B16):
    A = np.ascontiguousarray(A16, dtype=np.float16)
    B = np.ascontiguousarray(B16, dtype=np.float16)
    M, K = A.shape
    N = B.shape[1]
    Cm = np.empty((M, N), np.float64)
    lib().oracle_gemm_f16_f64acc(M, K, N, _ptr(A), _ptr(B), _ptr(Cm))
    return Cm


def fp16_err(C, R):
    """Per-element relative error with a 0.1%-of-range floor: max|c-r| / max(|r|, 1e-3 max|r|)."""
    C = np.asarray(C, np.float64)
    R = np.asarray(R, np.float64)
    floor = 1e-3 * float(np.max(np.abs(R))) if R.size else 0.0
    den = np.maximum(np.abs(R), floor)
    den[den == 0] = 1.0
    return float(np.max(np.abs(C - R) / den)) if R.size else 0.0


# ---- generators of the reference tests' inputs (for replaying their goldens) ----
class LCGState:
    def __init__(self, sd):
        self.sd = np.array([sd], dtype=np.uint32)


def gen_quant_frand(st, n):
    out = np.empty(n, np.float32)
    lib().oracle_gen_quant_frand(_ptr(st.sd), _ptr(out), n)
    return out


def quant_test_weights(B_kn):
    B = np.ascontiguousarray(B_kn, np.float32)
    K, N = B.shape
    ws = np.empty(N, np.float32)
    Bq = np.empty((K, N), np.int8)
    lib().oracle_quant_test_weights(K, N, _ptr(B), _ptr(ws), _ptr(Bq))
    return ws, Bq


def quant_test_acts(A_mk):
    A = np.ascontiguousarray(A_mk, np.float32)
    M, K = A.shape
    a_s = np.empty(M, np.float32)
    Aq = np.empty((M, K), np.int8)
    lib().oracle_quant_test_acts(M, K, _ptr(A), _ptr(a_s), _ptr(Aq))
    return a_s, Aq


def gen_tm_rnd(st, n):
    out = np.empty(n, np.uint8)
    lib().oracle_gen_tm_rnd(_ptr(st.sd), _ptr(out), n)
    return out


def lcg_skip(st, n):
    st.sd[0] = lib().oracle_lcg_skip(int(st.sd[0]), int(n))


def gen_i4_test(M, K, N):
    A = np.empty((M, K), np.int8)
    B = np.empty((K, N), np.int8)
    lib().oracle_gen_i4_test(M, K, N, _ptr(A), _ptr(B))
    return A, B


def gen_i4_sattest(M, K, N):
    A = np.empty((M, K), np.int8)
    B = np.empty((K, N), np.int8)
    lib().oracle_gen_i4_sattest(M, K, N, _ptr(A), _ptr(B))
    return A, B


def gen_cpu_gemm(st, lo, hi, n):
    out = np.empty(n, np.int8)
    lib().oracle_gen_cpu_gemm(_ptr(st.sd), lo, hi, _ptr(out), n)
    return out


def gen_tm_gauss(st, n):
    out = np.empty(n, np.float32)
    lib().oracle_gen_tm_gauss(_ptr(st.sd), _ptr(out), n)
    return out
