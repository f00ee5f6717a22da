"""ctypes binding of libork_npu.so -- the same C-ABI a C caller links against (include/ork_npu.h).

Used by the tests, smoke() and bench.py to drive the drop-in boundary exactly as the reference's C
examples drive theirs: ork_npu_init -> ork_*_mm_pack -> ork_*_mm_run -> ork_w_free -> ork_npu_free.
Numpy arrays are passed as plain pointers; nothing here computes. Loading fails loudly when the
library has not been built.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libork_npu.so")

_P = C.c_void_p

# Every symbol include/ork_npu.h declares: name -> (restype, argtypes)
API = {
    "ork_npu_version": (C.c_char_p, []),
    "ork_pack_format_version": (C.c_uint32, []),
    "ork_npu_init": (_P, []),
    "ork_npu_init_offline": (_P, [C.c_char_p]),
    "ork_npu_free": (None, [_P]),
    "ork_npu_soc": (C.c_char_p, [_P]),
    "ork_npu_soc_id": (C.c_char_p, [_P]),
    "ork_npu_cores": (C.c_int, [_P]),
    "ork_npu_validated": (C.c_int, [_P]),
    "ork_npu_set_core_budget": (None, [_P, C.c_int]),
    "ork_io_failures": (C.c_long, []),
    "ork_io_expected_failures": (C.c_long, []),
    "ork_dma_alloc": (_P, [_P, C.c_size_t]),
    "ork_dma_free": (None, [_P, _P]),
    "ork_f16_mm_pack": (_P, [_P, C.c_int, C.c_int, _P]),
    "ork_i8_mm_pack": (_P, [_P, C.c_int, C.c_int, _P]),
    "ork_i8_mm_pack_f32": (_P, [_P, C.c_int, C.c_int, _P, _P]),
    "ork_i4a8_mm_pack": (_P, [_P, C.c_int, C.c_int, _P, _P]),
    "ork_i4a8_mm_pack_im": (_P, [_P, C.c_int, C.c_int, _P, _P, _P]),
    "ork_i4_mm_pack": (_P, [_P, C.c_int, C.c_int, _P]),
    "ork_w_free": (None, [_P]),
    "ork_mm_free": (None, [_P, _P]),
    "ork_w_bytes": (C.c_size_t, [_P]),
    "ork_w_dims": (None, [_P, _P, _P]),
    "ork_w_quant_kind": (C.c_int, [_P]),
    "ork_w_bscale": (_P, [_P]),
    "ork_w_codes": (_P, [_P]),
    "ork_i4a8_w_dump": (C.c_size_t, [_P, _P, C.c_size_t]),
    "ork_pack_hdr_bytes": (C.c_size_t, []),
    "ork_i4_mm_pack_grouped": (_P, [_P, C.c_int, C.c_int, _P, C.c_int]),
    "ork_w_set_group": (C.c_int, [_P, C.c_int]),
    "ork_i4a8_mm_load_tiled": (_P, [_P, C.c_int, C.c_int, _P, C.c_size_t, C.c_int]),
    "ork_i8_mm_run_grouped": (C.c_int, [_P, _P, C.c_int, _P, _P, _P, _P]),
    "ork_i4_mm_run_grouped": (C.c_int, [_P, _P, C.c_int, _P, _P, _P, _P]),
    "ork_w_dump": (C.c_size_t, [_P, _P, C.c_size_t]),
    "ork_i8_w_dump_cpu": (C.c_size_t, [_P, C.c_int, C.c_int, _P, _P, C.c_size_t]),
    "ork_i8_w_dump_bf_cpu": (C.c_size_t, [_P, C.c_int, C.c_int, _P, _P, C.c_size_t]),
    "ork_i4_w_dump_cpu": (C.c_size_t, [_P, C.c_int, C.c_int, _P, _P, C.c_size_t]),
    "ork_i8_mm_load": (_P, [_P, C.c_int, C.c_int, _P, C.c_size_t]),
    "ork_i4_mm_load": (_P, [_P, C.c_int, C.c_int, _P, C.c_size_t]),
    "ork_f16_mm_load": (_P, [_P, C.c_int, C.c_int, _P, C.c_size_t]),
    "ork_i8_mm_load_import": (_P, [_P, C.c_int, C.c_int, _P, C.c_size_t]),
    "ork_f16_mm_load_import": (_P, [_P, C.c_int, C.c_int, _P, C.c_size_t]),
    "ork_i4a8_mm_load": (_P, [_P, C.c_int, C.c_int, _P, C.c_size_t]),
    "ork_i4a8_pack_cpu_blob": (C.c_size_t, [_P, C.c_int, C.c_int, _P, _P, C.c_int, _P, C.c_size_t]),
    "ork_i4a8_pack_cpu_blob_qerr": (C.c_size_t, [_P, C.c_int, C.c_int, _P, _P, C.c_int, _P, C.c_size_t, _P]),
    "ork_f16_mm_run": (C.c_int, [_P, _P, C.c_int, _P, _P]),
    "ork_i8_mm_run": (C.c_int, [_P, _P, C.c_int, _P, _P]),
    "ork_i8_mm_run_noalloc": (C.c_int, [_P, _P, C.c_int, _P, _P]),
    "ork_i8_mm_run_row": (C.c_int, [_P, C.c_int, _P, _P]),
    "ork_i4_mm_run": (C.c_int, [_P, _P, C.c_int, _P, _P]),
    "ork_i8_mm_run_cpu": (None, [C.c_int, C.c_int, C.c_int, _P, _P, _P]),
    "ork_i8_mm_run_chain": (C.c_int, [_P, C.c_int, _P]),
    "ork_i8_mm_run_stream": (C.c_int, [_P, C.c_int, _P]),
    "ork_i4_mm_run_chain": (C.c_int, [_P, C.c_int, _P]),
    "ork_i4_mm_run_stream": (C.c_int, [_P, C.c_int, _P]),
    "ork_f16_mm_run_stream": (C.c_int, [_P, C.c_int, _P]),
    "ork_dev_alloc": (_P, [_P, C.c_size_t]),
    "ork_dev_free": (None, [_P, _P]),
    "ork_dev_upload": (C.c_int, [_P, _P, _P, C.c_size_t]),
    "ork_dev_download": (C.c_int, [_P, _P, _P, C.c_size_t]),
    "ork_npu_set_async": (None, [_P, C.c_int]),
    "ork_npu_sync": (C.c_int, [_P]),
    "ork_npu_stream": (_P, [_P]),
    "ork_npu_mark": (C.c_int, [_P, _P]),
    "ork_npu_wallclock_khz": (C.c_int, [_P]),
    "ork_npu_read_probe": (C.c_longlong, [_P, _P, C.c_size_t, _P]),
    "ork_w_device_panels": (C.c_int, [_P, _P, _P, _P, _P]),
    "ork_w_plan_name": (C.c_char_p, [_P, _P, C.c_int]),
    "ork_w_grouped_plan_name": (C.c_char_p, [_P, _P, C.c_int]),
}



class TaskI8(C.Structure):
    """ork_mm_task_i8 (include/ork/chain.h)"""
    _fields_ = [("w", _P), ("M", C.c_int), ("A", _P), ("C", _P), ("cstride", C.c_int)]


class TaskI4(C.Structure):
    """ork_mm_task_i4 / ork_mm_task_f16 (same layout: w, M, A, C)"""
    _fields_ = [("w", _P), ("M", C.c_int), ("A", _P), ("C", _P)]


TaskF16 = TaskI4

ROW_RMSNORM, ROW_QUANT = 0, 1                 # ork_row_op.prologue (include/ork/hip.h)
COL_STORE, COL_RESID, COL_SWIGLU = 0, 1, 2    # ork_row_op.epilogue


class RowOp(C.Structure):
    """ork_row_op (include/ork/hip.h): device pointers as ints"""
    _fields_ = [("prologue", C.c_int), ("row", _P), ("norm_w", _P), ("eps", C.c_float), ("row_scale", _P),
                ("epilogue", C.c_int), ("C", _P * 3), ("w_scale", _P * 2), ("out", _P)]


def tasks(cls, rows):
    """A ctypes array of task structs from tuples (w, M, A, C[, cstride]); A and C are arrays or ints. The structs
    hold raw pointers only: the caller keeps the arrays alive until the run has returned."""
    arr = (cls * len(rows))()
    for i, r in enumerate(rows):
        arr[i].w = r[0]
        arr[i].M = r[1]
        arr[i].A = ptr(r[2])
        arr[i].C = ptr(r[3])
        if len(r) > 4:
            arr[i].cstride = r[4]
    return arr


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"libork_npu.so is not built ({LIB_PATH}); run __graft_entry__.build()")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in API.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def ptr(a):
    if a is None:
        return None
    if isinstance(a, int):
        return a
    return a.ctypes.data_as(_P)


class Npu:
    """One device context (ork_npu *). Weights are plain handles (ints); free them explicitly."""

    def __init__(self, offline=None):
        L = lib()
        self.h = L.ork_npu_init_offline(offline.encode()) if offline else L.ork_npu_init()
        if not self.h:
            raise RuntimeError("ork_npu_init failed")

    def close(self):
        if self.h:
            lib().ork_npu_free(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    # ---- packs ----
    def pack_i8(self, B_kn):
        B = np.ascontiguousarray(B_kn, np.int8)
        return lib().ork_i8_mm_pack(self.h, B.shape[0], B.shape[1], ptr(B))

    def pack_i8_f32(self, f32_nk, want_bscale=True):
        f = np.ascontiguousarray(f32_nk, np.float32)
        N, K = f.shape
        bs = np.empty(N, np.float32) if want_bscale else None
        w = lib().ork_i8_mm_pack_f32(self.h, K, N, ptr(f), ptr(bs))
        return (w, bs) if want_bscale else w

    def pack_f16(self, B_kn):
        B = np.ascontiguousarray(B_kn, np.float16)
        return lib().ork_f16_mm_pack(self.h, B.shape[0], B.shape[1], ptr(B))

    def pack_i4a8(self, f32_nk, imatrix=None, want_bscale=True):
        f = np.ascontiguousarray(f32_nk, np.float32)
        N, K = f.shape
        bs = np.empty(N, np.float32) if want_bscale else None
        im = None if imatrix is None else np.ascontiguousarray(imatrix, np.float32)
        w = lib().ork_i4a8_mm_pack_im(self.h, K, N, ptr(f), ptr(im), ptr(bs))
        return (w, bs) if want_bscale else w

    def pack_i4(self, B_kn):
        B = np.ascontiguousarray(B_kn, np.int8)
        return lib().ork_i4_mm_pack(self.h, B.shape[0], B.shape[1], ptr(B))

    def load_i4a8(self, K, N, blob):
        b = np.ascontiguousarray(blob, np.uint8)
        return lib().ork_i4a8_mm_load(self.h, K, N, ptr(b), b.nbytes)

    # ---- runs: return (rc, C) ----
    def run_i8(self, w, A, C=None):
        A = np.ascontiguousarray(A, np.int8)
        M = A.shape[0]
        N = dims(w)[1]
        if C is None:
            C = np.empty((M, N), np.int32)
        return lib().ork_i8_mm_run(self.h, w, M, ptr(A), ptr(C)), C

    def run_i4(self, w, A, C=None):
        A = np.ascontiguousarray(A, np.int8)
        M = A.shape[0]
        N = dims(w)[1]
        if C is None:
            C = np.empty((M, N), np.int32)
        return lib().ork_i4_mm_run(self.h, w, M, ptr(A), ptr(C)), C

    def run_f16(self, w, A, C=None):
        A = np.ascontiguousarray(A, np.float16)
        M = A.shape[0]
        N = dims(w)[1]
        if C is None:
            C = np.empty((M, N), np.float32)
        return lib().ork_f16_mm_run(self.h, w, M, ptr(A), ptr(C)), C

    def plan_name(self, w, M):
        return lib().ork_w_plan_name(self.h, w, M).decode()

    def grouped_plan_name(self, w, M):
        return lib().ork_w_grouped_plan_name(self.h, w, M).decode()


def dims(w):
    K = C.c_int()
    N = C.c_int()
    lib().ork_w_dims(w, C.byref(K), C.byref(N))
    return K.value, N.value


def free(w):
    lib().ork_w_free(w)


def bscale(w, N):
    p = lib().ork_w_bscale(w)
    if not p:
        return None
    return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_float)), shape=(N,)).copy()


def codes(w, K, N):
    p = lib().ork_w_codes(w)
    if not p:
        return None
    return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_int8)), shape=(K, N)).copy()


def dump_i4a8(w):
    L = lib()
    need = L.ork_i4a8_w_dump(w, None, 0)
    if not need:
        return None
    out = np.zeros(need, np.uint8)
    got = L.ork_i4a8_w_dump(w, ptr(out), need)
    assert got == need
    return out


def dump(w):
    """ork_w_dump: the 4 KiB OAPK header + the resident panels, or None."""
    L = lib()
    need = L.ork_w_dump(w, None, 0)
    if not need:
        return None
    out = np.zeros(need, np.uint8)
    assert L.ork_w_dump(w, ptr(out), need) == need
    return out


def dump_cpu(ctx, B_kn, w4a4=False):
    """ork_i8_w_dump_cpu / ork_i4_w_dump_cpu of B[K][N], or None."""
    B = np.ascontiguousarray(B_kn, np.int8)
    K, N = B.shape
    fn = lib().ork_i4_w_dump_cpu if w4a4 else lib().ork_i8_w_dump_cpu
    need = fn(ctx, K, N, ptr(B), None, 0)
    if not need:
        return None
    out = np.zeros(need, np.uint8)
    assert fn(ctx, K, N, ptr(B), ptr(out), need) == need
    return out


def cpu_blob(K, N, f32_nk, imatrix=None, nf4=False, ctx=None, qerr=False):
    f = np.ascontiguousarray(f32_nk, np.float32)
    im = None if imatrix is None else np.ascontiguousarray(imatrix, np.float32)
    L = lib()
    need = L.ork_i4a8_pack_cpu_blob(ctx, K, N, ptr(f), ptr(im), int(nf4), None, 0)
    if not need:
        return None
    out = np.zeros(need, np.uint8)
    q = np.zeros(1, np.float32)
    got = L.ork_i4a8_pack_cpu_blob_qerr(ctx, K, N, ptr(f), ptr(im), int(nf4), ptr(out), need,
                                        ptr(q) if qerr else None)
    assert got == need
    return (out, float(q[0])) if qerr else out
