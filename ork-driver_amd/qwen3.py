"""ctypes binding of libork_qwen3.so, the Qwen3-shaped decoder harness (csrc/qwen3/qwen3.h).

The harness is a consumer of the public matmul API (like the reference's examples/bench.c): its
projections and LM head are ork_i8_mm_run / ork_i8_mm_run_chain calls on resident weights; its
non-matmul operators are fused HIP kernels. Nothing here computes; loading fails loudly when the
library has not been built.
"""
import ctypes as C
import os

import numpy as np

import ork

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libork_qwen3.so")
_P = C.c_void_p

WQ, WK, WV, WO, WG, WU, WD = range(7)
N_ATTN, N_FFN, N_Q, N_K = range(4)
LINEARS = (WQ, WK, WV, WO, WG, WU, WD)


class Cfg(C.Structure):
    """q3_cfg"""
    _fields_ = [(n, C.c_int) for n in ("layers", "hidden", "heads", "kv_heads", "head_dim", "ffn", "vocab",
                                        "max_ctx", "max_rows", "ffn_nf4")] + \
               [("rope_theta", C.c_float), ("eps", C.c_float)]


# Qwen3-1.7B (examples/bench.c:19-28 shapes; rope_theta and eps from the Qwen3 configuration)
QWEN3_1P7B = dict(layers=28, hidden=2048, heads=16, kv_heads=8, head_dim=128, ffn=6144, vocab=151936,
                  rope_theta=1e6, eps=1e-6)

API = {
    "q3_create": (_P, [_P, C.POINTER(Cfg)]),
    "q3_free": (None, [_P]),
    "q3_set_linear": (C.c_int, [_P, C.c_int, C.c_int, _P]),
    "q3_set_norm": (C.c_int, [_P, C.c_int, C.c_int, _P]),
    "q3_init_random": (C.c_int, [_P, C.c_uint64, C.c_float]),
    "q3_gen_linear": (C.c_int, [C.POINTER(Cfg), C.c_uint64, C.c_float, C.c_int, C.c_int, _P]),
    "q3_prefill": (C.c_int, [_P, _P, C.c_int]),
    "q3_decode": (C.c_int, [_P, C.c_int, C.c_int]),
    "q3_tokens": (C.c_int, [_P, _P, C.c_int]),
    "q3_positions": (C.c_int, [_P]),
    "q3_last_logits": (C.c_int, [_P, _P]),
    "q3_weight_bytes": (C.c_double, [_P]),
    "q3_set_fused": (C.c_int, [_P, C.c_int]),
    "q3_decode_fused": (C.c_int, [_P]),
    "q3_set_trace": (C.c_int, [_P, C.c_int]),
    "q3_layer_rows": (C.c_int, [_P, C.c_int, _P, C.c_int]),
}

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"libork_qwen3.so is not built ({LIB_PATH}); run __graft_entry__.build()")
        ork.lib()  # libork_npu.so first (the harness links it)
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in API.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def make_cfg(max_ctx, max_rows, ffn_nf4=0, **shape):
    c = Cfg()
    for k, v in shape.items():
        setattr(c, k, v)
    c.max_ctx, c.max_rows, c.ffn_nf4 = max_ctx, max_rows, int(ffn_nf4)
    return c


def lin_shape(cfg, layer, which):
    """(N, K) of a linear, as q3_set_linear takes it (f32[N][K])."""
    H, QD, KVD = cfg.hidden, cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
    if layer == -1:
        return cfg.vocab, H
    return {WQ: (QD, H), WK: (KVD, H), WV: (KVD, H), WO: (H, QD), WG: (cfg.ffn, H), WU: (cfg.ffn, H),
            WD: (H, cfg.ffn)}[which]


def gen_linear(cfg, seed, std, layer, which):
    N, K = lin_shape(cfg, layer, which)
    out = np.empty((N, K), np.float32)
    assert lib().q3_gen_linear(C.byref(cfg), seed, std, layer, which, ork.ptr(out)) == 0
    return out


class Model:
    """One harness model on an ork.Npu context."""

    def __init__(self, npu, cfg):
        self.cfg = cfg
        self.npu = npu
        self.h = lib().q3_create(npu.h, C.byref(cfg))
        if not self.h:
            raise RuntimeError("q3_create failed")

    def close(self):
        if self.h:
            lib().q3_free(self.h)
            self.h = None

    def set_linear(self, layer, which, w_nk):
        w = np.ascontiguousarray(w_nk, np.float32)
        assert w.shape == lin_shape(self.cfg, layer, which)
        return lib().q3_set_linear(self.h, layer, which, ork.ptr(w))

    def set_norm(self, layer, which, w):
        return lib().q3_set_norm(self.h, layer, which, ork.ptr(np.ascontiguousarray(w, np.float32)))

    def init_random(self, seed, std=0.02):
        return lib().q3_init_random(self.h, seed, std)

    def prefill(self, tokens):
        t = np.ascontiguousarray(tokens, np.int32)
        return lib().q3_prefill(self.h, ork.ptr(t), t.size)

    def decode(self, steps, graph=True):
        return lib().q3_decode(self.h, steps, int(graph))

    def set_fused(self, on):
        """Decode through the fused M = 1 kernels (default) or the unfused operator sequence."""
        return lib().q3_set_fused(self.h, int(on))

    def decode_fused(self):
        """Whether decode steps take the fused kernels with the current weights."""
        return bool(lib().q3_decode_fused(self.h))

    def positions(self):
        return lib().q3_positions(self.h)

    def tokens(self):
        """Tokens at every filled position plus the token sampled last."""
        n = self.positions() + 1
        out = np.zeros(n, np.int32)
        assert lib().q3_tokens(self.h, ork.ptr(out), n) == 0
        return out

    def last_logits(self):
        out = np.empty(self.cfg.vocab, np.float32)
        assert lib().q3_last_logits(self.h, ork.ptr(out)) == 0
        return out

    def set_trace(self, on):
        """Keep the residual rows entering each layer (and leaving the last) of every later pass."""
        return lib().q3_set_trace(self.h, int(on))

    def layer_rows(self, l, rows):
        """f32[rows][hidden]: the rows entering layer l in the last pass (l = layers: leaving the last layer)."""
        out = np.empty((rows, self.cfg.hidden), np.float32)
        assert lib().q3_layer_rows(self.h, l, ork.ptr(out), rows) == 0
        return out

    def weight_bytes(self):
        return lib().q3_weight_bytes(self.h)
