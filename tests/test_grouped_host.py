"""Grouped-scale surfaces on the host (no GPU): pack / set-group gates, the tiled int4 -> int8 load on an
offline context, and grouped runs on an offline context, which compute the per-group accumulate on the CPU as
the reference's offline branches do (src/npu/i8/run.c:48-49, src/npu/i4/run.c:368-369)."""
import numpy as np

import oracle as O

import ork
from test_persist_host import HDR, _load


def test_grouped_gates_offline():
    L = ork.lib()
    with ork.Npu(offline="gfx950") as off:
        K, N = 512, 128
        B = np.random.default_rng(1).integers(-8, 8, size=(K, N), dtype=np.int8)
        for G in (0, 48, 96, 1024, -32):                       # G <= 0, G % 32, K % G, G > K
            assert not L.ork_i4_mm_pack_grouped(off.h, K, N, ork.ptr(B), G), G
        assert not L.ork_i4_mm_pack_grouped(off.h, K, 96, ork.ptr(B[:, :96].copy()), 64)   # N % 64
        w = L.ork_i4_mm_pack_grouped(off.h, K, N, ork.ptr(B), 64)
        assert w and np.array_equal(ork.codes(w, K, N), B)
        rng = np.random.default_rng(3)
        A = rng.integers(-8, 8, size=(2, K), dtype=np.int8)
        aS = rng.uniform(1e-3, 2e-2, size=(2, K // 64)).astype(np.float32)
        bS = rng.uniform(1e-3, 2e-2, size=(K // 64, N)).astype(np.float32)
        for fn in (L.ork_i4_mm_run_grouped, L.ork_i8_mm_run_grouped):   # offline: the CPU accumulate, any dtype
            C = np.zeros((2, N), np.float32)
            assert fn(off.h, w, 2, ork.ptr(A), ork.ptr(aS), ork.ptr(bS), ork.ptr(C)) == 0
            assert np.array_equal(C, O.gemm_grouped(A, B, aS, bS, 64))
        L.ork_mm_free(off.h, w)
        wi = off.pack_i8(B)
        assert L.ork_w_set_group(wi, 64) == 0
        assert L.ork_w_set_group(wi, 96) == -1
        assert L.ork_w_set_group(wi, 0) == 0                       # clears
        assert L.ork_w_set_group(None, 64) == -1
        L.ork_mm_free(off.h, wi)


def test_load_tiled_offline_is_int8():
    L = ork.lib()
    with ork.Npu(offline="gfx950") as off:
        K, N = 1536, 256
        B = np.random.default_rng(2).integers(-8, 8, size=(K, N), dtype=np.int8)
        blob = ork.dump_cpu(off.h, B, w4a4=True)
        assert not L.ork_i4a8_mm_load_tiled(off.h, K, N, ork.ptr(blob), blob.nbytes, 100)   # K % G
        w = L.ork_i4a8_mm_load_tiled(off.h, K, N, ork.ptr(blob), blob.nbytes, 512)
        assert w and np.array_equal(ork.codes(w, K, N), B)
        # it computes as int8: it dumps as an int8 pack of the same codes
        assert np.array_equal(ork.dump(w), ork.dump_cpu(off.h, B))
        L.ork_mm_free(off.h, w)
        # an int8 pack is not a W4A4 pack
        b8 = ork.dump_cpu(off.h, B)
        assert not _load(L, lambda c, k, n, p, s: L.ork_i4a8_mm_load_tiled(c, k, n, p, s, 0), off.h, K, N, b8)
        assert HDR == L.ork_pack_hdr_bytes()
