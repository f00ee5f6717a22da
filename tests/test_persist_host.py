"""Persisted weights (OAPK header + resident panels), host side: no GPU needed.

Mirrors the reference's own tests of this surface:
  - examples/test_offline_load.c: CPU dump -> offline load recovers the exact codes, on its shapes
    (single block, long K, wide N, K not a power of two), for int8 and for the W4A4 twin;
  - examples/test_pack_gate.c: the loader must refuse each real failure mode (corrupt magic, another
    format, another caps id, a header K or dtype that disagrees, a pre-header body, a blob shorter than
    the header) while still accepting the honest pack. Its field pokes ((uint32_t *)blob)[0..4] pin the
    header's byte layout to the reference's struct.
The payload is this build's panel layout; it is pinned here against an independent numpy statement of
the layout formula (block (n/16, k/64) of 1 KiB, lane (k%64)/16*16 + n%16, byte k%16).
"""
import ctypes as C
import struct

import numpy as np
import pytest

import ork

HDR = 4096


@pytest.fixture(scope="module")
def off():
    ctx = ork.Npu(offline="gfx950")
    yield ctx
    ctx.close()


def _rand_i8(rng, K, N):
    return rng.integers(-128, 128, size=(K, N), dtype=np.int8)


def _load(L, fn, ctx, K, N, blob):
    b = np.ascontiguousarray(blob, np.uint8)
    return fn(ctx, K, N, ork.ptr(b), b.nbytes)


def test_header_layout(off):
    L = ork.lib()
    assert L.ork_pack_hdr_bytes() == HDR
    B = _rand_i8(np.random.default_rng(1), 96, 64)
    blob = ork.dump_cpu(off.h, B)
    magic, fmt, capid, dtype, K, N, hdr, flags = struct.unpack_from("<IIIIiiII", blob, 0)
    assert magic == 0x4B50414F and bytes(blob[:4]) == b"OAPK"
    assert fmt == L.ork_pack_format_version()
    assert capid != 0
    assert (dtype, K, N, hdr, flags) == (1, 96, 64, HDR, 0)
    assert bytes(blob[32:48]).rstrip(b"\0") == b"gfx950"
    assert not blob[48:HDR].any()                     # zero pad: reproducible blobs
    KB = (96 + 63) // 64
    assert blob.size == HDR + (64 // 16) * KB * 1024  # header + panels


def _panel_i8_ref(B):
    """The int8 panel layout restated: byte of B[k][n] at block (n//16, k//64), lane (k%64)//16*16 + n%16,
    byte k%16 of that lane's 16; K padded with zeros to whole blocks."""
    K, N = B.shape
    KB = (K + 63) // 64
    out = np.zeros((N // 16, KB, 1024), np.uint8)
    k = np.arange(K)[:, None]
    n = np.arange(N)[None, :]
    out[n // 16, k // 64, ((k % 64) // 16 * 16 + n % 16) * 16 + k % 16] = B.view(np.uint8)
    return out.reshape(-1)


def _panel_nib_ref(B):
    """Nibble panels restated: block (n//16, k//128); lane (k%128)//32*16 + n%16; within the lane's 16 bytes,
    dword (k%32)//8, byte k%4, low nibble for k%8 < 4, high nibble otherwise."""
    K, N = B.shape
    KB = (K + 127) // 128
    out = np.zeros((N // 16, KB, 1024), np.uint8)
    for k in range(K):
        r = k % 128
        q = r % 32
        idx = ((r // 32) * 16 + np.arange(N) % 16) * 16 + (q // 8) * 4 + (q % 4)
        nib = (B[k].astype(np.int16) & 0xF).astype(np.uint8) << (4 * ((q % 8) // 4))
        out[np.arange(N) // 16, k // 128, idx] |= nib
    return out.reshape(-1)


@pytest.mark.parametrize("K,N", [(1024, 1024), (4096, 512), (1024, 8192), (1536, 256), (96, 32)])
def test_i8_cpu_dump_offline_load_exact(off, K, N):
    """examples/test_offline_load.c one_i8: CPU dump -> offline load -> codes exact."""
    L = ork.lib()
    B = _rand_i8(np.random.default_rng(K * 7 + N), K, N)
    blob = ork.dump_cpu(off.h, B)
    assert np.array_equal(blob[HDR:], _panel_i8_ref(B))
    w = _load(L, L.ork_i8_mm_load, off.h, K, N, blob)
    assert w
    assert np.array_equal(ork.codes(w, K, N), B)
    # ork_w_dump of the offline weight is the same pack, byte for byte
    assert np.array_equal(ork.dump(w), blob)
    L.ork_mm_free(off.h, w)


@pytest.mark.parametrize("K,N", [(1024, 1024), (4096, 512), (1536, 256), (96, 64)])
def test_i4_cpu_dump_offline_load_exact(off, K, N):
    L = ork.lib()
    B = np.random.default_rng(K + N).integers(-8, 8, size=(K, N), dtype=np.int8)
    blob = ork.dump_cpu(off.h, B, w4a4=True)
    assert np.array_equal(blob[HDR:], _panel_nib_ref(B))
    assert struct.unpack_from("<I", blob, 12)[0] == 2  # dtype I4
    w = _load(L, L.ork_i4_mm_load, off.h, K, N, blob)
    assert w
    assert np.array_equal(ork.codes(w, K, N), B)
    assert np.array_equal(ork.dump(w), blob)
    L.ork_mm_free(off.h, w)
    # an offline W4A4 pack dumps the same bytes as the CPU dumper
    wp = off.pack_i4(B)
    assert np.array_equal(ork.dump(wp), blob)
    L.ork_mm_free(off.h, wp)


def test_offline_pack_dump_matches_cpu_dumper(off):
    L = ork.lib()
    B = _rand_i8(np.random.default_rng(3), 512, 256)
    w = off.pack_i8(B)
    assert np.array_equal(ork.dump(w), ork.dump_cpu(off.h, B))
    L.ork_mm_free(off.h, w)


def _gate_cases(good, K, N):
    """examples/test_pack_gate.c: every blob the loader must refuse."""
    def poke(fmt, off_, val):
        b = good.copy()
        struct.pack_into(fmt, b, off_, val)
        return b

    u32 = lambda i: struct.unpack_from("<I", good, 4 * i)[0]
    return [
        ("corrupt magic", poke("<I", 0, u32(0) ^ 0xFF), K, N),
        ("another format version", poke("<I", 4, u32(1) + 1), K, N),
        ("another caps id", poke("<I", 8, u32(2) ^ 0x5A5A), K, N),
        ("header K disagrees", poke("<i", 16, K * 2), K, N),
        ("header dtype disagrees", poke("<I", 12, 0xDEAD), K, N),
        ("unstamped (body only)", good[HDR:].copy(), K, N),
        ("shorter than the header", good[:16].copy(), K, N),
        ("request N disagrees", good, K, N * 2),
        ("payload truncated", good[:-1024].copy(), K, N),
    ]


def test_pack_gate_refuses_offline(off):
    L = ork.lib()
    K, N = 512, 256
    B = np.array([(i * 37) & 0x7F for i in range(K * N)], np.int32).reshape(K, N).astype(np.int8) - 64
    good = ork.dump_cpu(off.h, B)
    w = _load(L, L.ork_i8_mm_load, off.h, K, N, good)
    assert w, "the honest pack must load, or every refusal below is vacuous"
    L.ork_mm_free(off.h, w)
    for what, blob, k, n in _gate_cases(good, K, N):
        w = _load(L, L.ork_i8_mm_load, off.h, k, n, blob)
        assert not w, what
    # the int8 loader refuses a W4A4 pack of the same K, N and vice versa (dtype in the header)
    g4 = ork.dump_cpu(off.h, np.zeros((K, N), np.int8), w4a4=True)
    assert not _load(L, L.ork_i8_mm_load, off.h, K, N, g4)
    assert not _load(L, L.ork_i4_mm_load, off.h, K, N, good)


def test_dims_and_unsupported_surfaces(off):
    L = ork.lib()
    B = np.zeros((64, 48), np.int8)
    assert L.ork_i8_w_dump_cpu(off.h, 64, 48, ork.ptr(B), None, 0) == 0      # N % 32
    assert L.ork_i8_w_dump_cpu(off.h, 48, 64, ork.ptr(B), None, 0) == 0      # K % 32
    assert L.ork_i4_w_dump_cpu(off.h, 64, 32, ork.ptr(B), None, 0) == 0      # N % 64
    assert L.ork_i8_w_dump_cpu(None, 64, 32, ork.ptr(B), None, 0) == 0       # no context
    good = ork.dump_cpu(off.h, np.zeros((64, 64), np.int8))
    small = np.zeros(good.size - 1, np.uint8)
    Z = np.zeros((64, 64), np.int8)
    assert L.ork_i8_w_dump_cpu(off.h, 64, 64, ork.ptr(Z), ork.ptr(small), small.size) == 0  # cap too small
    assert L.ork_i8_w_dump_bf_cpu(off.h, 512, 64, ork.ptr(np.zeros((512, 64), np.int8)), None, 0) == 0
    assert not _load(L, L.ork_i8_mm_load_import, off.h, 64, 64, good)
    assert not _load(L, L.ork_f16_mm_load_import, off.h, 64, 64, good)
    assert L.ork_w_dump(None, None, 0) == 0
