/* panel.c -- host tilers from the API's weight layouts into the resident panel layout (../hip/orkh.h).
 *
 * Replaces the reference's NPU tilers (orki_i8_tile_range / orki_i8_tile_f32, src/npu/i8/pack.c:40-45,
 * :455-473; orki_f16_tile, src/npu/f16/run.c:32-87; tile_i4_Bslice, src/npu/i4/pack.c:396-402). The
 * layout is a storage choice for gfx950 (one 1 KiB block = one wave load = one MFMA B fragment), not
 * part of any contract: only codes and results are. Tiling runs panel-parallel on the host pool. */
#include <string.h>

#include "internal.h"

static int kpb(int rkind) {
    return rkind == ORKH_I8 ? 64 : rkind == ORKH_F16 ? 32 : 128;
}

size_t orki_panel_bytes(int rkind, int K, int N, int *KB_out) {
    const int KB = (K + kpb(rkind) - 1) / kpb(rkind);
    if (KB_out) *KB_out = KB;
    return (size_t)(N / 16) * KB * 1024;
}

/* ---- int8 ---- */
struct tile_arg {
    const void *src;
    int K, N, KB;
    uint8_t pad;
    uint8_t *out;
};

static void i8_nk_range(int lo, int hi, void *a) {
    const struct tile_arg *t = a;
    const int8_t *src = t->src;
    for (int nb = lo; nb < hi; nb++)
        for (int kb = 0; kb < t->KB; kb++) {
            uint8_t *blk = t->out + ((size_t)nb * t->KB + kb) * 1024;
            for (int l = 0; l < 64; l++) {
                const int n = nb * 16 + (l & 15), k0 = kb * 64 + (l >> 4) * 16;
                if (k0 < t->K) memcpy(blk + l * 16, src + (size_t)n * t->K + k0, 16);
                else memset(blk + l * 16, 0, 16);
            }
        }
}

void orki_tile_i8_nk(const int8_t *codes_nk, int K, int N, int KB, uint8_t *out) {
    struct tile_arg t = {codes_nk, K, N, KB, 0, out};
    orki_parallel_for(N / 16, i8_nk_range, &t);
}

static void i8_kn_range(int lo, int hi, void *a) {
    const struct tile_arg *t = a;
    const int8_t *src = t->src;
    for (int nb = lo; nb < hi; nb++)
        for (int kb = 0; kb < t->KB; kb++) {
            uint8_t *blk = t->out + ((size_t)nb * t->KB + kb) * 1024;
            for (int g = 0; g < 4; g++)
                for (int i = 0; i < 16; i++) {
                    const int k = kb * 64 + g * 16 + i;
                    const int8_t *row = src + (size_t)k * t->N + nb * 16;
                    for (int j = 0; j < 16; j++) blk[(g * 16 + j) * 16 + i] = k < t->K ? (uint8_t)row[j] : 0;
                }
        }
}

void orki_tile_i8_kn(const int8_t *B_kn, int K, int N, int KB, uint8_t *out) {
    struct tile_arg t = {B_kn, K, N, KB, 0, out};
    orki_parallel_for(N / 16, i8_kn_range, &t);
}

/* ---- fp16 ---- */
static void f16_kn_range(int lo, int hi, void *a) {
    const struct tile_arg *t = a;
    const uint16_t *src = t->src;
    for (int nb = lo; nb < hi; nb++)
        for (int kb = 0; kb < t->KB; kb++) {
            uint16_t *blk = (uint16_t *)(t->out + ((size_t)nb * t->KB + kb) * 1024);
            for (int g = 0; g < 4; g++)
                for (int i = 0; i < 8; i++) {
                    const int k = kb * 32 + g * 8 + i;
                    const uint16_t *row = src + (size_t)k * t->N + nb * 16;
                    for (int j = 0; j < 16; j++) blk[(g * 16 + j) * 8 + i] = k < t->K ? row[j] : 0;
                }
        }
}

void orki_tile_f16_kn(const uint16_t *B_kn, int K, int N, int KB, uint8_t *out) {
    struct tile_arg t = {B_kn, K, N, KB, 0, out};
    orki_parallel_for(N / 16, f16_kn_range, &t);
}

/* ---- nibbles ----
 * Block lane l holds column n = nb*16 + l%16, k in [kb*128 + (l/16)*32, +32): dword d, byte b has
 * k = base + d*8 + b in the low nibble and k + 4 in the high nibble. */
static void nib_nk_range(int lo, int hi, void *a) {
    const struct tile_arg *t = a;
    const uint8_t *src = t->src; /* [N][K/2], low nibble = even k */
    const int K = t->K;
    for (int nb = lo; nb < hi; nb++)
        for (int kb = 0; kb < t->KB; kb++) {
            uint8_t *blk = t->out + ((size_t)nb * t->KB + kb) * 1024;
            for (int l = 0; l < 64; l++) {
                const int n = nb * 16 + (l & 15), base = kb * 128 + (l >> 4) * 32;
                const uint8_t *row = src + (size_t)n * (K / 2);
                for (int d = 0; d < 4; d++)
                    for (int b = 0; b < 4; b++) {
                        const int k0 = base + d * 8 + b, k1 = k0 + 4;
                        const unsigned v0 = k0 < K ? (row[k0 >> 1] >> ((k0 & 1) * 4)) & 0xf : t->pad;
                        const unsigned v1 = k1 < K ? (row[k1 >> 1] >> ((k1 & 1) * 4)) & 0xf : t->pad;
                        blk[l * 16 + d * 4 + b] = (uint8_t)(v0 | (v1 << 4));
                    }
            }
        }
}

void orki_tile_nib_nk(const uint8_t *nib_nk, int K, int N, int KB, uint8_t pad, uint8_t *out) {
    struct tile_arg t = {nib_nk, K, N, KB, pad, out};
    orki_parallel_for(N / 16, nib_nk_range, &t);
}

static void nib_kn_range(int lo, int hi, void *a) {
    const struct tile_arg *t = a;
    const int8_t *src = t->src; /* [K][N] int4 values in int8 containers */
    const int K = t->K, N = t->N;
    for (int nb = lo; nb < hi; nb++)
        for (int kb = 0; kb < t->KB; kb++) {
            uint8_t *blk = t->out + ((size_t)nb * t->KB + kb) * 1024;
            for (int l = 0; l < 64; l++) {
                const int n = nb * 16 + (l & 15), base = kb * 128 + (l >> 4) * 32;
                for (int d = 0; d < 4; d++)
                    for (int b = 0; b < 4; b++) {
                        const int k0 = base + d * 8 + b, k1 = k0 + 4;
                        const unsigned v0 = k0 < K ? (unsigned)src[(size_t)k0 * N + n] & 0xf : 0;
                        const unsigned v1 = k1 < K ? (unsigned)src[(size_t)k1 * N + n] & 0xf : 0;
                        blk[l * 16 + d * 4 + b] = (uint8_t)(v0 | (v1 << 4));
                    }
            }
        }
}

void orki_tile_nib_kn(const int8_t *B_kn, int K, int N, int KB, uint8_t *out) {
    struct tile_arg t = {B_kn, K, N, KB, 0, out};
    orki_parallel_for(N / 16, nib_kn_range, &t);
}
