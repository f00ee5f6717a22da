// Host-memory stand-ins for the thin HIP layer (ork-driver_amd/csrc/hip/orkh.h), so that the host library can run
// under AddressSanitizer on a machine without a GPU (tests/test_host_asan.py): "device" buffers are malloc'd, every
// copy is a memcpy of exactly the size the library asks for (so ASan checks each transfer against both buffers),
// pointer queries consult the list of live "device" buffers, and launches do nothing (no results are checked).
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include "orkh.h"
int orkh_device_count(void) { return 1; }
int orkh_init(int ordinal, orkh_dev *out, void **stream_out) {
    if (out) { memset(out, 0, sizeof *out); out->ordinal = ordinal; out->cu_count = 256; out->clock_khz = 2400000;
        out->lds_per_block = 163840; out->hbm_bytes = (size_t)288 << 30; out->l2_bytes = 4 << 20;
        snprintf(out->arch, sizeof out->arch, "gfx950"); snprintf(out->name, sizeof out->name, "stub"); out->scratch = malloc(ORKH_SCRATCH_BYTES); out->wall_khz = 100000; }
    if (stream_out) *stream_out = (void *)0x1;
    return 0;
}
void orkh_stream_destroy(void *s) { (void)s; }
const char *orkh_last_error(void) { return "stub"; }
const char *orkh_launch_error(void) { return ""; }
#define MAXP 100000
static void *devp[MAXP]; static size_t devn[MAXP]; static int ndev;
void *orkh_malloc(size_t n) { void *p = malloc(n ? n : 1); if (ndev < MAXP) { devp[ndev] = p; devn[ndev++] = n; } return p; }
int orkh_free(void *p) { for (int i = 0; i < ndev; i++) if (devp[i] == p) { devp[i] = devp[--ndev]; devn[i] = devn[ndev]; break; } free(p); return 0; }
void *orkh_host_alloc(size_t n) { return malloc(n ? n : 1); }
int orkh_host_free(void *p) { free(p); return 0; }
void *orkh_host_devptr(void *p) { return p; }
int orkh_h2d(void *d, const void *s, size_t n, void *st) { (void)st; if (n) memcpy(d, s, n); return 0; }
int orkh_d2h(void *d, const void *s, size_t n, void *st) { (void)st; if (n) memcpy(d, s, n); return 0; }
int orkh_d2d(void *d, const void *s, size_t n, void *st) { (void)st; if (n) memmove(d, s, n); return 0; }
int orkh_d2h_2d(void *d, size_t dp, const void *s, size_t sp, size_t w, size_t r, void *st) {
    (void)st; for (size_t i = 0; i < r; i++) memcpy((char *)d + i * dp, (const char *)s + i * sp, w); return 0; }
int orkh_sync(void *s) { (void)s; return 0; }
int orkh_mark(void *p, void *s) { (void)s; memset(p, 0, 8); return 0; }
long long orkh_read_probe(const void *dev, size_t bytes, unsigned *sink, void *s) {
    (void)s;
    const long long grid = (long long)((bytes / 16 + 511) / 512);
    for (long long g = 0; g < grid; g++) {
        unsigned x = 0;
        for (size_t i = (size_t)g * 2048; i < bytes / 4 && i < (size_t)(g + 1) * 2048; i++) x ^= ((const unsigned *)dev)[i];
        sink[g] = x;
    }
    return grid;
}
int orkh_device_sync(void) { return 0; }
int orkh_stream_capturing(void *s) { (void)s; return 0; }
int orkh_row_launch(const orkh_row *p, void *s) { (void)p; (void)s; return 0; }
void *orkh_event_new(void) { return malloc(8); }
void orkh_event_free(void *e) { free(e); }
int orkh_event_record(void *e, void *s) { (void)s; memset(e, 0, 8); return 0; }
float orkh_event_ms(void *e0, void *e1) { (void)e0; (void)e1; return 0.001f; }
int orkh_ptr_is_device(const void *p) { for (int i = 0; i < ndev; i++) if ((const char *)p >= (char *)devp[i] && (const char *)p < (char *)devp[i] + (devn[i] ? devn[i] : 1)) return 1; return 0; }
int orkh_mm_launch(const orkh_mm *p, const orkh_plan *q, void *s) { (void)p; (void)q; (void)s; return 0; }
int orkh_mm_launch_grouped(const orkh_mm *p, const orkh_plan *q, int G, const float *aS, const float *bS, float *C, int ldc, void *s) { (void)ldc;
    (void)p; (void)q; (void)G; (void)aS; (void)bS; (void)C; (void)s; return 0; }
int orkh_mm_launch_group(const orkh_group *g, int wpg, void *s) { (void)g; (void)wpg; (void)s; return 0; }
int orkh_mm_launch_tgroup(const orkh_mm *p, int n, const orkh_plan *q, void *s) { (void)p; (void)n; (void)q; (void)s; return 0; }
int orkh_tiled2_ring_lds(int kind, int bm, int bn) { (void)kind; (void)bm; (void)bn; return 65536; }
int orkh_tiled2_ring2_ok(int kind, int bm, int bn) { (void)kind; (void)bm; (void)bn; return 0; }
const char *orkh_mm_variant(const orkh_mm *p, const orkh_plan *q) { (void)p; (void)q; return "stub"; }
