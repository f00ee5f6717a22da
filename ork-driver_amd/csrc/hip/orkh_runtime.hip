// orkh_runtime.hip -- device, memory and stream half of the thin C-ABI HIP layer (see orkh.h).
//
// Replaces the reference's L1 substrate for the matmul path: orki_bcreate / MEM_CREATE+MAP
// (src/npu/core/buf.c:47-80) become hipMalloc, orki_bsync cache maintenance becomes async copies on
// the context's stream, and the DRM submit ioctl (src/npu/core/submit.c:270-296) becomes a kernel
// launch on that stream (orkh_kernels.hip).
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <string.h>

#include "orkh.h"

static thread_local char g_err[256];

// The split-K workspace of the no-allocation run (ork_i8_mm_run_noalloc): one copy per GPU, 256-byte aligned like
// hipMalloc memory. Host code never uses this name as an address (on the host it is only a stand-in for the
// symbol): orkh_init resolves each device's copy with hipGetSymbolAddress and hands that pointer out.
static __device__ __align__(256) unsigned char scratch[ORKH_SCRATCH_BYTES];

static int fail(hipError_t e, const char *what) {
    snprintf(g_err, sizeof g_err, "%s: %s", what, hipGetErrorString(e));
    return -1;
}
#define CK(call, what)                                  \
    do {                                                \
        hipError_t e_ = (call);                         \
        if (e_ != hipSuccess) return fail(e_, what);    \
    } while (0)

// One thread stores the device wall clock (constant rate, orkh_dev.wall_khz): a timestamp in stream order.
__global__ void k_mark(unsigned long long *p) { *p = wall_clock64(); }

// Profiling: a plain streaming read of n16 16-byte chunks -- the M = 1 GEMV's loads without its arithmetic. Each
// workgroup of 4 waves reads RP_U contiguous KiB-runs per wave (RP_U loads per lane, all issued before any is
// used), XOR-folds them and stores one word, so a caller can check that every byte was read.
constexpr int RP_U = 2;
typedef int rp_v4i __attribute__((ext_vector_type(4)));
__global__ __launch_bounds__(256) void k_read_probe(const rp_v4i *__restrict__ p, long long n16, unsigned *sink) {
    __shared__ unsigned red[4];
    const long long i0 = (long long)blockIdx.x * (256 * RP_U) + threadIdx.x;
    rp_v4i r[RP_U];
#pragma unroll
    for (int u = 0; u < RP_U; u++) {
        const long long i = i0 + (long long)u * 256;
        r[u] = __builtin_nontemporal_load(p + (i < n16 ? i : n16 - 1));
    }
    unsigned x = 0;
#pragma unroll
    for (int u = 0; u < RP_U; u++)
        if (i0 + (long long)u * 256 < n16) x ^= (unsigned)(r[u].x ^ r[u].y ^ r[u].z ^ r[u].w);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x ^= (unsigned)__shfl_xor((int)x, o, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = x;
    __syncthreads();
    if (threadIdx.x == 0) sink[blockIdx.x] = red[0] ^ red[1] ^ red[2] ^ red[3];
}

extern "C" {

const char *orkh_last_error(void) { return g_err; }

int orkh_mark(void *dev_u64, void *stream) {
    if (!dev_u64 || (uintptr_t)dev_u64 % 8) {
        snprintf(g_err, sizeof g_err, "orkh_mark: destination must be 8-byte aligned device memory");
        return -1;
    }
    hipLaunchKernelGGL(k_mark, dim3(1), dim3(1), 0, (hipStream_t)stream, (unsigned long long *)dev_u64);
    CK(hipGetLastError(), "k_mark launch");
    return 0;
}

long long orkh_read_probe(const void *dev, size_t bytes, unsigned *sink, void *stream) {
    if (!dev || !sink || !bytes || bytes % 16 || (uintptr_t)dev % 16 || (uintptr_t)sink % 4) {
        snprintf(g_err, sizeof g_err, "orkh_read_probe: 16-byte aligned device bytes (a multiple of 16) and a "
                                      "4-byte aligned sink are required");
        return -1;
    }
    const long long n16 = (long long)(bytes / 16), grid = (n16 + 256 * RP_U - 1) / (256 * RP_U);
    if (grid >= (1LL << 31)) {
        snprintf(g_err, sizeof g_err, "orkh_read_probe: %zu bytes is too many", bytes);
        return -1;
    }
    hipLaunchKernelGGL(k_read_probe, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream, (const rp_v4i *)dev, n16,
                       sink);
    CK(hipGetLastError(), "k_read_probe launch");
    return grid;
}

int orkh_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

int orkh_init(int ordinal, orkh_dev *out, void **stream_out) {
    int n = 0;
    CK(hipGetDeviceCount(&n), "hipGetDeviceCount");
    if (ordinal < 0 || ordinal >= n) {
        snprintf(g_err, sizeof g_err, "device %d not present (%d visible)", ordinal, n);
        return -1;
    }
    CK(hipSetDevice(ordinal), "hipSetDevice");
    hipDeviceProp_t p;
    CK(hipGetDeviceProperties(&p, ordinal), "hipGetDeviceProperties");
    // this device's address of the scratch array, with the device current (each GPU holds its own copy)
    void *scr = nullptr;
    CK(hipGetSymbolAddress(&scr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    if (!scr) {
        snprintf(g_err, sizeof g_err, "hipGetSymbolAddress(scratch): NULL on device %d", ordinal);
        return -1;
    }
    if (out) {
        memset(out, 0, sizeof *out);
        out->ordinal = ordinal;
        out->cu_count = p.multiProcessorCount;
        out->clock_khz = p.clockRate;
        out->mem_clock_khz = p.memoryClockRate;
        out->mem_bus_bits = p.memoryBusWidth;
        out->lds_per_block = p.sharedMemPerBlock;
        out->hbm_bytes = p.totalGlobalMem;
        out->l2_bytes = p.l2CacheSize;
        snprintf(out->arch, sizeof out->arch, "%s", p.gcnArchName);
        snprintf(out->name, sizeof out->name, "%s", p.name);
        out->scratch = scr;
        int wk = 0;
        if (hipDeviceGetAttribute(&wk, hipDeviceAttributeWallClockRate, ordinal) != hipSuccess) wk = 0;
        out->wall_khz = wk;
    }
    if (stream_out) {
        hipStream_t s;
        // Default priority on purpose: one in-order stream per context.
        CK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate");
        *stream_out = (void *)s;
    }
    return 0;
}

void orkh_stream_destroy(void *stream) {
    if (stream) (void)hipStreamDestroy((hipStream_t)stream);
}

void *orkh_malloc(size_t n) {
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, n ? n : 1);
    if (e != hipSuccess) { fail(e, "hipMalloc"); return nullptr; }
    return p;
}

int orkh_free(void *p) {
    if (!p) return 0;
    CK(hipFree(p), "hipFree");
    return 0;
}

void *orkh_host_alloc(size_t n) {
    void *p = nullptr;
    hipError_t e = hipHostMalloc(&p, n ? n : 1, hipHostMallocMapped | hipHostMallocPortable);
    if (e != hipSuccess) { fail(e, "hipHostMalloc"); return nullptr; }
    return p;
}

int orkh_host_free(void *p) {
    if (!p) return 0;
    CK(hipHostFree(p), "hipHostFree");
    return 0;
}

void *orkh_host_devptr(void *p) {
    void *d = nullptr;
    hipError_t e = hipHostGetDevicePointer(&d, p, 0);
    if (e != hipSuccess) { fail(e, "hipHostGetDevicePointer"); return nullptr; }
    return d;
}

int orkh_h2d(void *dst, const void *src, size_t n, void *stream) {
    if (!n) return 0;
    CK(hipMemcpyAsync(dst, src, n, hipMemcpyDefault, (hipStream_t)stream), "hipMemcpyAsync H2D");
    return 0;
}

int orkh_d2h(void *dst, const void *src, size_t n, void *stream) {
    if (!n) return 0;
    CK(hipMemcpyAsync(dst, src, n, hipMemcpyDefault, (hipStream_t)stream), "hipMemcpyAsync D2H");
    return 0;
}

int orkh_d2h_2d(void *dst, size_t dpitch, const void *src, size_t spitch, size_t width, size_t rows, void *stream) {
    if (!width || !rows) return 0;
    CK(hipMemcpy2DAsync(dst, dpitch, src, spitch, width, rows, hipMemcpyDefault, (hipStream_t)stream),
       "hipMemcpy2DAsync D2H");
    return 0;
}

int orkh_d2d(void *dst, const void *src, size_t n, void *stream) {
    if (!n) return 0;
    CK(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToDevice, (hipStream_t)stream), "hipMemcpyAsync D2D");
    return 0;
}

int orkh_sync(void *stream) {
    CK(hipStreamSynchronize((hipStream_t)stream), "hipStreamSynchronize");
    return 0;
}

void *orkh_event_new(void) {
    hipEvent_t e = nullptr;
    hipError_t r = hipEventCreate(&e);
    if (r != hipSuccess) { fail(r, "hipEventCreate"); return nullptr; }
    return (void *)e;
}

void orkh_event_free(void *ev) {
    if (ev) (void)hipEventDestroy((hipEvent_t)ev);
}

int orkh_event_record(void *ev, void *stream) {
    CK(hipEventRecord((hipEvent_t)ev, (hipStream_t)stream), "hipEventRecord");
    return 0;
}

float orkh_event_ms(void *e0, void *e1) {
    if (hipEventSynchronize((hipEvent_t)e1) != hipSuccess) return -1.f;
    float ms = -1.f;
    if (hipEventElapsedTime(&ms, (hipEvent_t)e0, (hipEvent_t)e1) != hipSuccess) return -1.f;
    return ms;
}

int orkh_stream_capturing(void *stream) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing((hipStream_t)stream, &st) != hipSuccess) return -1;
    return st == hipStreamCaptureStatusActive ? 1 : 0;
}

int orkh_device_sync(void) {
    CK(hipDeviceSynchronize(), "hipDeviceSynchronize");
    return 0;
}

int orkh_ptr_is_device(const void *p) {
    if (!p) return 0;
    hipPointerAttribute_t a;
    if (hipPointerGetAttributes(&a, p) != hipSuccess) {
        (void)hipGetLastError();  // plain host memory reports an error here; clear it
        return 0;
    }
    return a.type == hipMemoryTypeDevice || a.type == hipMemoryTypeManaged;
}

}  // extern "C"
