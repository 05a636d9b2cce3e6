// rt.hip -- launch-layer error record, stream-ordered scratch and the runtime
// plumbing of nn_hip_rt.h.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <mutex>

#include "nn_hip_rt.h"
#include "nnk_common.h"

namespace {

struct ErrorRecord {
    int code = 0;
    char msg[512] = {0};
};

thread_local ErrorRecord g_err;

bool check_mode() {
    static int mode = -1;
    if (mode < 0) {
        const char* e = getenv("NNHIP_CHECK");
        mode = (e && e[0] == '1') ? 1 : 0;
    }
    return mode == 1;
}

}  // namespace

void nnk_set_error(int code, const char* fmt, ...) {
    if (g_err.code == 0) {
        g_err.code = code ? code : (int)hipErrorUnknown;
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(g_err.msg, sizeof g_err.msg, fmt, ap);
        va_end(ap);
    }
    if (check_mode()) {
        fprintf(stderr, "nnhip: %s\n", g_err.msg);
        abort();
    }
}

// NNHIP_VERBOSE=1: report on stderr why a launcher left its fast path.
void nnk_path_note(const char* fmt, ...) {
    static int verbose = -1;
    if (verbose < 0) {
        const char* e = getenv("NNHIP_VERBOSE");
        verbose = (e && e[0] == '1') ? 1 : 0;
    }
    if (!verbose) return;
    va_list ap;
    va_start(ap, fmt);
    fputs("nnhip: ", stderr);
    vfprintf(stderr, fmt, ap);
    fputc('\n', stderr);
    va_end(ap);
}

void nnk_after_launch(const char* what, hipStream_t s) {
    hipError_t e = hipGetLastError();
    if (e == hipSuccess && check_mode()) e = hipStreamSynchronize(s);
    if (e != hipSuccess) nnk_set_error((int)e, "%s: %s", what, hipGetErrorString(e));
}

// The launchers' stream-ordered scratch comes from a memory pool the library
// owns, one per device, whose release threshold keeps freed blocks cached:
// with the default threshold (0) every free hands the memory back at the next
// synchronisation and the next allocation maps it again, which costs more
// than the small kernels that use it.  The process's default pool is left as
// it is.
namespace {
constexpr int kMaxDevices = 64;
std::mutex g_pool_mu;
hipMemPool_t g_pools[kMaxDevices] = {};

hipMemPool_t scratch_pool(hipStream_t s, const char* what) {
    int dev = -1;
    hipError_t e = s ? hipStreamGetDevice(s, &dev) : hipGetDevice(&dev);
    if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        nnk_set_error(e != hipSuccess ? (int)e : (int)hipErrorInvalidDevice, "%s: no device for the stream", what);
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_pool_mu);
    if (!g_pools[dev]) {
        hipMemPoolProps props = {};
        props.allocType = hipMemAllocationTypePinned;
        props.location.type = hipMemLocationTypeDevice;
        props.location.id = dev;
        hipMemPool_t pool = nullptr;
        e = hipMemPoolCreate(&pool, &props);
        if (e == hipSuccess) {
            uint64_t keep = UINT64_MAX;
            e = hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &keep);
            if (e != hipSuccess) (void)hipMemPoolDestroy(pool);
        }
        if (e != hipSuccess) {
            nnk_set_error((int)e, "%s: scratch pool on device %d: %s", what, dev, hipGetErrorString(e));
            return nullptr;
        }
        g_pools[dev] = pool;
    }
    return g_pools[dev];
}
}  // namespace

float* nnk_scratch_acquire(size_t n_floats, hipStream_t s, const char* what) {
    hipMemPool_t pool = scratch_pool(s, what);
    if (!pool) return nullptr;
    void* p = nullptr;
    hipError_t e = hipMallocFromPoolAsync(&p, n_floats * sizeof(float) + 256, pool, s);
    if (e != hipSuccess) {
        nnk_set_error((int)e, "%s: scratch of %zu floats: %s", what, n_floats, hipGetErrorString(e));
        return nullptr;
    }
    return static_cast<float*>(p);
}

void nnk_scratch_release(float* p, hipStream_t s) {
    if (p) (void)hipFreeAsync(p, s);
}

__global__ __launch_bounds__(256) void fill_f32_kernel(float* __restrict__ p, float value, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        p[i] = value;
}

// ---------------------------------------------------------------------------
// Calibration copy: the same 4 x float4 per thread access pattern as the
// streaming elementwise kernels.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void copy_f32_kernel(float* __restrict__ dst,
    const float* __restrict__ src, long long n4, long long n) {
    const long long base = (long long)blockIdx.x * 1024 + threadIdx.x;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const long long q = base + u * 256;
        if (q < n4) nnk::st4(dst + 4 * q, nnk::ld4(src + 4 * q));
    }
    if (blockIdx.x == 0 && threadIdx.x < (n - 4 * n4)) {
        const long long i = 4 * n4 + threadIdx.x;
        dst[i] = src[i];
    }
}

extern "C" {

int nnhip_get_last_error(char* buf, int buflen) {
    const int code = g_err.code;
    if (buf && buflen > 0) {
        strncpy(buf, g_err.msg, (size_t)buflen - 1);
        buf[buflen - 1] = '\0';
    }
    g_err.code = 0;
    g_err.msg[0] = '\0';
    return code;
}

int nnhip_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

int nnhip_set_device(int dev) { return (int)hipSetDevice(dev); }

int nnhip_device_info(char* buf, int buflen) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, dev);
    if (e != hipSuccess) return (int)e;
    snprintf(buf, (size_t)buflen, "%s|%s|%d|%zu", prop.name, prop.gcnArchName,
        prop.multiProcessorCount, (size_t)prop.totalGlobalMem);
    return 0;
}

void* nnhip_malloc(size_t bytes) {
    void* p = nullptr;
    if (hipMalloc(&p, bytes ? bytes : 1) != hipSuccess) return nullptr;
    return p;
}

int nnhip_free(void* p) { return (int)hipFree(p); }

int nnhip_memcpy_htod(void* dst, const void* src, size_t bytes) {
    return (int)hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice);
}

int nnhip_memcpy_dtoh(void* dst, const void* src, size_t bytes) {
    return (int)hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost);
}

int nnhip_memcpy_dtod(void* dst, const void* src, size_t bytes) {
    return (int)hipMemcpy(dst, src, bytes, hipMemcpyDeviceToDevice);
}

int nnhip_memset(void* dst, int value, size_t bytes) { return (int)hipMemset(dst, value, bytes); }

int nnhip_memset_async(void* dst, int value, size_t bytes, hipStream_t s) {
    return (int)hipMemsetAsync(dst, value, bytes, s);
}

int nnhip_device_synchronize(void) { return (int)hipDeviceSynchronize(); }

hipStream_t nnhip_stream_create(void) {
    hipStream_t s = nullptr;
    if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess) return nullptr;
    return s;
}

int nnhip_stream_destroy(hipStream_t s) { return (int)hipStreamDestroy(s); }
int nnhip_stream_synchronize(hipStream_t s) { return (int)hipStreamSynchronize(s); }

hipEvent_t nnhip_event_create(void) {
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

int nnhip_event_destroy(hipEvent_t e) { return (int)hipEventDestroy(e); }
int nnhip_event_record(hipEvent_t e, hipStream_t s) { return (int)hipEventRecord(e, s); }
int nnhip_event_synchronize(hipEvent_t e) { return (int)hipEventSynchronize(e); }

float nnhip_event_elapsed_ms(hipEvent_t start, hipEvent_t stop) {
    float ms = -1.0f;
    if (hipEventElapsedTime(&ms, start, stop) != hipSuccess) return -1.0f;
    return ms;
}

void nnhip_fill_f32(float* p, float value, size_t n, hipStream_t s) {
    if (n == 0) return;
    NNK_REQUIRE(p, "fill", "nnhip_fill_f32: null pointer");
    const size_t blocks = (n + 255) / 256 < 4096 ? (n + 255) / 256 : 4096;
    fill_f32_kernel<<<dim3((unsigned)blocks), dim3(256), 0, s>>>(p, value, n);
    nnk_after_launch("nnhip_fill_f32", s);
}

void nnhip_copy_f32(float* dst, const float* src, size_t n, hipStream_t s) {
    if (n == 0) return;
    NNK_REQUIRE(nnk::aligned16(dst) && nnk::aligned16(src), "copy", "nnhip_copy_f32: pointers must be 16-byte aligned");
    const long long n4 = (long long)(n / 4);
    const long long blocks = (n4 + 1023) / 1024 > 0 ? (n4 + 1023) / 1024 : 1;
    copy_f32_kernel<<<dim3((unsigned)blocks), dim3(256), 0, s>>>(dst, src, n4, (long long)n);
    nnk_after_launch("nnhip_copy_f32", s);
}

}  // extern "C"
