// rt.hip -- launch-layer error record, stream-ordered scratch and the runtime
// plumbing of nn_hip_rt.h.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>
#include <mutex>
#include <vector>

#include "nn_hip_rt.h"
#include "nnk_common.h"

namespace {

struct ErrorRecord {
    int code = 0;
    char msg[512] = {0};
};

thread_local ErrorRecord g_err;

bool check_mode() {
    static const bool on = [] {  // read once (thread-safe static initialisation)
        const char* e = getenv("NNHIP_CHECK");
        return e && e[0] == '1';
    }();
    return on;
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
    static const bool verbose = [] {
        const char* e = getenv("NNHIP_VERBOSE");
        return e && e[0] == '1';
    }();
    if (!verbose) return;
    va_list ap;
    va_start(ap, fmt);
    fputs("nnhip: ", stderr);
    vfprintf(stderr, fmt, ap);
    fputc('\n', stderr);
    va_end(ap);
}

bool nnk_capturing(hipStream_t s) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    return s && hipStreamIsCapturing(s, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
}

int nnk_device_cus(hipStream_t s) {
    constexpr int kDev = 16;
    static std::atomic<int> cus_of[kDev];  // 0 = not yet queried (relaxed: racing callers store the same value)
    int dev = -1;
    if ((s ? hipStreamGetDevice(s, &dev) : hipGetDevice(&dev)) != hipSuccess || dev < 0 || dev >= kDev) {
        (void)hipGetLastError();
        return 0;
    }
    int n = cus_of[dev].load(std::memory_order_relaxed);
    if (n == 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) {
            (void)hipGetLastError();
            return 0;
        }
        cus_of[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

// Allocations the launch layer makes by itself (the scratch pools, their
// blocks and the wait flag below), counted for tests of the allocation-free
// entry points.  Explicit requests (nnhip_malloc, multi-tensor plans, module
// arenas) are not counted.
namespace {
unsigned long long g_hidden_allocs = 0;  // updated under a lock or at load
}

// The process-wide word that a streaming kernel's bounded wait sets when it
// gives up: host memory mapped into the device's address space (coherent, so
// the kernel's system-scope store is visible to the host once it is done).
// It is allocated once, when the library is loaded, and kept until the
// process ends, so that no launcher allocates it (the allocation-free entry
// point included).  Without a device at load time it stays absent and wait
// failures are reported through the workspace's own word only.
namespace {
unsigned* g_wait_flag_host = nullptr;
unsigned* g_wait_flag_dev = nullptr;

__attribute__((constructor)) void create_wait_flag() {
    void* p = nullptr;
    void* d = nullptr;
    if (hipHostMalloc(&p, 64, hipHostMallocMapped | hipHostMallocCoherent) != hipSuccess || !p ||
        hipHostGetDevicePointer(&d, p, 0) != hipSuccess || !d) {
        (void)hipGetLastError();
        if (p) (void)hipHostFree(p);
        return;
    }
    memset(p, 0, 64);
    ++g_hidden_allocs;
    g_wait_flag_dev = static_cast<unsigned*>(d);
    __atomic_store_n(&g_wait_flag_host, static_cast<unsigned*>(p), __ATOMIC_RELEASE);
}

// Move a wait failure the device has flagged into the error record.
void take_wait_flag() {
    unsigned* h = __atomic_load_n(&g_wait_flag_host, __ATOMIC_ACQUIRE);
    if (!h || __atomic_load_n(h, __ATOMIC_ACQUIRE) == 0) return;
    __atomic_store_n(h, 0u, __ATOMIC_RELAXED);
    nnk_set_error((int)hipErrorLaunchTimeOut,
        "streaming GroupNorm: a statistics wait ran out of polls; the outputs of that launch are invalid");
}
}  // namespace

unsigned* nnk_wait_flag() { return g_wait_flag_dev; }

void nnk_after_launch(const char* what, hipStream_t s) {
    hipError_t e = hipGetLastError();
    const bool sync = e == hipSuccess && check_mode() && !nnk_capturing(s);
    if (sync) e = hipStreamSynchronize(s);
    if (e != hipSuccess) nnk_set_error((int)e, "%s: %s", what, hipGetErrorString(e));
    else if (sync) take_wait_flag();
}

// Scratch for launchers whose reference signature has no workspace argument.
// Each (device, stream) keeps one cached block: work on one stream runs in
// order, so the next launch on the stream may reuse the block the previous
// one used.  A larger request replaces the block (the old one is freed in
// stream order, after its last use); a request that finds the stream's block
// in use (another host thread on the same stream) takes a block of its own.
// Blocks come from a memory pool the library owns, one per device, whose
// release threshold keeps freed memory cached; the process's default pool is
// left as it is.  Cached blocks are held until the process ends.
//
// Under stream capture a launcher may only take the stream's cached block as
// it is (the graph keeps its address): a capture that would need a new or
// larger block is refused with an error, so run the sequence once eagerly
// before capturing it.  A block that a capture has used is never freed: when
// the slot later grows or its stream is dropped, the old block is retired
// (kept until the process ends) because graphs may still replay on it.
namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
hipMemPool_t g_pools[kMaxDevices] = {};

struct Slot {
    int dev;
    hipStream_t stream;
    void* p;
    size_t bytes;
    bool busy;
    bool captured;  // a captured graph refers to p
};
Slot g_slots[256];
int g_nslots = 0;
std::vector<void*> g_retired;  // blocks graphs may still use

// Caller holds g_scratch_mu.  Give up slot's block: free it in stream order,
// or retire it if a captured graph refers to it.
void drop_block(Slot& slot) {
    if (!slot.p) return;
    if (slot.captured) g_retired.push_back(slot.p);
    else (void)hipFreeAsync(slot.p, slot.stream);
    slot.p = nullptr;
    slot.bytes = 0;
    slot.captured = false;
}

// Caller holds g_scratch_mu.
hipMemPool_t scratch_pool(int dev, const char* what) {
    if (!g_pools[dev]) {
        hipMemPoolProps props = {};
        props.allocType = hipMemAllocationTypePinned;
        props.location.type = hipMemLocationTypeDevice;
        props.location.id = dev;
        hipMemPool_t pool = nullptr;
        hipError_t e = hipMemPoolCreate(&pool, &props);
        if (e == hipSuccess) {
            ++g_hidden_allocs;
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

void* pool_alloc(hipMemPool_t pool, size_t bytes, hipStream_t s, const char* what) {
    void* p = nullptr;
    const hipError_t e = hipMallocFromPoolAsync(&p, bytes, pool, s);
    if (e != hipSuccess) {
        nnk_set_error((int)e, "%s: scratch of %zu bytes: %s", what, bytes, hipGetErrorString(e));
        return nullptr;
    }
    ++g_hidden_allocs;  // callers hold g_scratch_mu
    return p;
}
}  // namespace

float* nnk_scratch_acquire(size_t n_floats, hipStream_t s, const char* what) {
    int dev = -1;
    const hipError_t ed = s ? hipStreamGetDevice(s, &dev) : hipGetDevice(&dev);
    if (ed != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        nnk_set_error(ed != hipSuccess ? (int)ed : (int)hipErrorInvalidDevice, "%s: no device for the stream", what);
        return nullptr;
    }
    size_t need = n_floats * sizeof(float) + 256;
    const bool capturing = nnk_capturing(s);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    hipMemPool_t pool = scratch_pool(dev, what);
    if (!pool) return nullptr;
    Slot* slot = nullptr;
    for (int i = 0; i < g_nslots; ++i)
        if (g_slots[i].dev == dev && g_slots[i].stream == s) slot = &g_slots[i];
    if (!slot && g_nslots < (int)(sizeof g_slots / sizeof g_slots[0])) {
        slot = &g_slots[g_nslots++];
        *slot = Slot{dev, s, nullptr, 0, false, false};
    }
    if (capturing && (!slot || slot->busy || slot->bytes < need)) {
        nnk_set_error((int)hipErrorStreamCaptureUnsupported,
            "%s: scratch of %zu bytes is not cached for the capturing stream (run the sequence once before "
            "capturing it)", what, need);
        return nullptr;
    }
    if (!slot || slot->busy) return static_cast<float*>(pool_alloc(pool, need, s, what));
    if (slot->bytes < need) {
        size_t bytes = 1 << 16;
        while (bytes < need) bytes <<= 1;
        void* p = pool_alloc(pool, bytes, s, what);
        if (!p) return nullptr;
        drop_block(*slot);
        slot->p = p;
        slot->bytes = bytes;
    }
    if (capturing) slot->captured = true;
    slot->busy = true;
    return static_cast<float*>(slot->p);
}

// Drop stream s's cached block (freed in stream order).  Called before the
// stream goes away: a later stream could otherwise be handed the same handle
// value, find the slot and use the block while the old stream's work on it is
// still pending.
void nnk_scratch_forget_stream(hipStream_t s) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    for (int i = 0; i < g_nslots; ++i) {
        if (g_slots[i].stream != s) continue;
        drop_block(g_slots[i]);
        g_slots[i] = g_slots[--g_nslots];
        --i;
    }
}

void nnk_scratch_release(float* p, hipStream_t s) {
    if (!p) return;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    for (int i = 0; i < g_nslots; ++i) {
        if (g_slots[i].p == p && g_slots[i].stream == s && g_slots[i].busy) {
            g_slots[i].busy = false;
            return;
        }
    }
    (void)hipFreeAsync(p, s);  // a block of its own
}

__global__ __launch_bounds__(256) void fill_f32_kernel(float* __restrict__ p, float value, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        p[i] = value;
}

// ---------------------------------------------------------------------------
// Calibration copy for the HBM byte counters: a plain streaming copy, four
// float4 per thread.  What the counters read per byte moved does not depend
// on the access pattern, only that every byte is read and written once.
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
    if (g_err.code == 0) take_wait_flag();
    const int code = g_err.code;
    if (buf && buflen > 0) {
        strncpy(buf, g_err.msg, (size_t)buflen - 1);
        buf[buflen - 1] = '\0';
    }
    g_err.code = 0;
    g_err.msg[0] = '\0';
    return code;
}

unsigned long long nnhip_launch_allocations(void) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    return g_hidden_allocs;
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

int nnhip_stream_destroy(hipStream_t s) {
    if (s) nnk_scratch_forget_stream(s);
    return (int)hipStreamDestroy(s);
}

void nnhip_stream_scratch_release(hipStream_t s) { nnk_scratch_forget_stream(s); }
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

int nnhip_graph_capture_begin(hipStream_t s) {
    if (!s) return (int)hipErrorInvalidValue;
    return (int)hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal);
}

hipGraphExec_t nnhip_graph_capture_end(hipStream_t s) {
    hipGraph_t g = nullptr;
    if (!s || hipStreamEndCapture(s, &g) != hipSuccess || !g) return nullptr;
    hipGraphExec_t e = nullptr;
    const hipError_t r = hipGraphInstantiate(&e, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    return r == hipSuccess ? e : nullptr;
}

int nnhip_graph_launch(hipGraphExec_t g, hipStream_t s) { return (int)hipGraphLaunch(g, s); }
int nnhip_graph_destroy(hipGraphExec_t g) { return (int)hipGraphExecDestroy(g); }

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
