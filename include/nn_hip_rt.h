/* nn_hip_rt.h -- runtime plumbing exported beside the launch layer.
 *
 * The reference reaches device memory, copies and streams through the CUDA
 * runtime directly (cudaMalloc in src/nn.h:54-59, cudaMemcpy in the modules).
 * These few wrappers give foreign callers that do not link the HIP runtime
 * themselves (Python via ctypes, the bench harness) the same facilities, plus
 * the error record of the launch layer. They are plumbing, not part of the
 * kernel path. Every function returns 0 on success and a HIP error code
 * otherwise unless stated.
 */
#ifndef NN_HIP_RT_H
#define NN_HIP_RT_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- error record of the launch layer (thread-local) ---- */
/* Returns the first error recorded since the last call (0 = none) and clears
   it; the message is copied into buf when buf != NULL. */
int nnhip_get_last_error(char* buf, int buflen);

/* Number of allocations the launch layer has made by itself since the
   library was loaded: its scratch pools and their blocks (the launchers
   without a workspace argument draw them) and the host-mapped wait flag
   (made once, at load).  Allocations a caller asks for (nnhip_malloc,
   multi-tensor plans, module arenas) are not counted.  For tests of the
   allocation-free entry points. */
unsigned long long nnhip_launch_allocations(void);

/* ---- device ---- */
int nnhip_device_count(void);
int nnhip_set_device(int dev);
/* Writes "<name>|<gcnArchName>|<CUs>|<memory bytes>" into buf. */
int nnhip_device_info(char* buf, int buflen);

/* ---- memory ---- */
void* nnhip_malloc(size_t bytes); /* NULL on failure */
int nnhip_free(void* p);
int nnhip_memcpy_htod(void* dst, const void* src, size_t bytes);
int nnhip_memcpy_dtoh(void* dst, const void* src, size_t bytes);
int nnhip_memcpy_dtod(void* dst, const void* src, size_t bytes);
int nnhip_memset(void* dst, int value, size_t bytes);
int nnhip_memset_async(void* dst, int value, size_t bytes, hipStream_t s);
/* p[i] = value for n floats, by a kernel on stream s (so it is also safe
   inside a captured graph, unlike a memset node).  Errors are recorded in the
   launch layer's error record. */
void nnhip_fill_f32(float* p, float value, size_t n, hipStream_t s);
int nnhip_device_synchronize(void);

/* ---- streams and events ---- */
hipStream_t nnhip_stream_create(void); /* NULL stream on failure */
/* Also drops the launch layer's cached scratch block of s. */
int nnhip_stream_destroy(hipStream_t s);
/* The launchers without a workspace argument keep one scratch block per
   (device, stream) until the process ends.  Call this (it frees the block in
   stream order) before destroying a stream with hipStreamDestroy directly;
   nnhip_stream_destroy does it itself. */
void nnhip_stream_scratch_release(hipStream_t s);
int nnhip_stream_synchronize(hipStream_t s);
hipEvent_t nnhip_event_create(void);
int nnhip_event_destroy(hipEvent_t e);
int nnhip_event_record(hipEvent_t e, hipStream_t s);
int nnhip_event_synchronize(hipEvent_t e);
float nnhip_event_elapsed_ms(hipEvent_t start, hipEvent_t stop); /* < 0 on error */

/* ---- graphs ---- */
/* Capture the work issued to stream s (not the null stream) from this thread
   into a graph, then instantiate it: begin, issue launchers, end.  The
   launchers with a lent workspace issue kernels only (no memset, no
   allocation), so their sequences can be captured; the streaming GroupNorm
   keeps its launch tag in the workspace and advances it on the device, so
   each replay of a captured launch gets a tag of its own.  end returns NULL
   on failure. */
int nnhip_graph_capture_begin(hipStream_t s);
hipGraphExec_t nnhip_graph_capture_end(hipStream_t s);
int nnhip_graph_launch(hipGraphExec_t g, hipStream_t s);
int nnhip_graph_destroy(hipGraphExec_t g);

/* ---- host generator for weight initialisation ----
   The reference draws initial weights from a cuRAND generator held in its
   Context (src/nn.h:73, the fill at src/nn.h:117-135).  A caller that keeps
   the reference's host code holds one of these instead: xoshiro256**
   (Blackman and Vigna) seeded through SplitMix64, draws made on the host and
   copied into device memory with a synchronous copy (so a constructor may
   use the buffer at once, as after the reference's fill).  The library's own
   Context (nn_modules.h) carries the same generator. */
typedef struct {
    uint64_t s[4];
} NnHostRng;
void nnhip_rng_seed(NnHostRng* g, uint64_t seed);
/* dst[i] = mean + std * z_i with z_i ~ N(0, 1) (Box-Muller in double) for n
   floats of device memory.  Returns 0 or the HIP error of the copy. */
int nnhip_fill_normal(NnHostRng* g, float* dst, size_t n, float mean, float std);
/* dst[i] ~ U[0, 1) from the top 24 bits of one draw each.  Returns 0 or the
   HIP error of the copy. */
int nnhip_fill_uniform(NnHostRng* g, float* dst, size_t n);

/* ---- calibration ---- */
/* dst[i] = src[i] for n floats with the same 128-bit vector access pattern
   as the path's streaming kernels; used to scale HBM counters. */
void nnhip_copy_f32(float* dst, const float* src, size_t n, hipStream_t s);

#ifdef __cplusplus
}
#endif

#endif /* NN_HIP_RT_H */
