// k_weightnorm.hip -- forced unit-norm weight normalisation (forward, in place)
// and its backward with the gain gradient.
// Reference maths: src/kernels.cu:255-297 with launchers 330-344.
//
// W is [in, out] row-major and every output column j is normalised over its
// `in` rows.  Lanes walk 64 consecutive columns (coalesced 256-byte rows),
// waves and workgroups split the rows; per-chunk column partials go to a
// small scratch and are summed in a fixed order (ascending chunk), so the
// result does not depend on scheduling.  Two launches each way:
//   forward : partial sum of squares -> scale     (R W twice, W W once)
//   backward: partial <Wn_j, gW_j>    -> project   (R Wn, gW twice, W gW once)
// The gain gradient is sum_j dot_j added to *g_gain by one workgroup (fixed
// order) instead of the reference's per-column atomicAdd.
#include "nnk_common.h"

namespace {

using namespace nnk;

constexpr int kTpb = 256;
constexpr int kNw = kTpb / kWave;
constexpr int kRowsPerChunk = 64;

__global__ __launch_bounds__(kTpb) void wn_partial(float* __restrict__ part,
    const float* __restrict__ A, const float* __restrict__ B, int in, int out) {
    // part[chunk*out + j] = sum over the chunk's rows of A[i,j]*B[i,j]
    __shared__ float l[kNw][kWave];
    const int lane = threadIdx.x & (kWave - 1);
    const int wid = threadIdx.x / kWave;
    const int j = blockIdx.x * kWave + lane;
    const int r0 = blockIdx.y * kRowsPerChunk;
    const int r1 = min(in, r0 + kRowsPerChunk);
    float s = 0.0f;
    if (j < out)
        for (int i = r0 + wid; i < r1; i += kNw) s += A[(size_t)i * out + j] * B[(size_t)i * out + j];
    l[wid][lane] = s;
    __syncthreads();
    if (wid == 0 && j < out)
        part[(size_t)blockIdx.y * out + j] = ((l[0][lane] + l[1][lane]) + l[2][lane]) + l[3][lane];
}

__device__ __forceinline__ float column_total(const float* __restrict__ part, int chunks, int out, int j) {
    float s = 0.0f;
    for (int c = 0; c < chunks; ++c) s += part[(size_t)c * out + j];
    return s;
}

__global__ __launch_bounds__(kTpb) void wn_scale(float* __restrict__ W,
    const float* __restrict__ part, int chunks, int in, int out, float eps) {
    const int lane = threadIdx.x & (kWave - 1);
    const int wid = threadIdx.x / kWave;
    const int j = blockIdx.x * kWave + lane;
    if (j >= out) return;
    const float inv = rsqrtf(column_total(part, chunks, out, j) + eps);
    const int r0 = blockIdx.y * kRowsPerChunk;
    const int r1 = min(in, r0 + kRowsPerChunk);
    for (int i = r0 + wid; i < r1; i += kNw) W[(size_t)i * out + j] *= inv;
}

__global__ __launch_bounds__(kTpb) void wn_project(float* __restrict__ gW,
    const float* __restrict__ Wn, const float* __restrict__ gain, float* __restrict__ g_gain,
    const float* __restrict__ part, int chunks, int in, int out) {
    const int lane = threadIdx.x & (kWave - 1);
    const int wid = threadIdx.x / kWave;
    if (blockIdx.x == 0 && blockIdx.y == 0 && wid == 0) {
        // gain gradient: sum of all column dots, fixed order
        float t = 0.0f;
        for (int jj = lane; jj < out; jj += kWave) t += column_total(part, chunks, out, jj);
        t = wave_sum(t);
        if (lane == 0) g_gain[0] = g_gain[0] + t;
    }
    const int j = blockIdx.x * kWave + lane;
    if (j >= out) return;
    const float dot = column_total(part, chunks, out, j);
    const float g = gain[0];
    const int r0 = blockIdx.y * kRowsPerChunk;
    const int r1 = min(in, r0 + kRowsPerChunk);
    for (int i = r0 + wid; i < r1; i += kNw) {
        const size_t o = (size_t)i * out + j;
        gW[o] = g * (gW[o] - dot * Wn[o]);
    }
}

}  // namespace

extern "C" {

void launch_weight_normalize(float* W, int in, int out, float eps, hipStream_t s) {
    const char* what = "launch_weight_normalize";
    NNK_REQUIRE(in >= 0 && out >= 0, what, "%s: bad shape in=%d out=%d", what, in, out);
    if (in == 0 || out == 0) return;
    NNK_REQUIRE(W, what, "%s: null pointer", what);
    const int chunks = (in + kRowsPerChunk - 1) / kRowsPerChunk;
    float* part = nnk_scratch_acquire((size_t)chunks * out, s, what);
    if (!part) return;
    const dim3 grid((unsigned)((out + kWave - 1) / kWave), (unsigned)chunks);
    wn_partial<<<grid, kTpb, 0, s>>>(part, W, W, in, out);
    wn_scale<<<grid, kTpb, 0, s>>>(W, part, chunks, in, out, eps);
    nnk_scratch_release(part, s);
    nnk_after_launch(what, s);
}

void launch_weight_normalize_backward(float* gW, const float* Wn, const float* gain,
    float* g_gain, int in, int out, hipStream_t s) {
    const char* what = "launch_weight_normalize_backward";
    NNK_REQUIRE(in >= 0 && out >= 0, what, "%s: bad shape in=%d out=%d", what, in, out);
    if (out == 0) return;
    NNK_REQUIRE(gW && Wn && gain && g_gain, what, "%s: null pointer", what);
    const int chunks = in > 0 ? (in + kRowsPerChunk - 1) / kRowsPerChunk : 1;
    float* part = nnk_scratch_acquire((size_t)chunks * out, s, what);
    if (!part) return;
    const dim3 grid((unsigned)((out + kWave - 1) / kWave), (unsigned)chunks);
    wn_partial<<<grid, kTpb, 0, s>>>(part, Wn, gW, in, out);
    wn_project<<<grid, kTpb, 0, s>>>(gW, Wn, gain, g_gain, part, chunks, in, out);
    nnk_scratch_release(part, s);
    nnk_after_launch(what, s);
}

}  // extern "C"
