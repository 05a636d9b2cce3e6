// k_weightnorm.hip -- forced unit-norm weight normalisation (forward, in place)
// and its backward with the gain gradient.
// Reference maths: src/kernels.cu:255-297 with launchers 330-344.
//
// W is [in, out] row-major and every output column j is normalised over its
// `in` rows.  One 1024-thread workgroup owns kCols = 16 whole columns: a wave
// instruction covers 4 rows x 16 columns (64-byte row segments), lane (r, c)
// walks rows 4 w + r, + 64, ... of column 16 b + c with eight rows' loads in
// flight; its partial, the 4 row lanes of the wave and then the 16 waves are
// added in a fixed order.  Each column total therefore has a fixed order and
// needs no scratch or second pass; a [1152, 128] weight spreads over 8 CUs.
//   forward : column sum of squares, then W *= rsqrt(sum + eps)    (one launch;
//             the second read of W comes from cache)
//   backward: dot_j = <Wn_j, gW_j>, then gW = gain * (gW - dot_j Wn) (one
//             launch), and *g_gain += sum_j dot_j in a fixed order: with a
//             lent workspace the last workgroup to finish adds the
//             per-workgroup sums; otherwise a one-wave launch does (the
//             reference adds each column with atomicAdd).
#include "nnk_common.h"

namespace {

using namespace nnk;

constexpr int kTpb = 1024;
constexpr int kNw = kTpb / kWave;
constexpr int kCols = 16;              // columns per workgroup
constexpr int kRowsPerWave = kWave / kCols;
constexpr int kRowStep = kNw * kRowsPerWave;
constexpr int kBatch = 8;

// Total of A .* B over all rows of this lane's column (identical on the
// kRowsPerWave lanes of the column in every wave).  `l` is [kNw][kCols].
__device__ __forceinline__ float column_dot(const float* __restrict__ A, const float* __restrict__ B,
    int in, int out, float (*l)[kCols]) {
    const int lane = threadIdx.x & (kWave - 1);
    const int wid = threadIdx.x / kWave;
    const int c = lane % kCols, r = lane / kCols;
    const int j = blockIdx.x * kCols + c;
    float s = 0.0f;
    if (j < out) {
        int i = wid * kRowsPerWave + r;
        for (; i + (kBatch - 1) * kRowStep < in; i += kBatch * kRowStep) {
            float a[kBatch], b[kBatch];
#pragma unroll
            for (int u = 0; u < kBatch; ++u) {
                a[u] = A[(size_t)(i + u * kRowStep) * out + j];
                b[u] = B[(size_t)(i + u * kRowStep) * out + j];
            }
#pragma unroll
            for (int u = 0; u < kBatch; ++u) s += a[u] * b[u];
        }
        for (; i < in; i += kRowStep) s += A[(size_t)i * out + j] * B[(size_t)i * out + j];
    }
#pragma unroll
    for (int o = kCols; o < kWave; o <<= 1) s += __shfl_xor(s, o, kWave);
    if (r == 0) l[wid][c] = s;
    __syncthreads();
    float t = l[0][c];
#pragma unroll
    for (int w = 1; w < kNw; ++w) t += l[w][c];
    return t;
}

__global__ __launch_bounds__(kTpb) void wn_forward(float* __restrict__ W, int in, int out, float eps) {
    __shared__ float l[kNw][kCols];
    const int lane = threadIdx.x & (kWave - 1);
    const int wid = threadIdx.x / kWave;
    const int j = blockIdx.x * kCols + lane % kCols;
    const float inv = rsqrtf(column_dot(W, W, in, out, l) + eps);
    if (j >= out) return;
    for (int i = wid * kRowsPerWave + lane / kCols; i < in; i += kRowStep) W[(size_t)i * out + j] *= inv;
}

// gW = gain * (gW - dot_j * Wn); part[blockIdx.x] = sum of this block's dot_j.
// LAST: the last workgroup to arrive (counter) adds part[0..gridDim.x) to
// *g_gain in index order and re-arms the counter.
template <bool LAST>
__global__ __launch_bounds__(kTpb) void wn_backward(float* __restrict__ gW, const float* __restrict__ Wn,
    const float* __restrict__ gain, float* __restrict__ part, unsigned* __restrict__ counter,
    float* __restrict__ g_gain, int in, int out) {
    __shared__ float l[kNw][kCols];
    __shared__ int last;
    const int lane = threadIdx.x & (kWave - 1);
    const int wid = threadIdx.x / kWave;
    const int j = blockIdx.x * kCols + lane % kCols;
    const float dot = column_dot(Wn, gW, in, out, l);  // its barrier orders every read of gW before the writes below
    if (wid == 0) {
        // lanes 0..kCols-1 hold the block's column totals (r == 0 lanes)
        const float t = wave_sum(lane < kCols && j < out ? dot : 0.0f);
        if (lane == 0) part[blockIdx.x] = t;
    }
    if constexpr (LAST) {
        __syncthreads();
        if (threadIdx.x == 0) {
            __threadfence();  // this block's part is visible before it is counted
            last = atomicAdd(counter, 1u) == gridDim.x - 1;
        }
        __syncthreads();
        if (last && wid == 0) {
            __threadfence();  // every counted block's part is visible here
            float t = 0.0f;
            for (int k = lane; k < (int)gridDim.x; k += kWave) t += part[k];
            t = wave_sum(t);
            if (lane == 0) {
                g_gain[0] = g_gain[0] + t;
                *counter = 0u;
            }
        }
    }
    if (j >= out) return;
    const float g = gain[0];
    for (int i = wid * kRowsPerWave + lane / kCols; i < in; i += kRowStep) {
        const size_t o = (size_t)i * out + j;
        gW[o] = g * (gW[o] - dot * Wn[o]);
    }
}

// *g_gain += part[0] + part[1] + ... (one wave, fixed order).
__global__ __launch_bounds__(kWave) void wn_gain_sum(float* __restrict__ g_gain, const float* __restrict__ part,
    int n) {
    float t = 0.0f;
    for (int k = threadIdx.x; k < n; k += kWave) t += part[k];
    t = wave_sum(t);
    if (threadIdx.x == 0) g_gain[0] = g_gain[0] + t;
}

int wn_blocks(int out) { return (out + kCols - 1) / kCols; }

bool wn_backward_args(const char* what, float* gW, const float* Wn, const float* gain, float* g_gain, int in,
    int out) {
    NNK_REQUIRE_RET(in >= 0 && out >= 0, false, what, "%s: bad shape in=%d out=%d", what, in, out);
    if (out == 0) return false;
    NNK_REQUIRE_RET(gW && Wn && gain && g_gain, false, what, "%s: null pointer", what);
    return true;
}

}  // namespace

extern "C" {

void launch_weight_normalize(float* W, int in, int out, float eps, hipStream_t s) {
    const char* what = "launch_weight_normalize";
    NNK_REQUIRE(in >= 0 && out >= 0, what, "%s: bad shape in=%d out=%d", what, in, out);
    if (in == 0 || out == 0) return;
    NNK_REQUIRE(W, what, "%s: null pointer", what);
    wn_forward<<<dim3((unsigned)wn_blocks(out)), kTpb, 0, s>>>(W, in, out, eps);
    nnk_after_launch(what, s);
}

void launch_weight_normalize_backward(float* gW, const float* Wn, const float* gain,
    float* g_gain, int in, int out, hipStream_t s) {
    const char* what = "launch_weight_normalize_backward";
    if (!wn_backward_args(what, gW, Wn, gain, g_gain, in, out)) return;
    const int blocks = wn_blocks(out);
    float* part = nnk_scratch_acquire((size_t)blocks, s, what);
    if (!part) return;
    wn_backward<false><<<dim3((unsigned)blocks), kTpb, 0, s>>>(gW, Wn, gain, part, nullptr, g_gain, in, out);
    wn_gain_sum<<<dim3(1), kWave, 0, s>>>(g_gain, part, blocks);
    nnk_scratch_release(part, s);
    nnk_after_launch(what, s);
}

size_t nnhip_weight_normalize_backward_workspace(int out) {
    return out > 0 ? (size_t)64 + (size_t)wn_blocks(out) : 0;
}

void launch_weight_normalize_backward_ws(float* gW, const float* Wn, const float* gain, float* g_gain,
    int in, int out, float* workspace, hipStream_t s) {
    const char* what = "launch_weight_normalize_backward_ws";
    if (!wn_backward_args(what, gW, Wn, gain, g_gain, in, out)) return;
    NNK_REQUIRE(workspace, what, "%s: null workspace", what);
    unsigned* counter = reinterpret_cast<unsigned*>(workspace);
    wn_backward<true><<<dim3((unsigned)wn_blocks(out)), kTpb, 0, s>>>(gW, Wn, gain, workspace + 64, counter,
        g_gain, in, out);
    nnk_after_launch(what, s);
}

}  // extern "C"
