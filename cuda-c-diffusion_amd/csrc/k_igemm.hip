// k_igemm.hip -- NHWC convolution forward as an implicit GEMM on the fp32
// matrix cores (v_mfma_f32_32x32x2f32), replacing im2col + GEMM + bias/gain
// pass of the reference's conv2d forward (src/conv2d.c:17-34: launch_im2col,
// gemm_forward, launch_add_bias or launch_scale_by_scalar).
//
//   Y[m, n] = sum_k A[m, k] WT[n, k]  (+ bias[n] | * gain[0])
//   m = (b, oh, ow), k = (kh, kw, ci), A[m, k] = X[b, oh s + kh - p, ow s + kw - p, ci]
//   (0 outside the image), WT = the [K*K*C_in, C_out] weight transposed.
//
// The im2col matrix is never written: each workgroup gathers its A tile from X
// directly (a k-slice of 32 channels of one (kh, kw) is 128 contiguous bytes
// of one input pixel).
//
// Workgroup tile 128 (m) x 128 (n), k in slices of 32; 4 waves of 64 x 64,
// each a 2 x 2 grid of 32 x 32 MFMA accumulators (64 registers).  Per slice a
// thread loads 4 float4 of A and 4 of WT into registers, the slice before it
// computes from LDS, then the registers go to the other LDS buffer (two
// buffers of 2 x 16 KB; two workgroups fit a CU).  LDS tiles are [128 rows][8
// float4 chunks] with the chunk index xor-swizzled by the row, so the 128-bit
// fragment reads of a wave (32 rows, one chunk per half-wave) and the tile
// writes are both free of bank conflicts.
//
// Lane layout of v_mfma_f32_32x32x2f32 (checked on the device): lane l supplies
// A[l % 32][l / 32] and B[l / 32][l % 32]; accumulator register r of lane l
// holds D[8 (r / 4) + 4 (l / 32) + r % 4][l % 32].  A 128-bit fragment read
// gives a lane 4 consecutive k of its row; component c feeds the c-th MFMA,
// which pairs k = 4h + c of the two half-waves h: any pairing of k is the same
// sum, as long as A and B use the same one.
//
// Summation order: each output is a fixed-order fp32 sum (per slice, pairs of
// k in MFMA order, slices in k order); it differs from a library GEMM's order
// by rounding only, and is the same on every run.
#include "nnk_common.h"

namespace {

using namespace nnk;

constexpr int kBM = 128, kBN = 128, kBK = 32, kTpb = 256;
typedef float f32x16 __attribute__((ext_vector_type(16)));

struct ConvShape {
    int B, H, W, Cin, Cout, K, stride, pad, Ho, Wo;
    int M;    // B * Ho * Wo
    int KKC;  // K * K * Cin
};

// float4 slot of (row, chunk) in a [128][8] tile.
__device__ __forceinline__ int slot(int row, int chunk) { return row * 8 + (chunk ^ (row & 7)); }

enum { kEpiNone = 0, kEpiBias = 1, kEpiGain = 2 };

template <int EPI>
__global__ __launch_bounds__(kTpb, 2) void igemm_fwd(float* __restrict__ Y, const float* __restrict__ X,
    const float* __restrict__ WT, const float* __restrict__ bias, const float* __restrict__ gain, ConvShape sh) {
    __shared__ float4 As[2][kBM * 8];
    __shared__ float4 Bs[2][kBN * 8];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int wm = w >> 1, wn = w & 1;
    const int m0 = blockIdx.x * kBM, n0 = blockIdx.y * kBN;
    // loader role: chunk ch of rows r0 + 32 q
    const int ch = tid & 7, r0 = tid >> 3;
    int pix[4], ihb[4], iwb[4];
    bool rok[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int m = m0 + r0 + 32 * q;
        rok[q] = m < sh.M;
        const int mm = rok[q] ? m : 0;
        const int ow = mm % sh.Wo, t = mm / sh.Wo;
        const int oh = t % sh.Ho, b = t / sh.Ho;
        pix[q] = b * sh.H * sh.W;
        ihb[q] = oh * sh.stride - sh.pad;
        iwb[q] = ow * sh.stride - sh.pad;
    }
    const float* wrow = WT + (size_t)(n0 + r0) * sh.KKC + ch * 4;
    const size_t wstep = (size_t)32 * sh.KKC;

    float4 ra[4], rb[4];
    auto load = [&](int kt) {
        const int k0 = kt * kBK;
        const int khw = k0 / sh.Cin, ci = k0 - khw * sh.Cin + ch * 4;
        const int kh = khw / sh.K, kw = khw - kh * sh.K;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int ih = ihb[q] + kh, iw = iwb[q] + kw;
            const bool ok = rok[q] && (unsigned)ih < (unsigned)sh.H && (unsigned)iw < (unsigned)sh.W;
            ra[q] = ok ? ld4(X + (size_t)(pix[q] + ih * sh.W + iw) * sh.Cin + ci) : make_float4(0.f, 0.f, 0.f, 0.f);
            rb[q] = ld4(wrow + q * wstep + k0);
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            As[buf][slot(r0 + 32 * q, ch)] = ra[q];
            Bs[buf][slot(r0 + 32 * q, ch)] = rb[q];
        }
    };

    f32x16 acc[2][2];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int u = 0; u < 2; ++u) acc[t][u] = (f32x16){};
    const int nk = sh.KKC / kBK;
    load(0);
    store(0);
    __syncthreads();
    const int fr = lane & 31, fh = lane >> 5;
    for (int kt = 0; kt < nk; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < nk) load(kt + 1);
#pragma unroll
        for (int kq = 0; kq < 4; ++kq) {
            const int c = 2 * kq + fh;
            float4 a[2], b[2];
#pragma unroll
            for (int t = 0; t < 2; ++t) a[t] = As[buf][slot(wm * 64 + 32 * t + fr, c)];
#pragma unroll
            for (int u = 0; u < 2; ++u) b[u] = Bs[buf][slot(wn * 64 + 32 * u + fr, c)];
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int u = 0; u < 2; ++u) acc[t][u] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[t].x, b[u].x, acc[t][u], 0, 0, 0);
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int u = 0; u < 2; ++u) acc[t][u] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[t].y, b[u].y, acc[t][u], 0, 0, 0);
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int u = 0; u < 2; ++u) acc[t][u] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[t].z, b[u].z, acc[t][u], 0, 0, 0);
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int u = 0; u < 2; ++u) acc[t][u] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[t].w, b[u].w, acc[t][u], 0, 0, 0);
        }
        if (kt + 1 < nk) store(buf ^ 1);
        __syncthreads();
    }

    // epilogue: lanes 0-31 and 32-63 each write 32 consecutive outputs of a row
    float g = 1.0f;
    if constexpr (EPI == kEpiGain) g = gain[0];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int n = n0 + wn * 64 + 32 * u + fr;
        float bn = 0.0f;
        if constexpr (EPI == kEpiBias) bn = bias[n];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + wm * 64 + 32 * t + 8 * (r >> 2) + 4 * fh + (r & 3);
                if (m < sh.M) {
                    float v = acc[t][u][r];
                    if constexpr (EPI == kEpiBias) v = v + bn;
                    if constexpr (EPI == kEpiGain) v = v * g;
                    Y[(size_t)m * sh.Cout + n] = v;
                }
            }
        }
    }
}

// out[c][r] = in[r][c] for a row-major [rows, cols] matrix (32 x 32 LDS tiles).
__global__ __launch_bounds__(256) void transpose_kernel(float* __restrict__ out, const float* __restrict__ in,
    int rows, int cols) {
    __shared__ float tile[32][33];
    const int c0 = blockIdx.x * 32, r0 = blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
    for (int k = ty; k < 32; k += 8) {
        const int r = r0 + k, c = c0 + tx;
        if (r < rows && c < cols) tile[k][tx] = in[(size_t)r * cols + c];
    }
    __syncthreads();
    for (int k = ty; k < 32; k += 8) {
        const int c = c0 + k, r = r0 + tx;
        if (r < rows && c < cols) out[(size_t)c * rows + r] = tile[tx][k];
    }
}

}  // namespace

extern "C" {

int nnhip_conv2d_implicit_supported(int C_in, int C_out) {
    return C_in > 0 && C_out > 0 && C_in % kBK == 0 && C_out % kBN == 0;
}

void launch_transpose(float* out, const float* in, int rows, int cols, hipStream_t s) {
    const char* what = "launch_transpose";
    NNK_REQUIRE(rows >= 0 && cols >= 0, what, "%s: bad shape %d x %d", what, rows, cols);
    if ((long long)rows * cols == 0) return;
    NNK_REQUIRE(out && in && out != in, what, "%s: null or aliased pointers", what);
    const dim3 grid((unsigned)((cols + 31) / 32), (unsigned)((rows + 31) / 32));
    transpose_kernel<<<grid, 256, 0, s>>>(out, in, rows, cols);
    nnk_after_launch(what, s);
}

void launch_conv2d_forward_implicit(float* Y, const float* X, const float* WT, const float* bias,
    const float* gain, int batch, int H, int W, int C_in, int C_out, int K, int stride, int pad, int H_out,
    int W_out, hipStream_t s) {
    const char* what = "launch_conv2d_forward_implicit";
    NNK_REQUIRE(batch >= 0 && H > 0 && W > 0 && K > 0 && stride > 0 && pad >= 0, what, "%s: bad geometry", what);
    NNK_REQUIRE(nnhip_conv2d_implicit_supported(C_in, C_out), what,
        "%s: needs C_in %% %d == 0 and C_out %% %d == 0 (C_in=%d C_out=%d)", what, kBK, kBN, C_in, C_out);
    NNK_REQUIRE(H_out == (H + 2 * pad - K) / stride + 1 && W_out == (W + 2 * pad - K) / stride + 1 && H_out > 0 &&
                    W_out > 0,
        what, "%s: output size %dx%d does not match the geometry", what, H_out, W_out);
    NNK_REQUIRE((long long)batch * H * W * C_in < (1LL << 31) && (long long)batch * H_out * W_out * C_out < (1LL << 31),
        what, "%s: tensor exceeds the 32-bit index range", what);
    NNK_REQUIRE(!(bias && gain), what, "%s: bias and gain are exclusive", what);
    if (batch == 0) return;
    NNK_REQUIRE(Y && X && WT, what, "%s: null pointer", what);
    NNK_REQUIRE(aligned16(X) && aligned16(WT), what, "%s: X and WT must be 16-byte aligned", what);
    ConvShape sh{batch, H, W, C_in, C_out, K, stride, pad, H_out, W_out, batch * H_out * W_out, K * K * C_in};
    const dim3 grid((unsigned)((sh.M + kBM - 1) / kBM), (unsigned)(C_out / kBN));
    if (bias) igemm_fwd<kEpiBias><<<grid, kTpb, 0, s>>>(Y, X, WT, bias, nullptr, sh);
    else if (gain) igemm_fwd<kEpiGain><<<grid, kTpb, 0, s>>>(Y, X, WT, nullptr, gain, sh);
    else igemm_fwd<kEpiNone><<<grid, kTpb, 0, s>>>(Y, X, WT, nullptr, nullptr, sh);
    nnk_after_launch(what, s);
}

}  // extern "C"
