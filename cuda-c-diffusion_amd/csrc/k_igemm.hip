// k_igemm.hip -- NHWC convolution forward as an implicit GEMM on the fp32
// matrix cores (v_mfma_f32_32x32x2f32), replacing im2col + GEMM + bias/gain
// pass of the reference's conv2d forward (src/conv2d.c:17-34: launch_im2col,
// gemm_forward, launch_add_bias or launch_scale_by_scalar), and the stride-1
// input gradient as the same kernel over dy with the kernel flipped
// (replacing gemm_dX + col2im, src/conv2d.c:48-65).
//
//   Y[m, n] = sum_k A[m, k] Wt[k, n]  (+ bias[n] | * gain[0])
//   m = (b, oh, ow), k = (kh, kw, ci), A[m, k] = X[b, oh s + kh - p, ow s + kw - p, ci]
//   (0 outside the image), Wt = the reference's [K*K*C_in, C_out] weight.
//
// The im2col matrix is never written: each workgroup gathers its A tile from X
// directly (a k-slice of 32 channels of one (kh, kw) is 128 contiguous bytes
// of one input pixel).  The weight is read in the reference's layout too, with
// no transposed or flipped copy: the forward stages its [32 k][BN n] slice as
// it lies in Wt and reads the B operand 32 bits at a time; the input
// gradient's operand B[ci][(kh, kw, co)] = Wt[((K-1-kh) K + (K-1-kw)) C_in +
// ci][co] is k-contiguous and is staged like A.
//
// Workgroup tile 128 (m) x BN (n, 128 or 64), k in slices of 32; 4 waves of
// 64 x BN/2, each a 2 x BN/64 grid of 32 x 32 MFMA accumulators.  Per slice a
// thread loads 4 float4 of A and up to 4 of the weight into registers, the
// slice before it computes from LDS, then the registers go to the other LDS
// buffer (two buffers of 2 x 16 KB; two workgroups fit a CU).  A tiles (and
// the input gradient's B) are [128 rows][8 float4 chunks of 4 k] with the
// chunk index xor-swizzled by the row (slot()), so the 128-bit fragment reads
// of a wave (32 rows, one chunk per half-wave) and the tile writes are free of
// bank conflicts.  The forward's B tile is [32 k][BN n], each row rotated by
// 32 n on alternate groups of 4 rows (kslot()), so the two half-waves of a
// 32-bit fragment read (rows k and k + 4, 32 consecutive n each) use
// disjoint banks.
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
#include "igemm.h"

extern "C" {

int nnhip_conv2d_implicit_supported(int C_in, int C_out) {
    return C_in > 0 && C_out > 0 && C_in % kBK == 0 && C_out % kBNmin == 0;
}

void launch_conv2d_forward_implicit(float* Y, const float* X, const float* Wt, const float* bias,
    const float* gain, int batch, int H, int W, int C_in, int C_out, int K, int stride, int pad, int H_out,
    int W_out, hipStream_t s) {
    const char* what = "launch_conv2d_forward_implicit";
    ConvShape sh;
    if (fwd_setup(what, Y, X, Wt, bias, gain, batch, H, W, C_in, C_out, K, stride, pad, H_out, W_out, sh) <= 0)
        return;
    const int BN = tile_n(C_out);
    const dim3 grid((unsigned)((sh.M + kBM - 1) / kBM), (unsigned)(C_out / BN));
#define NNK_IGEMM_FWD(BN_)                                                                               \
    if (bias) igemm_fwd<kEpiBias, BN_, kWFwd><<<grid, kTpb, 0, s>>>(Y, X, Wt, bias, nullptr, sh, ConvEpi{});       \
    else if (gain) igemm_fwd<kEpiGain, BN_, kWFwd><<<grid, kTpb, 0, s>>>(Y, X, Wt, nullptr, gain, sh, ConvEpi{});  \
    else igemm_fwd<kEpiNone, BN_, kWFwd><<<grid, kTpb, 0, s>>>(Y, X, Wt, nullptr, nullptr, sh, ConvEpi{});
    if (BN == 128) {
        NNK_IGEMM_FWD(128)
    } else {
        NNK_IGEMM_FWD(64)
    }
#undef NNK_IGEMM_FWD
    nnk_after_launch(what, s);
}

int nnhip_conv2d_input_grad_implicit_supported(int C_in, int C_out, int K, int stride, int pad) {
    return stride == 1 && K > 0 && pad >= 0 && pad <= K - 1 && nnhip_conv2d_implicit_supported(C_out, C_in);
}

void launch_conv2d_input_grad_implicit(float* dX, const float* dY, const float* Wt, const float* gain, int batch,
    int H, int W, int C_in, int C_out, int K, int pad, hipStream_t s) {
    const char* what = "launch_conv2d_input_grad_implicit";
    ConvShape sh;
    if (dgrad_setup(what, dX, dY, Wt, batch, H, W, C_in, C_out, K, pad, sh) <= 0) return;
    const int BN = tile_n(C_in);
    const dim3 grid((unsigned)((sh.M + kBM - 1) / kBM), (unsigned)(C_in / BN));
#define NNK_IGEMM_DGRAD(BN_)                                                                                  \
    if (gain) igemm_fwd<kEpiGain, BN_, kWFlip><<<grid, kTpb, 0, s>>>(dX, dY, Wt, nullptr, gain, sh, ConvEpi{});           \
    else igemm_fwd<kEpiNone, BN_, kWFlip><<<grid, kTpb, 0, s>>>(dX, dY, Wt, nullptr, nullptr, sh, ConvEpi{});
    if (BN == 128) {
        NNK_IGEMM_DGRAD(128)
    } else {
        NNK_IGEMM_DGRAD(64)
    }
#undef NNK_IGEMM_DGRAD
    nnk_after_launch(what, s);
}

int nnhip_conv2d_wgrad_implicit_supported(int C_in, int C_out) {
    return C_in > 0 && C_out > 0 && C_in % 4 == 0 && C_out % kBNmin == 0;
}

size_t nnhip_conv2d_wgrad_workspace(int batch, int C_in, int C_out, int K, int H_out, int W_out) {
    if (batch <= 0 || !nnhip_conv2d_wgrad_implicit_supported(C_in, C_out)) return 0;
    const long long M = (long long)batch * H_out * W_out;
    if (M <= 0 || M >= (1LL << 31)) return 0;
    const WgradPlan p = wgrad_plan((int)M, K * K * C_in, C_out);
    return p.S > 1 ? (size_t)p.S * K * K * C_in * C_out : 0;
}

void launch_conv2d_weight_grad_implicit(float* gW, const float* X, const float* dY, int batch, int H, int W,
    int C_in, int C_out, int K, int stride, int pad, int H_out, int W_out, float* workspace, hipStream_t s) {
    wgrad_launch("launch_conv2d_weight_grad_implicit", gW, X, dY, batch, H, W, C_in, C_out, K, stride, pad, H_out,
        W_out, workspace, s);
}

}  // extern "C"
