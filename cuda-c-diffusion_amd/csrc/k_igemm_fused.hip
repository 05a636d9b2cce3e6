// k_igemm_fused.hip -- the implicit-GEMM convolutions with a neighbouring pass
// of the diffusion blocks folded in, so that the tensor between the two is
// never written to HBM or read back:
//   forward + residual        y = wa res + wb conv           (src/cond_conv_residual.c:34-35,
//                                                              src/conv_residual.c:38-39)
//   forward + modulate + act  y = conv, y2 = act(y (c + 1))  (src/cond_conv_residual.c:29, 31-33)
//   input gradient + act' + residual
//                             dx = wa res + 1 (conv^T(dy) act'(x))
//                                                            (src/cond_conv_residual.c:53-54, 61)
// The kernels are those of k_igemm.hip (igemm.h) with the pass in the
// epilogue; each computes with the replaced pass's operation order, so the
// outputs equal the separate launches' bit for bit.  Only these combinations
// are built.
#include "igemm.h"

namespace {

bool act_fusable(int act) { return act == ACT_SILU || act == ACT_MP_SILU; }

}  // namespace

extern "C" {

void launch_conv2d_forward_implicit_fused(float* Y, const float* X, const float* Wt, const float* bias,
    const float* gain, int batch, int H, int W, int C_in, int C_out, int K, int stride, int pad, int H_out,
    int W_out, const NnConvFusion* f, hipStream_t s) {
    const char* what = "launch_conv2d_forward_implicit_fused";
    NNK_REQUIRE(f, what, "%s: null fusion", what);
    NNK_REQUIRE(!f->act_in, what, "%s: act_in belongs to the input gradient", what);
    NNK_REQUIRE((f->res != nullptr) != (f->cond != nullptr), what,
        "%s: exactly one of res (residual) and cond (modulate + activation) is fused", what);
    if (f->cond) {
        NNK_REQUIRE(act_fusable(f->act), what, "%s: the modulate epilogue takes ACT_SILU or ACT_MP_SILU, not %d",
            what, (int)f->act);
    }
    ConvShape sh;
    if (fwd_setup(what, Y, X, Wt, bias, gain, batch, H, W, C_in, C_out, K, stride, pad, H_out, W_out, sh) <= 0)
        return;
    NNK_REQUIRE(!f->cond || f->y2, what, "%s: null y2", what);
    ConvEpi ep{};
    ep.res = f->res;
    ep.wa = f->res_w;
    ep.wb = f->out_w;
    ep.cond = f->cond;
    ep.y2 = f->y2;
    ep.hw = FastDiv((uint32_t)(H_out * W_out));
    const int BN = tile_n(C_out);
    const dim3 grid((unsigned)((sh.M + kBM - 1) / kBM), (unsigned)(C_out / BN));
#define NNK_FWD_EPI(XE_, ACT_, BN_)                                                                             \
    do {                                                                                                        \
        if (bias) igemm_fwd<kEpiBias, BN_, kWFwd, XE_, ACT_><<<grid, kTpb, 0, s>>>(Y, X, Wt, bias, nullptr, sh, ep); \
        else if (gain) igemm_fwd<kEpiGain, BN_, kWFwd, XE_, ACT_><<<grid, kTpb, 0, s>>>(Y, X, Wt, nullptr, gain, sh, ep); \
        else igemm_fwd<kEpiNone, BN_, kWFwd, XE_, ACT_><<<grid, kTpb, 0, s>>>(Y, X, Wt, nullptr, nullptr, sh, ep); \
    } while (0)
#define NNK_FWD_BN(XE_, ACT_)                 \
    do {                                      \
        if (BN == 128) NNK_FWD_EPI(XE_, ACT_, 128); \
        else NNK_FWD_EPI(XE_, ACT_, 64);      \
    } while (0)
    if (f->res) NNK_FWD_BN(kXeRes, 0);
    else if (f->act == ACT_SILU) NNK_FWD_BN(kXeMod, ACT_SILU);
    else NNK_FWD_BN(kXeMod, ACT_MP_SILU);
#undef NNK_FWD_BN
#undef NNK_FWD_EPI
    nnk_after_launch(what, s);
}

void launch_conv2d_input_grad_implicit_fused(float* dX, const float* dY, const float* Wt, const float* gain,
    int batch, int H, int W, int C_in, int C_out, int K, int pad, const NnConvFusion* f, hipStream_t s) {
    const char* what = "launch_conv2d_input_grad_implicit_fused";
    NNK_REQUIRE(f, what, "%s: null fusion", what);
    NNK_REQUIRE(!f->cond && !f->y2, what, "%s: cond and y2 belong to the forward", what);
    NNK_REQUIRE(f->act_in && f->res, what, "%s: builds act_in with res", what);
    NNK_REQUIRE(act_fusable(f->act), what,
        "%s: the activation-gradient epilogue takes ACT_SILU or ACT_MP_SILU, not %d", what, (int)f->act);
    ConvShape sh;
    if (dgrad_setup(what, dX, dY, Wt, batch, H, W, C_in, C_out, K, pad, sh) <= 0) return;
    ConvEpi ep{};
    ep.res = f->res;
    ep.xa = f->act_in;
    ep.wa = f->res_w;
    ep.wb = f->out_w;
    const int BN = tile_n(C_in);
    const dim3 grid((unsigned)((sh.M + kBM - 1) / kBM), (unsigned)(C_in / BN));
#define NNK_DGRAD_EPI(ACT_, BN_)                                                                                 \
    do {                                                                                                         \
        if (gain) igemm_fwd<kEpiGain, BN_, kWFlip, kXeActG | kXeRes, ACT_><<<grid, kTpb, 0, s>>>(dX, dY, Wt, nullptr, gain, sh, ep); \
        else igemm_fwd<kEpiNone, BN_, kWFlip, kXeActG | kXeRes, ACT_><<<grid, kTpb, 0, s>>>(dX, dY, Wt, nullptr, nullptr, sh, ep); \
    } while (0)
#define NNK_DGRAD_BN(ACT_)                 \
    do {                                   \
        if (BN == 128) NNK_DGRAD_EPI(ACT_, 128); \
        else NNK_DGRAD_EPI(ACT_, 64);      \
    } while (0)
    if (f->act == ACT_SILU) NNK_DGRAD_BN(ACT_SILU);
    else NNK_DGRAD_BN(ACT_MP_SILU);
#undef NNK_DGRAD_BN
#undef NNK_DGRAD_EPI
    nnk_after_launch(what, s);
}

}  // extern "C"
