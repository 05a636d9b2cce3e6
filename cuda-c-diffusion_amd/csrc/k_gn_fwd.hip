// k_gn_fwd.hip -- instantiations of the register-resident GroupNorm forward.
#include "gn_kernels.h"

namespace {

using namespace nnk;
using namespace nnk::gn;

template <int TPB, int NV>
bool fwd_variant(int v4pp, int act, float* y, float* mu, float* rstd, const float* x,
    const float* gamma, const float* beta, int B, int G, int HW, int C, float eps,
    hipStream_t s) {
    const dim3 grid((unsigned)(B * G)), block(TPB);
    switch (v4pp) {
    case 1:
        return NNK_ACT_DISPATCH(act, A,
            gn_fwd_reg<TPB, NV, 1, A><<<grid, block, 0, s>>>(y, mu, rstd, x, gamma, beta, G, HW, C, eps));
    case 2:
        return NNK_ACT_DISPATCH(act, A,
            gn_fwd_reg<TPB, NV, 2, A><<<grid, block, 0, s>>>(y, mu, rstd, x, gamma, beta, G, HW, C, eps));
    case 4:
        return NNK_ACT_DISPATCH(act, A,
            gn_fwd_reg<TPB, NV, 4, A><<<grid, block, 0, s>>>(y, mu, rstd, x, gamma, beta, G, HW, C, eps));
    default:
        return false;
    }
}

}  // namespace

bool nnk_gn_fwd_reg_dispatch(int cfg, int v4pp, int act, float* y, float* mu, float* rstd,
    const float* x, const float* gamma, const float* beta,
    int B, int G, int HW, int C, float eps, hipStream_t s) {
    static_assert(kNumRegConfigs == 5, "config table and dispatch out of step");
    switch (cfg) {
    case 0: return fwd_variant<256, 1>(v4pp, act, y, mu, rstd, x, gamma, beta, B, G, HW, C, eps, s);
    case 1: return fwd_variant<256, 4>(v4pp, act, y, mu, rstd, x, gamma, beta, B, G, HW, C, eps, s);
    case 2: return fwd_variant<512, 4>(v4pp, act, y, mu, rstd, x, gamma, beta, B, G, HW, C, eps, s);
    case 3: return fwd_variant<1024, 4>(v4pp, act, y, mu, rstd, x, gamma, beta, B, G, HW, C, eps, s);
    case 4: return fwd_variant<1024, 8>(v4pp, act, y, mu, rstd, x, gamma, beta, B, G, HW, C, eps, s);
    default: return false;
    }
}
