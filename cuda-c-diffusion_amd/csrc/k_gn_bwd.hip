// k_gn_bwd.hip -- instantiations of the register-resident GroupNorm backward.
#include "gn_kernels.h"

namespace {

using namespace nnk;
using namespace nnk::gn;

template <int TPB, int NV>
bool bwd_variant(int v4pp, int act, float* dx, float* pg, float* pb, const float* dy,
    const float* x, const float* gamma, const float* beta, const float* mu,
    const float* rstd, int B, int G, int HW, int C, hipStream_t s) {
    const dim3 grid((unsigned)(B * G)), block(TPB);
    switch (v4pp) {
    case 1:
        return NNK_ACT_DISPATCH(act, A,
            gn_bwd_reg<TPB, NV, 1, A><<<grid, block, 0, s>>>(dx, pg, pb, dy, x, gamma, beta, mu, rstd, G, HW, C));
    case 2:
        return NNK_ACT_DISPATCH(act, A,
            gn_bwd_reg<TPB, NV, 2, A><<<grid, block, 0, s>>>(dx, pg, pb, dy, x, gamma, beta, mu, rstd, G, HW, C));
    case 4:
        return NNK_ACT_DISPATCH(act, A,
            gn_bwd_reg<TPB, NV, 4, A><<<grid, block, 0, s>>>(dx, pg, pb, dy, x, gamma, beta, mu, rstd, G, HW, C));
    default:
        return false;
    }
}

}  // namespace

bool nnk_gn_bwd_reg_dispatch(int cfg, int v4pp, int act, float* dx, float* part_g, float* part_b,
    const float* dy, const float* x, const float* gamma, const float* beta,
    const float* mu, const float* rstd, int B, int G, int HW, int C, hipStream_t s) {
    static_assert(kNumRegConfigs == 5, "config table and dispatch out of step");
    switch (cfg) {
    case 0: return bwd_variant<256, 1>(v4pp, act, dx, part_g, part_b, dy, x, gamma, beta, mu, rstd, B, G, HW, C, s);
    case 1: return bwd_variant<256, 4>(v4pp, act, dx, part_g, part_b, dy, x, gamma, beta, mu, rstd, B, G, HW, C, s);
    case 2: return bwd_variant<512, 4>(v4pp, act, dx, part_g, part_b, dy, x, gamma, beta, mu, rstd, B, G, HW, C, s);
    case 3: return bwd_variant<1024, 4>(v4pp, act, dx, part_g, part_b, dy, x, gamma, beta, mu, rstd, B, G, HW, C, s);
    case 4: return bwd_variant<1024, 8>(v4pp, act, dx, part_g, part_b, dy, x, gamma, beta, mu, rstd, B, G, HW, C, s);
    default: return false;
    }
}
