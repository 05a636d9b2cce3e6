// k_gns_bwd.hip -- instantiations and launch of the streaming GroupNorm
// backward (gn_stream.h); dgamma/dbeta are reduced inside the kernel.
#include "gn_stream.h"

int nnk_gns_grid(const void* fn, int key, size_t lds, int unit);
bool nnk_gns_launch(const void* fn, int P, void** args, hipStream_t s, const char* what);
unsigned nnk_gns_spin_limit();

namespace {

using namespace nnk;
using namespace nnk::gns;

template <int ACT, int CPG4, int RPL, bool NT>
bool launch(const Plan& p, float* dx, float* ggamma, float* gbeta, const float* dy, const float* x,
    const float* gamma, const float* beta, const float* mu, const float* rstd, float* ws, hipStream_t s) {
    using Gm = Geom<kTpb, kBwdTp, kBwdCw4, CPG4>;
    const void* fn = reinterpret_cast<const void*>(&gns_bwd<Gm, ACT, RPL, NT>);
    const size_t lds = 0;  // all LDS is static (stage, parked, reduction buffers)
    const int key = 128 + ((ACT * 3 + (CPG4 == 1 ? 0 : CPG4 == 2 ? 1 : 2)) * 2 + (RPL - 1)) * 2 + (NT ? 1 : 0);
    const int P = nnk_gns_grid(fn, key, lds, p.sh.T * p.sh.NCB);
    if (P <= 0) return false;
    Shape sh = p.sh;
    Work wk;
    wk.err = reinterpret_cast<unsigned*>(ws);
    unsigned* hf = nnk_wait_flag(s);
    wk.hflag = hf ? hf : wk.err;
    wk.ep = reinterpret_cast<unsigned*>(ws) + 1;
    wk.count = reinterpret_cast<unsigned*>(reinterpret_cast<char*>(ws) + kCountOffset);
    wk.rec = reinterpret_cast<unsigned long long*>(reinterpret_cast<char*>(ws) + p.rec_offset);
    wk.part = reinterpret_cast<unsigned long long*>(reinterpret_cast<char*>(ws) + p.part_offset);
    wk.tpart = reinterpret_cast<unsigned long long*>(reinterpret_cast<char*>(ws) + p.tpart_offset);
    unsigned limit = nnk_gns_spin_limit();
    void* args[] = {&dx, &ggamma, &gbeta, const_cast<float**>(&dy), const_cast<float**>(&x), const_cast<float**>(&gamma),
        const_cast<float**>(&beta), const_cast<float**>(&mu), const_cast<float**>(&rstd), &sh, &wk,
        &limit};
    return nnk_gns_launch(fn, P, args, s, "streaming GroupNorm backward");
}

template <int ACT>
bool by_shape(const Plan& p, float* dx, float* ggamma, float* gbeta, const float* dy, const float* x,
    const float* gamma, const float* beta, const float* mu, const float* rstd, float* ws, hipStream_t s) {
    const bool nt = use_nt(12LL * p.sh.B * p.sh.HW * p.sh.C);
#define NNK_GNS_BWD_CASE(CPG4, RPL)                                                                          \
    if (p.cpg4 == CPG4 && p.rpl == RPL)                                                                      \
        return nt ? launch<ACT, CPG4, RPL, true>(p, dx, ggamma, gbeta, dy, x, gamma, beta, mu, rstd, ws, s)  \
                  : launch<ACT, CPG4, RPL, false>(p, dx, ggamma, gbeta, dy, x, gamma, beta, mu, rstd, ws, s);
    NNK_GNS_BWD_CASE(1, 1)
    NNK_GNS_BWD_CASE(1, 2)
    NNK_GNS_BWD_CASE(2, 1)
    NNK_GNS_BWD_CASE(2, 2)
    NNK_GNS_BWD_CASE(4, 1)
    NNK_GNS_BWD_CASE(4, 2)
#undef NNK_GNS_BWD_CASE
    return false;
}

}  // namespace

bool nnk_gns_backward(int act, float* dx, float* ggamma, float* gbeta, const float* dy, const float* x,
    const float* gamma, const float* beta, const float* mu, const float* rstd, int B, int HW, int C, int G,
    float* ws, hipStream_t s) {
    const Plan p = make_plan(true, B, HW, C, G);
    if (!p.ok || !ws) return false;
    bool launched = false;
    NNK_ACT_DISPATCH(act, A, launched = by_shape<A>(p, dx, ggamma, gbeta, dy, x, gamma, beta, mu, rstd, ws, s));
    return launched;
}
