// k_gns_fwd.hip -- instantiations and launch of the streaming GroupNorm
// forward (gn_stream.h).
#include "gn_stream.h"

int nnk_gns_grid(const void* fn, int key, size_t lds, int unit);
bool nnk_gns_launch(const void* fn, int P, void** args, hipStream_t s, const char* what);
unsigned nnk_gns_spin_limit();

namespace {

using namespace nnk;
using namespace nnk::gns;

template <int ACT, int CPG4, int RPL, bool NT, bool SHIFT>
bool launch(const Plan& p, float* y, float* mu, float* rstd, const float* x, const float* gamma,
    const float* beta, const float* shift, float eps, float* ws, hipStream_t s) {
    using Gm = Geom<kTpb, kFwdTp, kFwdCw4, CPG4>;
    const void* fn = reinterpret_cast<const void*>(&gns_fwd<Gm, ACT, RPL, NT, SHIFT>);
    const size_t lds = 0;  // all LDS is static (stage, parked, reduction buffers)
    const int key =
        (((ACT * 3 + (CPG4 == 1 ? 0 : CPG4 == 2 ? 1 : 2)) * 2 + (RPL - 1)) * 2 + (NT ? 1 : 0)) * 2 + (SHIFT ? 1 : 0);
    const int P = nnk_gns_grid(fn, key, lds, p.sh.T * p.sh.NCB);
    if (P <= 0) return false;
    Shape sh = p.sh;
    Work wk;
    wk.err = reinterpret_cast<unsigned*>(ws);
    unsigned* hf = nnk_wait_flag();
    wk.hflag = hf ? hf : wk.err;
    wk.ep = reinterpret_cast<unsigned*>(ws) + 1;
    wk.count = reinterpret_cast<unsigned*>(reinterpret_cast<char*>(ws) + kCountOffset);
    wk.rec = reinterpret_cast<unsigned long long*>(reinterpret_cast<char*>(ws) + p.rec_offset);
    wk.part = nullptr;
    wk.tpart = nullptr;
    unsigned limit = nnk_gns_spin_limit();
    void* args[] = {&y, &mu, &rstd, const_cast<float**>(&x), const_cast<float**>(&gamma),
        const_cast<float**>(&beta), const_cast<float**>(&shift), &sh, &wk, &eps, &limit};
    return nnk_gns_launch(fn, P, args, s, "streaming GroupNorm forward");
}

template <int ACT, bool SHIFT>
bool by_shape(const Plan& p, float* y, float* mu, float* rstd, const float* x, const float* gamma,
    const float* beta, const float* shift, float eps, float* ws, hipStream_t s) {
    const bool nt = use_nt(8LL * p.sh.B * p.sh.HW * p.sh.C);
#define NNK_GNS_FWD_CASE(CPG4, RPL)                                                                      \
    if (p.cpg4 == CPG4 && p.rpl == RPL)                                                                  \
        return nt ? launch<ACT, CPG4, RPL, true, SHIFT>(p, y, mu, rstd, x, gamma, beta, shift, eps, ws, s) \
                  : launch<ACT, CPG4, RPL, false, SHIFT>(p, y, mu, rstd, x, gamma, beta, shift, eps, ws, s);
    // With a shift, 8 or 16 channels per group: at 4 the tile loop runs out
    // of registers and would spill inside the loop (a spill reload is a full
    // wait on the staged loads); the launcher refuses those shapes.
    if constexpr (SHIFT) {
        NNK_GNS_FWD_CASE(2, 1)
        NNK_GNS_FWD_CASE(2, 2)
        NNK_GNS_FWD_CASE(4, 1)
        NNK_GNS_FWD_CASE(4, 2)
    } else {
        NNK_GNS_FWD_CASE(1, 1)
        NNK_GNS_FWD_CASE(1, 2)
        NNK_GNS_FWD_CASE(2, 1)
        NNK_GNS_FWD_CASE(2, 2)
        NNK_GNS_FWD_CASE(4, 1)
        NNK_GNS_FWD_CASE(4, 2)
    }
#undef NNK_GNS_FWD_CASE
    return false;
}

}  // namespace

bool nnk_gns_shift_forward_shape_ok(int act, int B, int HW, int C, int G) {
    const Plan p = make_plan(false, B, HW, C, G);
    return p.ok && act == ACT_SILU && (p.cpg4 == 2 || p.cpg4 == 4);  // the SHIFT cases of by_shape
}

bool nnk_gns_forward(int act, float* y, float* mu, float* rstd, const float* x, const float* gamma,
    const float* beta, const float* shift, int B, int HW, int C, int G, float eps, float* ws, hipStream_t s) {
    const Plan p = make_plan(false, B, HW, C, G);
    if (!p.ok || !ws) return false;
    bool launched = false;
    // with a shift: SiLU only (the DDPM block's GN2)
    if (shift)
        launched = act == ACT_SILU &&
            by_shape<ACT_SILU, true>(p, y, mu, rstd, x, gamma, beta, shift, eps, ws, s);
    else
        NNK_ACT_DISPATCH(act, A, launched = by_shape<A, false>(p, y, mu, rstd, x, gamma, beta, shift, eps, ws, s));
    return launched;
}
