// k_gns_bwd.hip -- instantiations and launch of the streaming GroupNorm
// backward (gn_stream.h); dgamma/dbeta are reduced inside the kernel.
#include "gn_stream.h"

int nnk_gns_grid(const void* fn, int key, size_t lds, int unit);
bool nnk_gns_launch(const void* fn, int P, void** args, hipStream_t s, const char* what);
unsigned nnk_gns_spin_limit();

namespace {

using namespace nnk;
using namespace nnk::gns;

// gshift[b, c] = the sum over t of the column sums colpart[b][cb][t][cl] of the
// backward's tiles (c = cb * CHW + cl), in tile order.  Consecutive threads
// read consecutive channels.
template <int CHW>
__global__ __launch_bounds__(256) void gns_colsum(float* __restrict__ gshift, const float* __restrict__ colpart,
    int B, int C, int T) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= B * C) return;
    const int b = i / C, c = i % C;
    const int cb = c / CHW, cl = c % CHW;
    const float* p = colpart + ((size_t)(b * (C / CHW) + cb) * T) * CHW + cl;
    // kB tiles in flight (predicated at the end), added in tile order
    constexpr int kB = 16;
    float a = 0.0f;
    for (int t = 0; t < T; t += kB) {
        float v[kB];
#pragma unroll
        for (int u = 0; u < kB; ++u) v[u] = t + u < T ? p[(size_t)(t + u) * CHW] : 0.0f;
#pragma unroll
        for (int u = 0; u < kB; ++u)
            if (t + u < T) a += v[u];
    }
    gshift[i] = a;
}

template <int ACT, int CPG4, int RPL, bool NT, bool SHIFT>
bool launch(const Plan& p, float* dx, float* ggamma, float* gbeta, const float* dy, const float* x,
    const float* gamma, const float* beta, const float* mu, const float* rstd, const float* shift, float* gshift,
    float* ws, hipStream_t s) {
    using Gm = Geom<kTpb, kBwdTp, kBwdCw4, CPG4>;
    const void* fn = reinterpret_cast<const void*>(&gns_bwd<Gm, ACT, RPL, NT, SHIFT>);
    const size_t lds = 0;  // all LDS is static (stage, parked, reduction buffers)
    const int key = kGnsBwdKeys +
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
    wk.part = reinterpret_cast<unsigned long long*>(reinterpret_cast<char*>(ws) + p.part_offset);
    wk.tpart = reinterpret_cast<unsigned long long*>(reinterpret_cast<char*>(ws) + p.tpart_offset);
    float* colpart = SHIFT ? reinterpret_cast<float*>(reinterpret_cast<char*>(ws) + p.colpart_offset) : nullptr;
    unsigned limit = nnk_gns_spin_limit();
    void* args[] = {&dx, &ggamma, &gbeta, const_cast<float**>(&dy), const_cast<float**>(&x),
        const_cast<float**>(&gamma), const_cast<float**>(&beta), const_cast<float**>(&mu),
        const_cast<float**>(&rstd), const_cast<float**>(&shift), &colpart, &sh, &wk, &limit};
    if (!nnk_gns_launch(fn, P, args, s, "streaming GroupNorm backward")) return false;
    if constexpr (SHIFT) {
        constexpr int kChw = 4 * kBwdCw4;
        const int n = p.sh.B * p.sh.C;
        gns_colsum<kChw><<<dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s>>>(gshift, colpart, p.sh.B,
            p.sh.C, p.sh.T);
    }
    return true;
}

template <int ACT, bool SHIFT>
bool by_shape(const Plan& p, float* dx, float* ggamma, float* gbeta, const float* dy, const float* x,
    const float* gamma, const float* beta, const float* mu, const float* rstd, const float* shift, float* gshift,
    float* ws, hipStream_t s) {
    const bool nt = use_nt(12LL * p.sh.B * p.sh.HW * p.sh.C);
#define NNK_GNS_BWD_CASE(CPG4, RPL)                                                                            \
    if (p.cpg4 == CPG4 && p.rpl == RPL)                                                                        \
        return nt ? launch<ACT, CPG4, RPL, true, SHIFT>(p, dx, ggamma, gbeta, dy, x, gamma, beta, mu, rstd,     \
                        shift, gshift, ws, s)                                                                  \
                  : launch<ACT, CPG4, RPL, false, SHIFT>(p, dx, ggamma, gbeta, dy, x, gamma, beta, mu, rstd,    \
                        shift, gshift, ws, s);
    // With a shift, one record per merging lane: with two, the tile loop runs
    // out of registers and would spill inside the loop (a spill reload is a
    // full wait on the staged loads); the launcher refuses those shapes.
    NNK_GNS_BWD_CASE(1, 1)
    NNK_GNS_BWD_CASE(2, 1)
    NNK_GNS_BWD_CASE(4, 1)
    if constexpr (!SHIFT) {
        NNK_GNS_BWD_CASE(1, 2)
        NNK_GNS_BWD_CASE(2, 2)
        NNK_GNS_BWD_CASE(4, 2)
    }
#undef NNK_GNS_BWD_CASE
    return false;
}

}  // namespace

bool nnk_gns_shift_backward_shape_ok(int act, int B, int HW, int C, int G) {
    const Plan p = make_plan(true, B, HW, C, G);
    return p.ok && act == ACT_SILU && p.rpl == 1;  // the SHIFT cases of by_shape
}

bool nnk_gns_backward(int act, float* dx, float* ggamma, float* gbeta, const float* dy, const float* x,
    const float* gamma, const float* beta, const float* mu, const float* rstd, const float* shift, float* gshift,
    int B, int HW, int C, int G, float* ws, hipStream_t s) {
    const Plan p = make_plan(true, B, HW, C, G);
    if (!p.ok || !ws || (shift != nullptr) != (gshift != nullptr)) return false;
    bool launched = false;
    // with a shift: SiLU only (the DDPM block's GN2), as in the forward
    if (shift)
        launched = act == ACT_SILU &&
            by_shape<ACT_SILU, true>(p, dx, ggamma, gbeta, dy, x, gamma, beta, mu, rstd, shift, gshift, ws, s);
    else
        NNK_ACT_DISPATCH(act, A,
            launched = by_shape<A, false>(p, dx, ggamma, gbeta, dy, x, gamma, beta, mu, rstd, shift, gshift, ws, s));
    return launched;
}
