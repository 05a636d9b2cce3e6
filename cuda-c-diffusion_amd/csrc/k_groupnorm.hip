// k_groupnorm.hip -- GroupNorm launchers (reference src/kernels.cu:719-745 and
// the fused GroupNorm+activation additions) and the shape-generic kernels.
//
// Path choice per call:
//   * register-resident (gn_kernels.h): cpg in {4, 8, 16}, 16-byte aligned
//     tensors, group of at most 32768 floats.  One HBM pass.
//   * generic (below): any cpg / size / alignment.  Streams the group twice
//     (statistics, then output) and computes the dgamma/dbeta partials in a
//     separate coalesced kernel.  Same maths, same reduction discipline.
#include <stdlib.h>
#include <string.h>

#include <mutex>

#include "gn_kernels.h"
#include "gn_stream.h"


namespace {

using namespace nnk;
using namespace nnk::gn;

constexpr int kGenTpb = 256;
constexpr int kGenNw = kGenTpb / kWave;

template <int ACT>
__global__ __launch_bounds__(kGenTpb) void gn_fwd_generic(float* __restrict__ y,
    float* __restrict__ mu_out, float* __restrict__ rstd_out, const float* __restrict__ x,
    const float* __restrict__ gamma, const float* __restrict__ beta, int G, int HW, int C,
    int cpg, FastDiv div_cpg, float eps) {
    __shared__ float red[2 * kGenNw];
    const int work = blockIdx.x;
    const int b = work / G;
    const int g = work - b * G;
    const int n = HW * cpg;
    const size_t base = (size_t)b * HW * C + (size_t)g * cpg;
    const float* xb = x + base;

    float s = 0.0f;
    for (int i = threadIdx.x; i < n; i += kGenTpb) {
        uint32_t hw, cl;
        div_cpg.divmod((uint32_t)i, hw, cl);
        s += xb[(size_t)hw * C + cl];
    }
    const float nf = (float)n;
    const float mean = block_sum<kGenNw>(s, red) / nf;
    float q = 0.0f;
    for (int i = threadIdx.x; i < n; i += kGenTpb) {
        uint32_t hw, cl;
        div_cpg.divmod((uint32_t)i, hw, cl);
        const float d = xb[(size_t)hw * C + cl] - mean;
        q += d * d;
    }
    const float var = block_sum<kGenNw>(q, red + kGenNw) / nf;
    const float rs = rsqrtf(var + eps);
    if (threadIdx.x == 0) {
        mu_out[work] = mean;
        rstd_out[work] = rs;
    }
    for (int i = threadIdx.x; i < n; i += kGenTpb) {
        uint32_t hw, cl;
        div_cpg.divmod((uint32_t)i, hw, cl);
        const size_t o = (size_t)hw * C + cl;
        const int c = g * cpg + (int)cl;
        y[base + o] = act_fwd<ACT>(gamma[c] * ((xb[o] - mean) * rs) + beta[c]);
    }
}

// PART: cpg is a power of two <= 64, so each thread always meets the same
// channel (threadIdx.x % cpg) and the kernel also writes that sample's
// dgamma/dbeta partials part_g/part_b[b*C + c] (sum over the pixels of d*xhat
// and of d): per thread in element order, then a fixed xor tree over the
// wave's lanes of the channel, then the waves in order.  Otherwise
// gn_param_partial_generic computes them in a launch of its own.
template <int ACT, bool PART = false>
__global__ __launch_bounds__(kGenTpb) void gn_bwd_dx_generic(float* __restrict__ dx,
    const float* __restrict__ dy, const float* __restrict__ x, const float* __restrict__ gamma,
    const float* __restrict__ beta, const float* __restrict__ mu, const float* __restrict__ rstd,
    int G, int HW, int C, int cpg, FastDiv div_cpg, float* __restrict__ part_g = nullptr,
    float* __restrict__ part_b = nullptr) {
    __shared__ float red[2 * kGenNw];
    __shared__ float cred[PART ? 2 : 1][kGenNw][PART ? kWave : 1];
    const int work = blockIdx.x;
    const int b = work / G;
    const int g = work - b * G;
    const int n = HW * cpg;
    const size_t base = (size_t)b * HW * C + (size_t)g * cpg;
    const float mean = mu[work];
    const float rs = rstd[work];

    float pg = 0.0f, pgx = 0.0f;
    for (int i = threadIdx.x; i < n; i += kGenTpb) {
        uint32_t hw, cl;
        div_cpg.divmod((uint32_t)i, hw, cl);
        const size_t o = base + (size_t)hw * C + cl;
        const int c = g * cpg + (int)cl;
        const float xh = (x[o] - mean) * rs;
        float d = dy[o];
        if constexpr (ACT != ACT_IDENTITY) d = d * act_grad<ACT>(gamma[c] * xh + beta[c]);
        const float gg = d * gamma[c];
        pg += gg;
        pgx += gg * xh;
    }
    block_sum2<kGenNw>(pg, pgx, red);
    const float inv_n = 1.0f / (float)n;
    const float m1 = pg * inv_n;
    float sg = 0.0f, sb = 0.0f;
    for (int i = threadIdx.x; i < n; i += kGenTpb) {
        uint32_t hw, cl;
        div_cpg.divmod((uint32_t)i, hw, cl);
        const size_t o = base + (size_t)hw * C + cl;
        const int c = g * cpg + (int)cl;
        const float xh = (x[o] - mean) * rs;
        float d = dy[o];
        if constexpr (ACT != ACT_IDENTITY) d = d * act_grad<ACT>(gamma[c] * xh + beta[c]);
        const float gg = d * gamma[c];
        dx[o] = rs * ((gg - m1) - xh * pgx * inv_n);
        if constexpr (PART) {
            sg += d * xh;
            sb += d;
        }
    }
    if constexpr (PART) {
        const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
        for (int o = kWave / 2; o >= cpg; o >>= 1) {
            sg += __shfl_xor(sg, o);
            sb += __shfl_xor(sb, o);
        }
        if (lane < cpg) {
            cred[0][wid][lane] = sg;
            cred[1][wid][lane] = sb;
        }
        __syncthreads();
        if (threadIdx.x < cpg) {
            float ag = cred[0][0][threadIdx.x], ab = cred[1][0][threadIdx.x];
#pragma unroll
            for (int w = 1; w < kGenNw; ++w) {
                ag += cred[0][w][threadIdx.x];
                ab += cred[1][w][threadIdx.x];
            }
            part_g[(size_t)b * C + g * cpg + threadIdx.x] = ag;
            part_b[(size_t)b * C + g * cpg + threadIdx.x] = ab;
        }
    }
}

// part_g[b*C+c] = sum_hw d*xhat, part_b[b*C+c] = sum_hw d.  Grid (ceil(C/64), B);
// lanes walk 64 consecutive channels (coalesced), the 4 waves split the pixels.
template <int ACT>
__global__ __launch_bounds__(kGenTpb) void gn_param_partial_generic(float* __restrict__ part_g,
    float* __restrict__ part_b, const float* __restrict__ dy, const float* __restrict__ x,
    const float* __restrict__ gamma, const float* __restrict__ beta,
    const float* __restrict__ mu, const float* __restrict__ rstd, int G, int HW, int C, int cpg) {
    __shared__ float lg[kGenNw][kWave];
    __shared__ float lb[kGenNw][kWave];
    const int lane = threadIdx.x & (kWave - 1);
    const int wid = threadIdx.x / kWave;
    const int c = blockIdx.x * kWave + lane;
    const int b = blockIdx.y;
    float sg = 0.0f, sb = 0.0f;
    if (c < C) {
        const int g = c / cpg;
        const float mean = mu[b * G + g];
        const float rs = rstd[b * G + g];
        const float gmc = gamma[c];
        float btc = 0.0f;
        if constexpr (ACT != ACT_IDENTITY) btc = beta[c];
        for (int hw = wid; hw < HW; hw += kGenNw) {
            const size_t o = ((size_t)b * HW + hw) * C + c;
            const float xh = (x[o] - mean) * rs;
            float d = dy[o];
            if constexpr (ACT != ACT_IDENTITY) d = d * act_grad<ACT>(gmc * xh + btc);
            sg += d * xh;
            sb += d;
        }
    }
    lg[wid][lane] = sg;
    lb[wid][lane] = sb;
    __syncthreads();
    if (wid == 0 && c < C) {
        float ag = lg[0][lane], ab = lb[0][lane];
#pragma unroll
        for (int w = 1; w < kGenNw; ++w) {
            ag += lg[w][lane];
            ab += lb[w][lane];
        }
        part_g[(size_t)b * C + c] = ag;
        part_b[(size_t)b * C + c] = ab;
    }
}

// ggamma[c] = sum_b part_g[b*C+c] (and gbeta), fixed order: wave w of the
// 16 sums b = w, w+16, ... ascending, then the 16 wave sums are added in wave
// order.  One 1024-thread workgroup per 64 channels keeps the serial chain at
// B/16 loads.
constexpr int kRedTpb = 1024;
constexpr int kRedNw = kRedTpb / kWave;

__global__ __launch_bounds__(kRedTpb) void gn_param_reduce(float* __restrict__ ggamma,
    float* __restrict__ gbeta, const float* __restrict__ part_g,
    const float* __restrict__ part_b, int B, int C) {
    __shared__ float lg[kRedNw][kWave];
    __shared__ float lb[kRedNw][kWave];
    const int lane = threadIdx.x & (kWave - 1);
    const int wid = threadIdx.x / kWave;
    const int c = blockIdx.x * kWave + lane;
    float sg = 0.0f, sb = 0.0f;
    if (c < C) {
        for (int b = wid; b < B; b += kRedNw) {
            sg += part_g[(size_t)b * C + c];
            sb += part_b[(size_t)b * C + c];
        }
    }
    lg[wid][lane] = sg;
    lb[wid][lane] = sb;
    __syncthreads();
    if (wid == 0 && c < C) {
        float ag = lg[0][lane], ab = lb[0][lane];
#pragma unroll
        for (int w = 1; w < kRedNw; ++w) {
            ag += lg[w][lane];
            ab += lb[w][lane];
        }
        ggamma[c] = ag;
        gbeta[c] = ab;
    }
}

__global__ void fill_zero2(float* __restrict__ a, float* __restrict__ b, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        a[i] = 0.0f;
        b[i] = 0.0f;
    }
}

bool valid_act(int act) { return act >= ACT_IDENTITY && act <= ACT_MP_SILU; }

// v4pp for the register path, or 0 when the shape/alignment needs the generic path.
int reg_v4pp(int cpg, long long HW, const void* p0, const void* p1, const void* p2,
    const void* p3, int& cfg) {
    if (cpg % 4 != 0) return 0;
    const int v4pp = cpg / 4;
    if (v4pp != 1 && v4pp != 2 && v4pp != 4) return 0;
    if (!aligned16(p0) || !aligned16(p1) || !aligned16(p2) || (p3 && !aligned16(p3))) return 0;
    cfg = pick_reg_config(HW * v4pp);
    return cfg < 0 ? 0 : v4pp;
}

bool shape_ok(const char* what, int B, int HW, int C, int G) {
    if (B < 0 || HW <= 0 || C <= 0 || G <= 0) {
        nnk_set_error(hipErrorInvalidValue, "%s: bad shape batch=%d HW=%d C=%d G=%d", what, B, HW, C, G);
        return false;
    }
    if (C % G != 0) {
        nnk_set_error(hipErrorInvalidValue, "%s: C=%d is not divisible by G=%d", what, C, G);
        return false;
    }
    if ((long long)HW * (C / G) >= (1LL << 31) || (long long)B * G >= (1LL << 31)) {
        nnk_set_error(hipErrorInvalidValue, "%s: group too large (HW*C/G=%lld)", what,
            (long long)HW * (C / G));
        return false;
    }
    return true;
}

// Path policy: NNHIP_GN_PATH=stream uses the streaming kernels whenever the
// shape fits them, =reg never; unset (auto) uses them for tensors of at least
// kStreamMinElems elements, below which the register-resident kernels win,
// and for any size the register-resident kernels cannot take (their
// alternative is the two-pass generic kernel).
enum class GnPath { kAuto, kStream, kReg };

// A lent workspace starts with the streaming kernels' fixed-size header (its
// first word is their wait-timeout flag, set and never cleared by them; then
// their arrival counters); the other paths keep their data after it.
constexpr size_t kWsHeader = nnk::gns::kHeaderBytes / sizeof(float);
constexpr long long kStreamMinElems = 1LL << 22;

GnPath gn_path() {  // read per launch, so a process can switch paths
    const char* e = getenv("NNHIP_GN_PATH");
    if (e && strcmp(e, "stream") == 0) return GnPath::kStream;
    if (e && strcmp(e, "reg") == 0) return GnPath::kReg;
    return GnPath::kAuto;
}

bool want_stream(bool bwd, int B, int HW, int C, int G, bool reg_ok) {
    const GnPath path = gn_path();
    if (path == GnPath::kReg) return false;
    if (!nnk::gns::make_plan(bwd, B, HW, C, G).ok) return false;
    return path == GnPath::kStream || !reg_ok || (long long)B * HW * C >= kStreamMinElems;
}

// Streaming launch on the caller's workspace or on one drawn from the
// stream-ordered pool.  The kernels accept a statistics record only when it
// carries the launch's epoch, which the workspace itself keeps (one more than
// the last launch's on it, never 0; advanced on the device, so a graph replay
// gets a new one).  A lent workspace is zero-filled by its owner before first
// use and written only by these launchers, so it can hold only zeros and older
// epochs; a pool block may hold anything and is zeroed first.
// `shift`: the launch is a backward with a shift, whose workspace also holds
// the per-tile column sums (plain floats past the epoch-tagged region, which
// alone needs clearing).
template <class F>
bool run_stream(bool bwd, int B, int HW, int C, int G, float* ws, hipStream_t s, const char* what, F launch,
    bool shift = false) {
    const nnk::gns::Plan p = nnk::gns::make_plan(bwd, B, HW, C, G);
    float* w = ws;
    if (!w) {
        w = nnk_scratch_acquire(shift ? p.ws_shift_floats : p.ws_floats, s, what);
        if (!w) return false;
        nnk_clear_workspace(w, p.ws_floats, s);
    }
    const bool ok = launch(w);
    if (!ws) nnk_scratch_release(w, s);
    return ok;
}

template <class F>
bool try_stream(bool bwd, int B, int HW, int C, int G, bool reg_ok, float* ws, hipStream_t s, const char* what,
    F launch, bool shift = false) {
    return want_stream(bwd, B, HW, C, G, reg_ok) && run_stream(bwd, B, HW, C, G, ws, s, what, launch, shift);
}

// Offset (floats) of the register path's channel partials in a backward
// workspace: past the header and, where the streaming plan applies, past its
// records, so the two paths never write the same words.
size_t reg_partials_offset(int B, int HW, int C, int G) {
    const nnk::gns::Plan p = nnk::gns::make_plan(true, B, HW, C, G);
    return p.ok ? p.ws_floats : kWsHeader;
}

void gn_forward_impl(const char* what, float* y, float* mu, float* rstd, const float* x,
    const float* gamma, const float* beta, int B, int HW, int C, int G, float eps, int act,
    float* ws, hipStream_t s) {
    if (!shape_ok(what, B, HW, C, G)) return;
    NNK_REQUIRE(valid_act(act), what, "%s: unknown activation %d", what, act);
    if (B == 0) return;
    NNK_REQUIRE(y && mu && rstd && x && gamma && beta, what, "%s: null pointer", what);
    NNK_REQUIRE(ws == nullptr || aligned16(ws), what, "%s: workspace must be 16-byte aligned", what);
    const int cpg = C / G;
    int cfg = -1;
    const int v4pp = reg_v4pp(cpg, HW, x, y, gamma, beta, cfg);
    bool launched = false;
    const bool stream_aligned = aligned16(x) && aligned16(y) && aligned16(gamma) && aligned16(beta);
    if (stream_aligned && try_stream(false, B, HW, C, G, v4pp != 0, ws, s, what, [&](float* w) {
            return nnk_gns_forward(act, y, mu, rstd, x, gamma, beta, nullptr, B, HW, C, G, eps, w, s);
        })) {
        nnk_after_launch(what, s);
        return;
    }
    if (v4pp) launched = nnk_gn_fwd_reg_dispatch(cfg, v4pp, act, y, mu, rstd, x, gamma, beta, B, G, HW, C, eps, s);
    if (!launched) {
        const FastDiv dv((uint32_t)cpg);
        const dim3 grid((unsigned)(B * G)), block(kGenTpb);
        NNK_ACT_DISPATCH(act, A,
            gn_fwd_generic<A><<<grid, block, 0, s>>>(y, mu, rstd, x, gamma, beta, G, HW, C, cpg, dv, eps));
    }
    nnk_after_launch(what, s);
}

// Whether a backward on these pointers and this shape takes the streaming
// kernels (the choice gn_backward_impl makes; it falls back to the register
// or generic path only if the streaming launch itself is refused).
bool bwd_stream_selected(const float* dx, const float* dy, const float* x, const float* gamma, const float* beta,
    int B, int HW, int C, int G, int act) {
    const bool stream_aligned = aligned16(x) && aligned16(dy) && aligned16(dx) && aligned16(gamma) &&
        (act == ACT_IDENTITY || aligned16(beta));
    if (!stream_aligned) return false;
    int cfg = -1;
    const bool reg_ok =
        reg_v4pp(C / G, HW, x, dy, dx, gamma, cfg) != 0 && (act == ACT_IDENTITY || aligned16(beta));
    return want_stream(true, B, HW, C, G, reg_ok);
}

// ws: a lent workspace (nullptr: draw from the stream's pool block).
// reg_ws: where the register and generic paths keep their 2 * B * C channel
// partials (nullptr: in ws past its streaming region, or in the pool block).
void gn_backward_impl(const char* what, float* dx, float* ggamma, float* gbeta, const float* dy,
    const float* x, const float* gamma, const float* beta, const float* mu, const float* rstd,
    int B, int HW, int C, int G, int act, float* ws, hipStream_t s, float* reg_ws = nullptr) {
    if (!shape_ok(what, B, HW, C, G)) return;
    NNK_REQUIRE(valid_act(act), what, "%s: unknown activation %d", what, act);
    NNK_REQUIRE(ggamma && gbeta, what, "%s: null pointer", what);
    if (B == 0) {
        fill_zero2<<<dim3((unsigned)((C + 255) / 256)), dim3(256), 0, s>>>(ggamma, gbeta, C);
        nnk_after_launch(what, s);
        return;
    }
    NNK_REQUIRE(dx && dy && x && gamma && mu && rstd, what, "%s: null pointer", what);
    NNK_REQUIRE(act == ACT_IDENTITY || beta, what, "%s: beta is required with an activation", what);
    NNK_REQUIRE(ws == nullptr || aligned16(ws), what, "%s: workspace must be 16-byte aligned", what);
    if (bwd_stream_selected(dx, dy, x, gamma, beta, B, HW, C, G, act) &&
        run_stream(true, B, HW, C, G, ws, s, what, [&](float* w) {
            return nnk_gns_backward(act, dx, ggamma, gbeta, dy, x, gamma, beta, mu, rstd, nullptr, nullptr, B, HW,
                C, G, w, s);
        })) {
        nnk_after_launch(what, s);
        return;
    }
    float* scratch = reg_ws ? reg_ws : ws;
    const size_t part_off = (ws && !reg_ws) ? reg_partials_offset(B, HW, C, G) : 0;
    if (!scratch) {
        scratch = nnk_scratch_acquire((size_t)2 * B * C, s, what);
        if (!scratch) return;
    }
    float* part_g = scratch + part_off;
    float* part_b = part_g + (size_t)B * C;
    const int cpg = C / G;
    int cfg = -1;
    const int v4pp = reg_v4pp(cpg, HW, x, dy, dx, gamma, cfg);
    const bool beta_ok = act == ACT_IDENTITY || aligned16(beta);
    bool launched = false;
    if (v4pp && beta_ok)
        launched = nnk_gn_bwd_reg_dispatch(cfg, v4pp, act, dx, part_g, part_b, dy, x, gamma, beta,
            mu, rstd, B, G, HW, C, s);
    if (!launched) {
        const FastDiv dv((uint32_t)cpg);
        // powers of two up to 64 channels per group: the partials come out of
        // the dx kernel (one launch fewer, and the separate kernel has only
        // ceil(C / 64) * B workgroups: 8 at the reference DDPM's first level)
        const bool fused_part = cpg <= kWave && (cpg & (cpg - 1)) == 0;
        NNK_ACT_DISPATCH(act, A, {
            if (fused_part) {
                gn_bwd_dx_generic<A, true><<<dim3((unsigned)(B * G)), dim3(kGenTpb), 0, s>>>(dx, dy, x, gamma,
                    beta, mu, rstd, G, HW, C, cpg, dv, part_g, part_b);
            } else {
                gn_bwd_dx_generic<A><<<dim3((unsigned)(B * G)), dim3(kGenTpb), 0, s>>>(dx, dy, x, gamma,
                    beta, mu, rstd, G, HW, C, cpg, dv);
                gn_param_partial_generic<A><<<dim3((unsigned)((C + kWave - 1) / kWave), (unsigned)B),
                    dim3(kGenTpb), 0, s>>>(part_g, part_b, dy, x, gamma, beta, mu, rstd, G, HW, C, cpg);
            }
        });
    }
    gn_param_reduce<<<dim3((unsigned)((C + kWave - 1) / kWave)), dim3(kRedTpb), 0, s>>>(ggamma,
        gbeta, part_g, part_b, B, C);
    if (!ws && !reg_ws) nnk_scratch_release(scratch, s);
    nnk_after_launch(what, s);
}

// Whether the shift launchers run their fused kernels on this shape, given
// 16-byte aligned pointers: a streaming plan with a shift kernel for it, and
// the path policy choosing the streaming kernels (as for the plain launchers).
bool shift_fused(bool bwd, int B, int HW, int C, int G, int act) {
    if (B <= 0 || HW <= 0 || C <= 0 || G <= 0 || C % G != 0) return false;
    if (!(bwd ? nnk_gns_shift_backward_shape_ok(act, B, HW, C, G) : nnk_gns_shift_forward_shape_ok(act, B, HW, C, G)))
        return false;
    const void* aligned = reinterpret_cast<const void*>(uintptr_t(256));
    int cfg = -1;
    const bool reg_ok = reg_v4pp(C / G, HW, aligned, aligned, aligned, aligned, cfg) != 0;
    return want_stream(bwd, B, HW, C, G, reg_ok);
}

// The shift launchers only ever run the fused kernels, on the caller's
// workspace: a shape those kernels do not take is refused (the caller adds
// the shift itself, as the reference does, and calls the plain launchers).
void gn_shift_forward_impl(const char* what, float* y, float* mu, float* rstd, const float* x, const float* shift,
    const float* gamma, const float* beta, int B, int HW, int C, int G, float eps, int act, float* ws,
    hipStream_t s) {
    if (!shape_ok(what, B, HW, C, G)) return;
    NNK_REQUIRE(valid_act(act), what, "%s: unknown activation %d", what, act);
    if (B == 0) return;
    NNK_REQUIRE(y && mu && rstd && x && shift && gamma && beta && ws, what, "%s: null pointer", what);
    NNK_REQUIRE(aligned16(x) && aligned16(y) && aligned16(gamma) && aligned16(beta) && aligned16(shift) &&
            aligned16(ws),
        what, "%s: pointers must be 16-byte aligned", what);
    NNK_REQUIRE(shift_fused(false, B, HW, C, G, act), what,
        "%s: [%d, %d, %d] G=%d, activation %d is not taken by the fused shift kernels "
        "(nnhip_groupnorm_shift_supported); add the shift with launch_spatial_add and call "
        "launch_groupnorm_act_forward_ws", what, B, HW, C, G, act);
    if (!run_stream(false, B, HW, C, G, ws, s, what, [&](float* w) {
            return nnk_gns_forward(act, y, mu, rstd, x, gamma, beta, shift, B, HW, C, G, eps, w, s);
        })) {
        nnk_set_error(hipErrorLaunchFailure, "%s: the persistent grid does not fit the device", what);
        return;
    }
    nnk_after_launch(what, s);
}

void gn_shift_backward_impl(const char* what, float* dx, float* gshift, float* ggamma, float* gbeta,
    const float* dy, const float* x, const float* shift, const float* gamma, const float* beta, const float* mu,
    const float* rstd, int B, int HW, int C, int G, int act, float* ws, hipStream_t s) {
    if (!shape_ok(what, B, HW, C, G)) return;
    NNK_REQUIRE(valid_act(act), what, "%s: unknown activation %d", what, act);
    NNK_REQUIRE(ggamma && gbeta && ws, what, "%s: null pointer", what);
    if (B == 0) {
        gn_backward_impl(what, dx, ggamma, gbeta, dy, x, gamma, beta, mu, rstd, B, HW, C, G, act, ws, s);
        return;
    }
    NNK_REQUIRE(dx && gshift && dy && x && shift && gamma && beta && mu && rstd, what, "%s: null pointer", what);
    NNK_REQUIRE(aligned16(x) && aligned16(dy) && aligned16(dx) && aligned16(gamma) && aligned16(beta) &&
            aligned16(shift) && aligned16(ws),
        what, "%s: pointers must be 16-byte aligned", what);
    NNK_REQUIRE(shift_fused(true, B, HW, C, G, act), what,
        "%s: [%d, %d, %d] G=%d, activation %d is not taken by the fused shift kernels "
        "(nnhip_groupnorm_shift_supported); call launch_groupnorm_act_backward_ws on x + shift and "
        "launch_spatial_reduce_sum_ws on its dx", what, B, HW, C, G, act);
    if (!run_stream(true, B, HW, C, G, ws, s, what, [&](float* w) {
            return nnk_gns_backward(act, dx, ggamma, gbeta, dy, x, gamma, beta, mu, rstd, shift, gshift, B, HW, C,
                G, w, s);
        })) {
        nnk_set_error(hipErrorLaunchFailure, "%s: the persistent grid does not fit the device", what);
        return;
    }
    nnk_after_launch(what, s);
}

}  // namespace

// Scratch of launch_groupnorm_act_backward_noalloc, for callers that cannot
// allocate.  A device global: each device the library runs on holds its own
// copy until the process ends; it is zero when the code object is loaded and
// written only by that entry point.  The first kNoAllocStreamBytes are the
// streaming kernels' workspace (header, epoch-tagged records and partials:
// the epoch lives in the header, so records left by earlier calls never match
// a later one and nothing needs clearing between calls); the rest holds the
// register and generic paths' untagged channel partials, apart, so that a
// streaming launch never reads them as records.
constexpr size_t kNoAllocStreamBytes = 12u << 20;
constexpr size_t kNoAllocPartialBytes = 4u << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocStreamBytes + kNoAllocPartialBytes];

namespace {
constexpr int kNoAllocDevices = 64;
std::mutex g_noalloc_mu;
float* g_noalloc_ptr[kNoAllocDevices] = {};  // address of `scratch` on each device

// The address of `scratch` on the device of stream s (the current device for
// the null stream), looked up once per device with that device current.
float* noalloc_scratch(hipStream_t s, const char* what) {
    int cur = -1, dev = -1;
    hipError_t e = hipGetDevice(&cur);
    if (e == hipSuccess) e = s ? hipStreamGetDevice(s, &dev) : hipGetDevice(&dev);
    if (e != hipSuccess || dev < 0 || dev >= kNoAllocDevices) {
        nnk_set_error(e != hipSuccess ? (int)e : (int)hipErrorInvalidDevice, "%s: no device for the stream", what);
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_noalloc_mu);
    if (!g_noalloc_ptr[dev]) {
        if (dev != cur && (e = hipSetDevice(dev)) != hipSuccess) {
            nnk_set_error((int)e, "%s: hipSetDevice(%d): %s", what, dev, hipGetErrorString(e));
            return nullptr;
        }
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (dev != cur) (void)hipSetDevice(cur);
        if (e != hipSuccess || !p) {
            nnk_set_error(e != hipSuccess ? (int)e : (int)hipErrorInvalidSymbol, "%s: scratch address: %s", what,
                hipGetErrorString(e));
            return nullptr;
        }
        g_noalloc_ptr[dev] = static_cast<float*>(p);
    }
    return g_noalloc_ptr[dev];
}
}  // namespace

extern "C" {

void launch_groupnorm_forward(float* y, float* mu, float* rstd, const float* x,
    const float* gamma, const float* beta, int batch, int HW, int C, int G, float eps,
    hipStream_t s) {
    gn_forward_impl("launch_groupnorm_forward", y, mu, rstd, x, gamma, beta, batch, HW, C, G,
        eps, ACT_IDENTITY, nullptr, s);
}

void launch_groupnorm_act_forward(float* y, float* mu, float* rstd, const float* x,
    const float* gamma, const float* beta, int batch, int HW, int C, int G, float eps,
    Activation act, hipStream_t s) {
    gn_forward_impl("launch_groupnorm_act_forward", y, mu, rstd, x, gamma, beta, batch, HW, C,
        G, eps, (int)act, nullptr, s);
}

void launch_groupnorm_act_forward_ws(float* y, float* mu, float* rstd, const float* x,
    const float* gamma, const float* beta, int batch, int HW, int C, int G, float eps,
    Activation act, float* workspace, hipStream_t s) {
    gn_forward_impl("launch_groupnorm_act_forward_ws", y, mu, rstd, x, gamma, beta, batch, HW, C,
        G, eps, (int)act, workspace, s);
}

size_t nnhip_groupnorm_forward_workspace(int batch, int HW, int C, int G) {
    const nnk::gns::Plan p = nnk::gns::make_plan(false, batch, HW, C, G);
    return p.ok ? p.ws_floats : 0;
}

int nnhip_groupnorm_workspace_status(const float* workspace) {
    if (!workspace) return 0;
    unsigned flag = 0;
    const hipError_t e = hipMemcpy(&flag, workspace, sizeof(flag), hipMemcpyDeviceToHost);
    if (e != hipSuccess) return -(int)e;
    return flag ? 1 : 0;
}

void launch_groupnorm_backward(float* dx, float* ggamma, float* gbeta, const float* dy,
    const float* x, const float* gamma, const float* mu, const float* rstd, int batch, int HW,
    int C, int G, hipStream_t s) {
    gn_backward_impl("launch_groupnorm_backward", dx, ggamma, gbeta, dy, x, gamma, nullptr, mu,
        rstd, batch, HW, C, G, ACT_IDENTITY, nullptr, s);
}

void launch_groupnorm_act_backward(float* dx, float* ggamma, float* gbeta, const float* dy,
    const float* x, const float* gamma, const float* beta, const float* mu, const float* rstd,
    int batch, int HW, int C, int G, Activation act, hipStream_t s) {
    gn_backward_impl("launch_groupnorm_act_backward", dx, ggamma, gbeta, dy, x, gamma, beta, mu,
        rstd, batch, HW, C, G, (int)act, nullptr, s);
}

void launch_groupnorm_act_backward_ws(float* dx, float* ggamma, float* gbeta, const float* dy,
    const float* x, const float* gamma, const float* beta, const float* mu, const float* rstd,
    int batch, int HW, int C, int G, Activation act, float* workspace, hipStream_t s) {
    if (!workspace) {
        nnk_set_error(hipErrorInvalidValue, "launch_groupnorm_act_backward_ws: null workspace");
        return;
    }
    gn_backward_impl("launch_groupnorm_act_backward_ws", dx, ggamma, gbeta, dy, x, gamma, beta,
        mu, rstd, batch, HW, C, G, (int)act, workspace, s);
}

void launch_groupnorm_act_backward_noalloc(float* dx, float* ggamma, float* gbeta, const float* dy,
    const float* x, const float* gamma, const float* beta, const float* mu, const float* rstd,
    int batch, int HW, int C, int G, Activation act, hipStream_t s) {
    const char* what = "launch_groupnorm_act_backward_noalloc";
    if (!shape_ok(what, batch, HW, C, G)) return;
    // The streaming kernels' workspace counts only when they will run; the
    // register and generic paths (also the streaming path's fallback) keep
    // their 2 * batch * C channel partials in the second region.
    const bool stream = batch > 0 && bwd_stream_selected(dx, dy, x, gamma, beta, batch, HW, C, G, (int)act);
    const size_t stream_bytes = stream ? reg_partials_offset(batch, HW, C, G) * sizeof(float) : 0;
    const size_t partial_bytes = (size_t)2 * batch * C * sizeof(float);
    NNK_REQUIRE(stream_bytes <= kNoAllocStreamBytes && partial_bytes <= kNoAllocPartialBytes, what,
        "%s: [%d, %d, %d] G=%d needs %zu + %zu bytes of scratch, more than its %zu + %zu (use "
        "launch_groupnorm_act_backward_ws with a workspace of nnhip_groupnorm_backward_workspace floats)",
        what, batch, HW, C, G, stream_bytes, partial_bytes, kNoAllocStreamBytes, kNoAllocPartialBytes);
    float* ws = noalloc_scratch(s, what);
    if (!ws) return;
    gn_backward_impl(what, dx, ggamma, gbeta, dy, x, gamma, beta, mu, rstd, batch, HW, C, G, (int)act, ws, s,
        ws + kNoAllocStreamBytes / sizeof(float));
}

size_t nnhip_groupnorm_backward_workspace(int batch, int HW, int C, int G) {
    if (batch <= 0 || C <= 0) return 0;
    return reg_partials_offset(batch, HW, C, G) + (size_t)2 * batch * C;
}

void launch_groupnorm_act_shift_forward_ws(float* y, float* mu, float* rstd, const float* x, const float* shift,
    const float* gamma, const float* beta, int batch, int HW, int C, int G, float eps, Activation act,
    float* workspace, hipStream_t s) {
    gn_shift_forward_impl("launch_groupnorm_act_shift_forward_ws", y, mu, rstd, x, shift, gamma, beta, batch, HW,
        C, G, eps, (int)act, workspace, s);
}

void launch_groupnorm_act_shift_backward_ws(float* dx, float* gshift, float* ggamma, float* gbeta,
    const float* dy, const float* x, const float* shift, const float* gamma, const float* beta, const float* mu,
    const float* rstd, int batch, int HW, int C, int G, Activation act, float* workspace, hipStream_t s) {
    gn_shift_backward_impl("launch_groupnorm_act_shift_backward_ws", dx, gshift, ggamma, gbeta, dy, x, shift,
        gamma, beta, mu, rstd, batch, HW, C, G, (int)act, workspace, s);
}

int nnhip_groupnorm_shift_supported(int batch, int HW, int C, int G, Activation act) {
    return (shift_fused(false, batch, HW, C, G, (int)act) ? 1 : 0) |
        (shift_fused(true, batch, HW, C, G, (int)act) ? 2 : 0);
}

size_t nnhip_groupnorm_shift_backward_workspace(int batch, int HW, int C, int G) {
    const size_t plain = nnhip_groupnorm_backward_workspace(batch, HW, C, G);
    const nnk::gns::Plan p = nnk::gns::make_plan(true, batch, HW, C, G);
    return p.ok && p.ws_shift_floats > plain ? p.ws_shift_floats : plain;
}

}  // extern "C"
