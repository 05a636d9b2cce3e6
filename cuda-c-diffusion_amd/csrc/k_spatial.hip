// k_spatial.hip -- per (sample, channel) broadcasts and reductions over NHWC
// tensors, the neighbours of GroupNorm+SiLU in the diffusion blocks:
//   spatial_add        x[b,hw,c] += v[b,c]              src/kernels.cu:1132-1142
//   spatial_reduce_sum out[b,c] = sum_hw x[b,hw,c]      src/kernels.cu:1145-1158
//   spatial_modulate   out = x * (cond[b,c] + 1)        src/kernels.cu:1055-1067
//   its backward       gin = gout * (cond + 1), gcond[b,c] = sum_hw gout * x
//                                                       src/kernels.cu:1070-1101
// and the fused pairs of the EDM block (src/cond_conv_residual.c:30-33, 46-49):
//   modulate + activation forward: out = act(x * (cond + 1))        (8 B/elem)
//   activation + modulate backward: g2 = gout * act'(x (cond + 1)),
//     gin = g2 (cond + 1), gcond = sum_hw g2 x                       (12 B/elem)
// replacing 16 and 32 B/elem of separate passes (the intermediate
// x * (cond + 1) is recomputed, never stored).
//
// Elementwise parts: one float4 per lane and four in flight per thread, the
// [B, C] vector read through the cache.  Every product is the reference's
// (m = cond + 1 first, then the product; the activation in its exact form),
// so these outputs are bit-identical to the reference's operation order.
//
// Reductions over HW: the reference walks HW serially in one thread per
// (b, c) (the pathological part).  Here workgroup (segment s, sample b) sums
// rows [s R, s R + R) of all channels: lanes over float4 columns, rows over
// the rest of the workgroup, eight rows in flight per lane; the row lanes
// are added in order in LDS and the segment partials, when there is more than
// one segment, by a second launch in segment order.  Fixed order throughout.
#include "nn_hip_rt.h"
#include "nnk_common.h"

namespace {

using namespace nnk;

constexpr int kTpb = 256;
constexpr int kUnroll = 1;  // one float4 per thread, one-shot grid (as k_elementwise.hip)

enum { kOpAdd = 0, kOpMod = 1 };

// x' = x + v (kOpAdd, in place: out may equal in) or act(x * (v + 1)) (kOpMod).
template <int OP, int ACT, bool NT>
__global__ __launch_bounds__(kTpb) void spatial_ew_vec(float* out, const float* in,
    const float* __restrict__ v, long long n4, FastDiv c4, FastDiv hwc4) {
    const long long stride = (long long)gridDim.x * kTpb * kUnroll;
    for (long long base = (long long)blockIdx.x * kTpb * kUnroll + threadIdx.x; base < n4; base += stride) {
        float4 x[kUnroll], w[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const long long i = base + u * kTpb;
            if (i < n4) {
                uint32_t b, r, q, c;
                hwc4.divmod((uint32_t)i, b, r);
                c4.divmod(r, q, c);
                x[u] = ldS<NT>(in + 4 * i);
                w[u] = ld4(v + ((size_t)b * c4.d + c) * 4);
            }
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const long long i = base + u * kTpb;
            if (i < n4) {
                float4 o;
                if constexpr (OP == kOpAdd) {
                    o.x = x[u].x + w[u].x;
                    o.y = x[u].y + w[u].y;
                    o.z = x[u].z + w[u].z;
                    o.w = x[u].w + w[u].w;
                } else {
                    o.x = act_fwd<ACT, false>(x[u].x * (w[u].x + 1.0f));
                    o.y = act_fwd<ACT, false>(x[u].y * (w[u].y + 1.0f));
                    o.z = act_fwd<ACT, false>(x[u].z * (w[u].z + 1.0f));
                    o.w = act_fwd<ACT, false>(x[u].w * (w[u].w + 1.0f));
                }
                stS<NT>(out + 4 * i, o);
            }
        }
    }
}

// Scalar form for C % 4 != 0 or unaligned pointers.
template <int OP, int ACT>
__global__ __launch_bounds__(kTpb) void spatial_ew_scalar(float* out, const float* in,
    const float* __restrict__ v, long long n, FastDiv cdiv, FastDiv hwc) {
    for (long long i = (long long)blockIdx.x * kTpb + threadIdx.x; i < n; i += (long long)gridDim.x * kTpb) {
        uint32_t b, r, q, c;
        hwc.divmod((uint32_t)i, b, r);
        cdiv.divmod(r, q, c);
        const float w = v[(size_t)b * cdiv.d + c];
        if constexpr (OP == kOpAdd) out[i] = in[i] + w;
        else out[i] = act_fwd<ACT, false>(in[i] * (w + 1.0f));
    }
}

// Reduction modes: what a row element contributes and what it writes.
enum { kRedSum = 0, kRedModBwd = 1 };

// Workgroup b S + s: rows [s R, min(HW, s R + R)) of sample b.  Lane layout:
// CL lanes over the VW-float column units (a power of two <= 64), RP = kTpb / CL
// row lanes.  part[(b S + s) C + c] receives the segment sum of channel c.
template <int MODE, int ACT, int VW, bool NT, int TPB = kTpb>
__global__ __launch_bounds__(TPB) void spatial_reduce(float* __restrict__ part, float* __restrict__ gin,
    const float* __restrict__ gout, const float* __restrict__ x, const float* __restrict__ cond, int HW, int C,
    int S, int R, int CL) {
    typedef float vec __attribute__((ext_vector_type(VW)));
    __shared__ vec red[TPB];
    const int b = blockIdx.x / S, s = blockIdx.x % S;
    const int lc = threadIdx.x % CL, lr = threadIdx.x / CL, RP = TPB / CL;
    const int CU = C / VW;  // column units per row
    const int r0 = s * R, r1 = min(HW, r0 + R);
    const size_t sample = (size_t)b * HW * C;
    for (int cu0 = 0; cu0 < CU; cu0 += CL) {
        const int cu = cu0 + lc;
        vec acc = {};
        if (cu < CU) {
            vec m = {};
            if constexpr (MODE == kRedModBwd) {
                m = *reinterpret_cast<const vec*>(cond + (size_t)b * C + cu * VW);
                m = m + 1.0f;
            }
            auto elem = [&](int r) {
                const size_t k = sample + (size_t)r * C + cu * VW;
                if constexpr (MODE == kRedSum) {
                    return NT ? __builtin_nontemporal_load(reinterpret_cast<const vec*>(gout + k))
                              : *reinterpret_cast<const vec*>(gout + k);
                } else {
                    const vec g = NT ? __builtin_nontemporal_load(reinterpret_cast<const vec*>(gout + k))
                                     : *reinterpret_cast<const vec*>(gout + k);
                    const vec xv = NT ? __builtin_nontemporal_load(reinterpret_cast<const vec*>(x + k))
                                      : *reinterpret_cast<const vec*>(x + k);
                    vec g2;
#pragma unroll
                    for (int j = 0; j < VW; ++j) g2[j] = g[j] * act_grad<ACT, false>(xv[j] * m[j]);
                    const vec gi = g2 * m;
                    if constexpr (NT) __builtin_nontemporal_store(gi, reinterpret_cast<vec*>(gin + k));
                    else *reinterpret_cast<vec*>(gin + k) = gi;
                    return g2 * xv;
                }
            };
            int r = r0 + lr;
            constexpr int kRows = 8;
            if constexpr (TPB == 1024 && MODE == kRedModBwd) {
                // one workgroup per sample, rows in batches of kP per lane,
                // double-buffered: the next batch's loads are issued before
                // the current batch's activation gradient, so with one
                // workgroup per CU the arithmetic overlaps the memory traffic
                // (the schedule barriers keep the compiler from sinking those
                // loads below the current batch's stores of gin).  Rows are
                // added in the same order as one row at a time.
                constexpr int kP = 4;
                const int step = kP * RP;
                auto load_batch = [&](vec (&gv)[kP], vec (&xv)[kP], int rr) {
#pragma unroll
                    for (int u = 0; u < kP; ++u) {
                        const size_t k = sample + (size_t)(rr + u * RP) * C + cu * VW;
                        gv[u] = NT ? __builtin_nontemporal_load(reinterpret_cast<const vec*>(gout + k))
                                   : *reinterpret_cast<const vec*>(gout + k);
                        xv[u] = NT ? __builtin_nontemporal_load(reinterpret_cast<const vec*>(x + k))
                                   : *reinterpret_cast<const vec*>(x + k);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                };
                auto use_batch = [&](const vec (&gv)[kP], const vec (&xv)[kP], int rr) {
#pragma unroll
                    for (int u = 0; u < kP; ++u) {
                        const size_t k = sample + (size_t)(rr + u * RP) * C + cu * VW;
                        vec g2;
#pragma unroll
                        for (int j = 0; j < VW; ++j) g2[j] = gv[u][j] * act_grad<ACT, false>(xv[u][j] * m[j]);
                        const vec gi = g2 * m;
                        if constexpr (NT) __builtin_nontemporal_store(gi, reinterpret_cast<vec*>(gin + k));
                        else *reinterpret_cast<vec*>(gin + k) = gi;
                        acc += g2 * xv[u];
                    }
                    __builtin_amdgcn_sched_barrier(0);
                };
                if (r + (kP - 1) * RP < r1) {
                    vec ga[kP], xa[kP], gb[kP], xb[kP];
                    load_batch(ga, xa, r);
                    for (;;) {
                        const int ra = r + step;  // the batch after the one in (ga, xa)
                        const bool more_a = ra + (kP - 1) * RP < r1;
                        if (more_a) load_batch(gb, xb, ra);
                        use_batch(ga, xa, r);
                        r = ra;
                        if (!more_a) break;
                        const int rb = r + step;  // the batch after the one in (gb, xb)
                        const bool more_b = rb + (kP - 1) * RP < r1;
                        if (more_b) load_batch(ga, xa, rb);
                        use_batch(gb, xb, r);
                        r = rb;
                        if (!more_b) break;
                    }
                }
            } else {
                for (; r + (kRows - 1) * RP < r1; r += kRows * RP) {
                    vec t[kRows];
#pragma unroll
                    for (int u = 0; u < kRows; ++u) t[u] = elem(r + u * RP);
#pragma unroll
                    for (int u = 0; u < kRows; ++u) acc += t[u];
                }
            }
            for (; r < r1; r += RP) acc += elem(r);
        }
        red[threadIdx.x] = acc;
        __syncthreads();
        if (lr == 0 && cu < CU) {
            vec t = red[lc];
            for (int k = 1; k < RP; ++k) t += red[k * CL + lc];
            *reinterpret_cast<vec*>(part + ((size_t)b * S + s) * C + cu * VW) = t;
        }
        __syncthreads();
    }
}

// out[b, c] = part[b, 0, c] + part[b, 1, c] + ... (segment order).
__global__ __launch_bounds__(kTpb) void spatial_segments_sum(float* __restrict__ out,
    const float* __restrict__ part, int B, int S, int C) {
    const long long i = (long long)blockIdx.x * kTpb + threadIdx.x;
    if (i >= (long long)B * C) return;
    const long long b = i / C, c = i % C;
    const float* p = part + b * S * C + c;
    // kB segments in flight (a short last batch too: predicated loads, not a
    // loop of one load each), added in segment order from the first
    constexpr int kB = 16;
    float t = 0.0f;
    for (int s = 0; s < S; s += kB) {
        float v[kB];
#pragma unroll
        for (int u = 0; u < kB; ++u) v[u] = s + u < S ? p[(size_t)(s + u) * C] : 0.0f;
#pragma unroll
        for (int u = 0; u < kB; ++u)
            if (s + u < S) t = s + u == 0 ? v[0] : t + v[u];
    }
    out[i] = t;
}

bool shape_ok(const char* what, int B, int HW, int C) {
    NNK_REQUIRE_RET(B >= 0 && HW >= 0 && C >= 0, false, what, "%s: bad shape B=%d HW=%d C=%d", what, B, HW, C);
    NNK_REQUIRE_RET((long long)B * HW * C < (1LL << 31), false, what,
        "%s: %lld elements exceed the 32-bit index range", what, (long long)B * HW * C);
    return true;
}

// One-shot grid (the kernels keep a grid-stride loop, so any grid is correct).
unsigned ew_grid(long long units, int per_block) {
    long long g = (units + per_block - 1) / per_block;
    if (g > (1LL << 30)) g = 1LL << 30;
    return (unsigned)(g < 1 ? 1 : g);
}

// Elementwise launcher: out = x + v (OP add) or act(x * (v + 1)).
template <int OP>
void launch_ew(const char* what, float* out, const float* in, const float* v, int B, int HW, int C, int act,
    hipStream_t s) {
    if (!shape_ok(what, B, HW, C)) return;
    const long long n = (long long)B * HW * C;
    if (n == 0) return;
    NNK_REQUIRE(out && in && v, what, "%s: null pointer", what);
    const bool vec = C % 4 == 0 && aligned16(out) && aligned16(in) && aligned16(v);
    const bool nt = use_nt(8LL * n);
    bool ok;
    if (vec) {
        const long long n4 = n / 4;
        const FastDiv c4((uint32_t)(C / 4)), hwc4((uint32_t)((long long)HW * C / 4));
        const unsigned g = ew_grid(n4, kTpb * kUnroll);
        ok = NNK_ACT_DISPATCH(act, A, {
            if (nt) spatial_ew_vec<OP, A, true><<<g, kTpb, 0, s>>>(out, in, v, n4, c4, hwc4);
            else spatial_ew_vec<OP, A, false><<<g, kTpb, 0, s>>>(out, in, v, n4, c4, hwc4);
        });
    } else {
        const FastDiv cd((uint32_t)C), hwc((uint32_t)((long long)HW * C));
        const unsigned g = ew_grid(n, kTpb);
        ok = NNK_ACT_DISPATCH(act, A, { spatial_ew_scalar<OP, A><<<g, kTpb, 0, s>>>(out, in, v, n, cd, hwc); });
    }
    NNK_REQUIRE(ok, what, "%s: unknown activation %d", what, act);
    nnk_after_launch(what, s);
}

// Reduction plan: segments per sample and rows per segment.
struct RedPlan {
    int VW, CL, S, R, TPB;
};

// One 1024-thread workgroup per sample when there are enough samples to give
// every CU of the device (256 on MI355X) one and each is large: same-box A/B
// of the modulate backward at [256, 4096, 64] and [256, 1024, 256]: 146.6 and
// 146.1 us against 162.7 and 162.1 us segmented.  At [256, 1024, 128] (131K
// elements a sample) it was 5 % slower, and at 128 samples (half the CUs) 20 %.
constexpr int kBigBatch = 256;
constexpr long long kBigSample = 1 << 18;

RedPlan red_plan(int B, int HW, int C, bool vec) {
    RedPlan p;
    p.VW = vec ? 4 : 1;
    const int CU = C / p.VW;
    p.CL = 1;
    while (p.CL * 2 <= CU && p.CL * 2 <= 64) p.CL *= 2;
    if (vec && B >= kBigBatch && (long long)HW * C >= kBigSample && HW >= 8 * (1024 / p.CL)) {
        // one workgroup per sample: no segment partials, no second launch
        p.TPB = 1024;
        p.S = 1;
        p.R = HW;
        return p;
    }
    p.TPB = kTpb;
    const int RP = kTpb / p.CL;
    // enough workgroups to fill the device (~2048), segments of >= 8 row passes
    int S = (2048 + B - 1) / (B > 0 ? B : 1);
    const int smax = (HW + 8 * RP - 1) / (8 * RP);
    if (S > smax) S = smax;
    if (S < 1) S = 1;
    p.R = (HW + S - 1) / S;
    p.S = HW > 0 ? (HW + p.R - 1) / p.R : 1;
    return p;
}

size_t red_workspace(const RedPlan& p, int B, int C) { return p.S > 1 ? (size_t)B * p.S * C : 0; }

// An upper bound of b * S over every batch b <= B (S = the plan's segments):
// S <= ceil(2048 / b) and S <= smax, so b S <= min(b smax, 2047 + b), which
// grows with b.  (b S itself does not: 102 ceil(2048 / 102) = 2142 >
// 103 ceil(2048 / 103) = 2060.)  A workspace sized with it for a batch
// therefore serves every smaller batch of the same HW and C.
long long red_rows_bound(int B, int HW, int C, bool vec) {
    const int CU = C / (vec ? 4 : 1);
    int CL = 1;
    while (CL * 2 <= CU && CL * 2 <= 64) CL *= 2;
    const long long RP = kTpb / CL;
    const long long smax = (HW + 8 * RP - 1) / (8 * RP);
    const long long a = (long long)B * (smax > 1 ? smax : 1), c = 2047LL + B;
    return a < c ? a : c;
}

// Reductions: out[b, c] = sum over HW of (x) [kRedSum] or of (g2 x) with
// gin = g2 (cond + 1) [kRedModBwd].  ws: caller workspace or null (scratch).
template <int MODE>
void launch_red(const char* what, float* out, float* gin, const float* gout, const float* x, const float* cond,
    int B, int HW, int C, int act, float* ws, hipStream_t s) {
    if (!shape_ok(what, B, HW, C)) return;
    if ((long long)B * C == 0) return;
    NNK_REQUIRE(out && gout, what, "%s: null pointer", what);
    if constexpr (MODE == kRedModBwd) NNK_REQUIRE(gin && x && cond, what, "%s: null pointer", what);
    bool vec = C % 4 == 0 && aligned16(out) && aligned16(gout);
    if constexpr (MODE == kRedModBwd) vec = vec && aligned16(gin) && aligned16(x) && aligned16(cond);
    const RedPlan p = red_plan(B, HW, C, vec);
    const size_t need = red_workspace(p, B, C);
    float* part = out;
    bool pooled = false;
    if (need) {
        if (ws) {
            part = ws;
        } else {
            part = nnk_scratch_acquire(need, s, what);
            if (!part) return;
            pooled = true;
        }
        if (vec) NNK_REQUIRE(aligned16(part), what, "%s: workspace must be 16-byte aligned", what);
    }
    const long long bytes = (MODE == kRedSum ? 4LL : 12LL) * B * HW * C;
    const bool nt = use_nt(bytes);
    const dim3 grid((unsigned)((long long)p.S * B));
    bool ok;
#define NNK_RED(VW_)                                                                                           \
    ok = NNK_ACT_DISPATCH(act, A, {                                                                            \
        if (p.TPB == 1024) {                                                                                   \
            if (nt) spatial_reduce<MODE, A, VW_, true, 1024><<<grid, 1024, 0, s>>>(part, gin, gout, x, cond, HW, \
                C, p.S, p.R, p.CL);                                                                            \
            else spatial_reduce<MODE, A, VW_, false, 1024><<<grid, 1024, 0, s>>>(part, gin, gout, x, cond, HW,  \
                C, p.S, p.R, p.CL);                                                                            \
        } else if (nt) spatial_reduce<MODE, A, VW_, true><<<grid, kTpb, 0, s>>>(part, gin, gout, x, cond, HW, C, \
            p.S, p.R, p.CL);                                                                                   \
        else spatial_reduce<MODE, A, VW_, false><<<grid, kTpb, 0, s>>>(part, gin, gout, x, cond, HW, C, p.S,   \
            p.R, p.CL);                                                                                        \
    })
    if (HW == 0) {
        // empty sums: zero gradients (the reference writes 0 for each (b, c))
        nnhip_fill_f32(out, 0.0f, (size_t)B * C, s);
        ok = true;
    } else if (p.VW == 4) {
        NNK_RED(4);
    } else {
        NNK_RED(1);
    }
#undef NNK_RED
    if (ok && HW > 0 && p.S > 1) {
        const long long nbc = (long long)B * C;
        spatial_segments_sum<<<(unsigned)((nbc + kTpb - 1) / kTpb), kTpb, 0, s>>>(out, part, B, p.S, C);
    }
    if (pooled) nnk_scratch_release(part, s);
    NNK_REQUIRE(ok, what, "%s: unknown activation %d", what, act);
    nnk_after_launch(what, s);
}

}  // namespace

extern "C" {

void launch_spatial_add(float* inout, const float* bias, int batch, int H, int W, int C, hipStream_t s) {
    launch_ew<kOpAdd>("launch_spatial_add", inout, inout, bias, batch, H * W, C, ACT_IDENTITY, s);
}

void launch_spatial_reduce_sum(float* out, const float* in, int batch, int HW, int C, hipStream_t s) {
    launch_red<kRedSum>("launch_spatial_reduce_sum", out, nullptr, in, nullptr, nullptr, batch, HW, C,
        ACT_IDENTITY, nullptr, s);
}

void launch_spatial_modulate(float* out, const float* in, const float* cond, int batch, int H, int W, int C,
    hipStream_t s) {
    launch_ew<kOpMod>("launch_spatial_modulate", out, in, cond, batch, H * W, C, ACT_IDENTITY, s);
}

void launch_spatial_modulate_backward(float* grad_in, float* grad_cond, const float* grad_out, const float* in,
    const float* cond, int batch, int H, int W, int C, hipStream_t s) {
    launch_red<kRedModBwd>("launch_spatial_modulate_backward", grad_cond, grad_in, grad_out, in, cond, batch,
        H * W, C, ACT_IDENTITY, nullptr, s);
}

void launch_spatial_modulate_act_forward(float* out, const float* in, const float* cond, int batch, int H,
    int W, int C, Activation act, hipStream_t s) {
    launch_ew<kOpMod>("launch_spatial_modulate_act_forward", out, in, cond, batch, H * W, C, (int)act, s);
}

void launch_spatial_modulate_act_backward(float* grad_in, float* grad_cond, const float* grad_out,
    const float* in, const float* cond, int batch, int H, int W, int C, Activation act, float* workspace,
    hipStream_t s) {
    launch_red<kRedModBwd>("launch_spatial_modulate_act_backward", grad_cond, grad_in, grad_out, in, cond,
        batch, H * W, C, (int)act, workspace, s);
}

void launch_spatial_reduce_sum_ws(float* out, const float* in, int batch, int HW, int C, float* workspace,
    hipStream_t s) {
    launch_red<kRedSum>("launch_spatial_reduce_sum_ws", out, nullptr, in, nullptr, nullptr, batch, HW, C,
        ACT_IDENTITY, workspace, s);
}

size_t nnhip_spatial_reduce_workspace(int batch, int HW, int C) {
    if (batch <= 0 || HW <= 0 || C <= 0) return 0;
    // Both layouts (vector and scalar) and every batch up to `batch` (callers
    // size the workspace for their largest batch).  A bound of `batch` rows
    // means one segment per sample at every batch: no workspace.
    const long long rv = red_rows_bound(batch, HW, C, true), rs = red_rows_bound(batch, HW, C, false);
    const long long rows = rv > rs ? rv : rs;
    return rows <= batch ? 0 : (size_t)rows * C;
}

}  // extern "C"
