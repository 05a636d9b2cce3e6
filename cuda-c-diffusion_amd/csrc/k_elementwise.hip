// k_elementwise.hip -- streaming elementwise kernels of the launch layer:
// activations, weighted sum / mp_sum, scale by a device scalar, SGD, add_bias,
// bias_grad, mp_cat and the NHWC mp channel cat/split.
//
// Streaming shape: 256 threads, each thread moves 4 float4 spaced 256 apart,
// so a wave touches 1 KB contiguous per access; a scalar tail covers n % 4.
// Launches touching at least kNtBytes stream their tensors with nontemporal
// loads and stores (NT = true; see use_nt); per-channel vectors that are
// re-read (bias) always use ordinary loads.
// When any pointer is not 16-byte aligned the same kernels run in a scalar
// shape (one float per slot).  All bandwidth-bound: bytes per element are
// stated per kernel.
#include "nnk_common.h"

namespace {

using namespace nnk;

// One float4 per thread and one-shot workgroups: measured at 1 GiB per tensor,
// this streams 1-read/1-write at 0.79-0.83 of the HBM peak against 0.70-0.77
// with four float4 per thread, and a grid-stride loop over a capped grid was
// slower still (0.57-0.70): new workgroups are dispatched in address order,
// which keeps the set of open DRAM pages small.
constexpr int kTpb = 256;
constexpr int kUnroll = 1;
constexpr long long kPerBlock = (long long)kTpb * kUnroll;

inline unsigned blocks_for(long long units) {
    long long b = (units + kPerBlock - 1) / kPerBlock;
    return (unsigned)(b > 0 ? b : 1);
}

// Apply `op(i4)` to float4 slot i4 < n4 and `tail(i)` to elements 4*n4 + t.
template <typename Vec, typename Tail>
__device__ __forceinline__ void stream_loop(long long n4, long long n, Vec op, Tail tail) {
    const long long base = (long long)blockIdx.x * kPerBlock + threadIdx.x;
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const long long q = base + (long long)u * kTpb;
        if (q < n4) op(q);
    }
    if (blockIdx.x == 0 && threadIdx.x < n - 4 * n4) tail(4 * n4 + threadIdx.x);
}

// ---------------- activations: fwd 8 B/elem, bwd 12 B/elem ----------------
// Exact Pade form (correctly rounded quotient, no contraction): these kernels
// are HBM-bound, so the exact arithmetic costs nothing measurable.
template <int ACT, bool VEC, bool NT>
__global__ __launch_bounds__(kTpb) void act_fwd_kernel(float* __restrict__ out,
    const float* __restrict__ in, long long n) {
    if constexpr (VEC) {
        stream_loop(n / 4, n,
            [&](long long q) {
                float4 v = ldS<NT>(in + 4 * q);
                v.x = act_fwd<ACT, false>(v.x);
                v.y = act_fwd<ACT, false>(v.y);
                v.z = act_fwd<ACT, false>(v.z);
                v.w = act_fwd<ACT, false>(v.w);
                stS<NT>(out + 4 * q, v);
            },
            [&](long long i) { out[i] = act_fwd<ACT, false>(in[i]); });
    } else {
        const long long base = (long long)blockIdx.x * kPerBlock + threadIdx.x;
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const long long i = base + (long long)u * kTpb;
            if (i < n) out[i] = act_fwd<ACT, false>(in[i]);
        }
    }
}

template <int ACT, bool VEC, bool NT>
__global__ __launch_bounds__(kTpb) void act_bwd_kernel(float* __restrict__ gin,
    const float* __restrict__ gout, const float* __restrict__ in, long long n) {
    if constexpr (VEC) {
        stream_loop(n / 4, n,
            [&](long long q) {
                const float4 z = ldS<NT>(in + 4 * q);
                float4 g = ldS<NT>(gout + 4 * q);
                g.x = g.x * act_grad<ACT, false>(z.x);
                g.y = g.y * act_grad<ACT, false>(z.y);
                g.z = g.z * act_grad<ACT, false>(z.z);
                g.w = g.w * act_grad<ACT, false>(z.w);
                stS<NT>(gin + 4 * q, g);
            },
            [&](long long i) { gin[i] = gout[i] * act_grad<ACT, false>(in[i]); });
    } else {
        const long long base = (long long)blockIdx.x * kPerBlock + threadIdx.x;
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const long long i = base + (long long)u * kTpb;
            if (i < n) gin[i] = gout[i] * act_grad<ACT, false>(in[i]);
        }
    }
}

// ---------------- out = wa*a + wb*b: 12 B/elem ----------------
template <bool VEC, bool NT>
__global__ __launch_bounds__(kTpb) void weighted_sum_kernel(float* out, const float* a,
    const float* b, float wa, float wb, long long n) {
    // out may alias a or b (EMA updates shadow in place): no __restrict__.
    if constexpr (VEC) {
        stream_loop(n / 4, n,
            [&](long long q) {
                const float4 x = ldS<NT>(a + 4 * q);
                const float4 y = ldS<NT>(b + 4 * q);
                float4 o;
                o.x = wa * x.x + wb * y.x;
                o.y = wa * x.y + wb * y.y;
                o.z = wa * x.z + wb * y.z;
                o.w = wa * x.w + wb * y.w;
                stS<NT>(out + 4 * q, o);
            },
            [&](long long i) { out[i] = wa * a[i] + wb * b[i]; });
    } else {
        const long long base = (long long)blockIdx.x * kPerBlock + threadIdx.x;
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const long long i = base + (long long)u * kTpb;
            if (i < n) out[i] = wa * a[i] + wb * b[i];
        }
    }
}

// ---------------- x *= s[0]: 8 B/elem ----------------
template <bool VEC, bool NT>
__global__ __launch_bounds__(kTpb) void scale_kernel(float* __restrict__ x,
    const float* __restrict__ s, long long n) {
    const float v = s[0];
    if constexpr (VEC) {
        stream_loop(n / 4, n,
            [&](long long q) {
                float4 t = ldS<NT>(x + 4 * q);
                t.x *= v;
                t.y *= v;
                t.z *= v;
                t.w *= v;
                stS<NT>(x + 4 * q, t);
            },
            [&](long long i) { x[i] *= v; });
    } else {
        const long long base = (long long)blockIdx.x * kPerBlock + threadIdx.x;
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const long long i = base + (long long)u * kTpb;
            if (i < n) x[i] *= v;
        }
    }
}

// ---------------- p -= lr*g: 12 B/elem ----------------
template <bool VEC, bool NT>
__global__ __launch_bounds__(kTpb) void sgd_kernel(float* __restrict__ p,
    const float* __restrict__ g, float lr, long long n) {
    if constexpr (VEC) {
        stream_loop(n / 4, n,
            [&](long long q) {
                float4 t = ldS<NT>(p + 4 * q);
                const float4 d = ldS<NT>(g + 4 * q);
                t.x -= lr * d.x;
                t.y -= lr * d.y;
                t.z -= lr * d.z;
                t.w -= lr * d.w;
                stS<NT>(p + 4 * q, t);
            },
            [&](long long i) { p[i] -= lr * g[i]; });
    } else {
        const long long base = (long long)blockIdx.x * kPerBlock + threadIdx.x;
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const long long i = base + (long long)u * kTpb;
            if (i < n) p[i] -= lr * g[i];
        }
    }
}

// ---------------- Y[m,n] += b[n]: 8 B/elem ----------------
__global__ __launch_bounds__(kTpb) void add_bias_kernel(float* __restrict__ Y,
    const float* __restrict__ bias, long long total, FastDiv divN) {
    const long long base = (long long)blockIdx.x * kPerBlock + threadIdx.x;
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const long long i = base + (long long)u * kTpb;
        if (i < total) {
            // total < 2^31 is checked by the launcher
            const uint32_t c = (uint32_t)i - divN.div((uint32_t)i) * divN.d;
            Y[i] += bias[c];
        }
    }
}

template <bool NT>
__global__ __launch_bounds__(kTpb) void add_bias_vec_kernel(float* __restrict__ Y,
    const float* __restrict__ bias, long long total4, FastDiv divN4) {
    const long long base = (long long)blockIdx.x * kPerBlock + threadIdx.x;
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const long long q = base + (long long)u * kTpb;
        if (q < total4) {
            const uint32_t c4 = (uint32_t)q - divN4.div((uint32_t)q) * divN4.d;
            float4 y = ldS<NT>(Y + 4 * q);
            const float4 bb = ld4(bias + 4 * c4);
            y.x += bb.x;
            y.y += bb.y;
            y.z += bb.z;
            y.w += bb.w;
            stS<NT>(Y + 4 * q, y);
        }
    }
}

// ---------------- bias_grad: gb[n] = sum_r g[r,n] ----------------
// Stage 1: grid (ceil(N/64), chunks); lanes walk 64 consecutive columns
// (coalesced), 4 waves split the chunk's rows.  part[chunk*N + n].
constexpr int kBgRows = 256;
__global__ __launch_bounds__(kTpb) void bias_grad_partial(float* __restrict__ part,
    const float* __restrict__ g, int rows, int N) {
    __shared__ float l[4][kWave];
    const int lane = threadIdx.x & (kWave - 1);
    const int wid = threadIdx.x / kWave;
    const int n = blockIdx.x * kWave + lane;
    const int r0 = blockIdx.y * kBgRows;
    const int r1 = min(rows, r0 + kBgRows);
    float s = 0.0f;
    if (n < N)
        for (int r = r0 + wid; r < r1; r += 4) s += g[(size_t)r * N + n];
    l[wid][lane] = s;
    __syncthreads();
    if (wid == 0 && n < N) part[(size_t)blockIdx.y * N + n] = ((l[0][lane] + l[1][lane]) + l[2][lane]) + l[3][lane];
}

__global__ __launch_bounds__(kTpb) void fill_kernel(float* __restrict__ p, float v, int n) {
    const int i = blockIdx.x * kTpb + threadIdx.x;
    if (i < n) p[i] = v;
}

__global__ __launch_bounds__(kTpb) void bias_grad_final(float* __restrict__ gb,
    const float* __restrict__ part, int chunks, int N) {
    const int n = blockIdx.x * kTpb + threadIdx.x;
    if (n >= N) return;
    float s = 0.0f;
    for (int c = 0; c < chunks; ++c) s += part[(size_t)c * N + n];
    gb[n] = s;
}

// ---------------- mp_cat / mp channel cat: 8 B/out-elem ----------------
// out[r, c] = c < Na ? wa*a[r*Na + c] : wb*b[r*Nb + c - Na]
__global__ __launch_bounds__(kTpb) void mp_cat_kernel(float* __restrict__ out,
    const float* __restrict__ a, const float* __restrict__ b, float wa, float wb,
    long long total, int Na, int Nb, FastDiv divN) {
    const long long base = (long long)blockIdx.x * kPerBlock + threadIdx.x;
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const long long i = base + (long long)u * kTpb;
        if (i < total) {
            uint32_t r, c;
            divN.divmod((uint32_t)i, r, c);
            out[i] = (int)c < Na ? wa * a[(size_t)r * Na + c] : wb * b[(size_t)r * Nb + (c - Na)];
        }
    }
}

// float4 form: Na, Nb multiples of 4, all pointers 16-byte aligned.
template <bool NT>
__global__ __launch_bounds__(kTpb) void mp_cat_vec_kernel(float* __restrict__ out,
    const float* __restrict__ a, const float* __restrict__ b, float wa, float wb,
    long long total4, int Na4, int Nb4, FastDiv divN4) {
    const long long base = (long long)blockIdx.x * kPerBlock + threadIdx.x;
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const long long q = base + (long long)u * kTpb;
        if (q < total4) {
            uint32_t r, c4;
            divN4.divmod((uint32_t)q, r, c4);
            float4 v;
            float w;
            if ((int)c4 < Na4) {
                v = ldS<NT>(a + 4 * ((size_t)r * Na4 + c4));
                w = wa;
            } else {
                v = ldS<NT>(b + 4 * ((size_t)r * Nb4 + (c4 - Na4)));
                w = wb;
            }
            v.x *= w;
            v.y *= w;
            v.z *= w;
            v.w *= w;
            stS<NT>(out + 4 * q, v);
        }
    }
}

// Backward: ga[r, c] = wa*g[r, c] (c < Ca), gb[r, c-Ca] = wb*g[r, c].
__global__ __launch_bounds__(kTpb) void mp_split_kernel(float* __restrict__ ga,
    float* __restrict__ gb, const float* __restrict__ g, float wa, float wb, long long total,
    int Ca, int Cb, FastDiv divN) {
    const long long base = (long long)blockIdx.x * kPerBlock + threadIdx.x;
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const long long i = base + (long long)u * kTpb;
        if (i < total) {
            uint32_t r, c;
            divN.divmod((uint32_t)i, r, c);
            if ((int)c < Ca) ga[(size_t)r * Ca + c] = wa * g[i];
            else gb[(size_t)r * Cb + (c - Ca)] = wb * g[i];
        }
    }
}

template <bool NT>
__global__ __launch_bounds__(kTpb) void mp_split_vec_kernel(float* __restrict__ ga,
    float* __restrict__ gb, const float* __restrict__ g, float wa, float wb, long long total4,
    int Ca4, int Cb4, FastDiv divN4) {
    const long long base = (long long)blockIdx.x * kPerBlock + threadIdx.x;
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const long long q = base + (long long)u * kTpb;
        if (q < total4) {
            uint32_t r, c4;
            divN4.divmod((uint32_t)q, r, c4);
            float4 v = ldS<NT>(g + 4 * q);
            if ((int)c4 < Ca4) {
                v.x *= wa;
                v.y *= wa;
                v.z *= wa;
                v.w *= wa;
                stS<NT>(ga + 4 * ((size_t)r * Ca4 + c4), v);
            } else {
                v.x *= wb;
                v.y *= wb;
                v.z *= wb;
                v.w *= wb;
                stS<NT>(gb + 4 * ((size_t)r * Cb4 + (c4 - Ca4)), v);
            }
        }
    }
}

// Host-side magnitude-preserving weights, in float as the reference computes
// them (src/kernels.cu:363-364 and 1251-1257).
void mp_sum_weights(float t, float* wa, float* wb) {
    const float d = sqrtf((1.0f - t) * (1.0f - t) + t * t);
    *wa = (1.0f - t) / d;
    *wb = t / d;
}

void mp_cat_weights(float t, int Na, int Nb, float* wa, float* wb) {
    const float denom = (1.0f - t) * (1.0f - t) + t * t;
    const float Cs = sqrtf((float)(Na + Nb) / denom);
    *wa = Cs / sqrtf((float)Na) * (1.0f - t);
    *wb = Cs / sqrtf((float)Nb) * t;
}

bool fits_i32(long long v) { return v >= 0 && v < (1LL << 31); }

void mp_cat_impl(const char* what, float* out, const float* a, const float* b, float wa,
    float wb, int rows, int Na, int Nb, hipStream_t s) {
    NNK_REQUIRE(rows >= 0 && Na > 0 && Nb > 0, what, "%s: bad shape rows=%d Na=%d Nb=%d", what, rows, Na, Nb);
    const long long total = (long long)rows * (Na + Nb);
    NNK_REQUIRE(fits_i32(total), what, "%s: %lld elements exceed 2^31", what, total);
    if (total == 0) return;
    NNK_REQUIRE(out && a && b, what, "%s: null pointer", what);
    if (Na % 4 == 0 && Nb % 4 == 0 && aligned16(out) && aligned16(a) && aligned16(b)) {
        const long long total4 = total / 4;
        if (use_nt(8 * total))
            mp_cat_vec_kernel<true><<<blocks_for(total4), kTpb, 0, s>>>(out, a, b, wa, wb, total4, Na / 4,
                Nb / 4, FastDiv((uint32_t)((Na + Nb) / 4)));
        else
            mp_cat_vec_kernel<false><<<blocks_for(total4), kTpb, 0, s>>>(out, a, b, wa, wb, total4, Na / 4,
                Nb / 4, FastDiv((uint32_t)((Na + Nb) / 4)));
    } else {
        mp_cat_kernel<<<blocks_for(total), kTpb, 0, s>>>(out, a, b, wa, wb, total, Na, Nb,
            FastDiv((uint32_t)(Na + Nb)));
    }
    nnk_after_launch(what, s);
}

}  // namespace

extern "C" {

void launch_activation_forward(float* out, const float* in, int n, Activation act, hipStream_t s) {
    NNK_REQUIRE(n >= 0, "act", "launch_activation_forward: n=%d", n);
    NNK_REQUIRE(act >= ACT_IDENTITY && act <= ACT_MP_SILU, "act", "launch_activation_forward: unknown activation %d", (int)act);
    if (n == 0) return;
    NNK_REQUIRE(out && in, "act", "launch_activation_forward: null pointer");
    const bool vec = aligned16(out) && aligned16(in);
    const unsigned blocks = blocks_for(vec ? n / 4 : n);
    if (vec && use_nt(8LL * n))
        NNK_ACT_DISPATCH(act, A, act_fwd_kernel<A, true, true><<<blocks, kTpb, 0, s>>>(out, in, n));
    else if (vec)
        NNK_ACT_DISPATCH(act, A, act_fwd_kernel<A, true, false><<<blocks, kTpb, 0, s>>>(out, in, n));
    else
        NNK_ACT_DISPATCH(act, A, act_fwd_kernel<A, false, false><<<blocks, kTpb, 0, s>>>(out, in, n));
    nnk_after_launch("launch_activation_forward", s);
}

void launch_activation_backward(float* grad_in, const float* grad_out, const float* in, int n,
    Activation act, hipStream_t s) {
    NNK_REQUIRE(n >= 0, "act", "launch_activation_backward: n=%d", n);
    NNK_REQUIRE(act >= ACT_IDENTITY && act <= ACT_MP_SILU, "act", "launch_activation_backward: unknown activation %d", (int)act);
    if (n == 0) return;
    NNK_REQUIRE(grad_in && grad_out && in, "act", "launch_activation_backward: null pointer");
    const bool vec = aligned16(grad_in) && aligned16(grad_out) && aligned16(in);
    const unsigned blocks = blocks_for(vec ? n / 4 : n);
    if (vec && use_nt(12LL * n))
        NNK_ACT_DISPATCH(act, A, act_bwd_kernel<A, true, true><<<blocks, kTpb, 0, s>>>(grad_in, grad_out, in, n));
    else if (vec)
        NNK_ACT_DISPATCH(act, A, act_bwd_kernel<A, true, false><<<blocks, kTpb, 0, s>>>(grad_in, grad_out, in, n));
    else
        NNK_ACT_DISPATCH(act, A, act_bwd_kernel<A, false, false><<<blocks, kTpb, 0, s>>>(grad_in, grad_out, in, n));
    nnk_after_launch("launch_activation_backward", s);
}

void launch_weighted_sum(float* out, const float* a, const float* b, float wa, float wb, int n,
    hipStream_t s) {
    NNK_REQUIRE(n >= 0, "ws", "launch_weighted_sum: n=%d", n);
    if (n == 0) return;
    NNK_REQUIRE(out && a && b, "ws", "launch_weighted_sum: null pointer");
    const bool vec = aligned16(out) && aligned16(a) && aligned16(b);
    if (vec && use_nt(12LL * n))
        weighted_sum_kernel<true, true><<<blocks_for(n / 4), kTpb, 0, s>>>(out, a, b, wa, wb, n);
    else if (vec)
        weighted_sum_kernel<true, false><<<blocks_for(n / 4), kTpb, 0, s>>>(out, a, b, wa, wb, n);
    else
        weighted_sum_kernel<false, false><<<blocks_for(n), kTpb, 0, s>>>(out, a, b, wa, wb, n);
    nnk_after_launch("launch_weighted_sum", s);
}

void launch_mp_sum(float* out, const float* a, const float* b, float t, int n, hipStream_t s) {
    float wa, wb;
    mp_sum_weights(t, &wa, &wb);
    launch_weighted_sum(out, a, b, wa, wb, n, s);
}

void launch_scale_by_scalar(float* x, const float* sc, int n, hipStream_t s) {
    NNK_REQUIRE(n >= 0, "scale", "launch_scale_by_scalar: n=%d", n);
    if (n == 0) return;
    NNK_REQUIRE(x && sc, "scale", "launch_scale_by_scalar: null pointer");
    if (aligned16(x) && use_nt(8LL * n))
        scale_kernel<true, true><<<blocks_for(n / 4), kTpb, 0, s>>>(x, sc, n);
    else if (aligned16(x))
        scale_kernel<true, false><<<blocks_for(n / 4), kTpb, 0, s>>>(x, sc, n);
    else
        scale_kernel<false, false><<<blocks_for(n), kTpb, 0, s>>>(x, sc, n);
    nnk_after_launch("launch_scale_by_scalar", s);
}

void launch_sgd_step(float* p, const float* g, float lr, int n, hipStream_t s) {
    NNK_REQUIRE(n >= 0, "sgd", "launch_sgd_step: n=%d", n);
    if (n == 0) return;
    NNK_REQUIRE(p && g, "sgd", "launch_sgd_step: null pointer");
    if (aligned16(p) && aligned16(g) && use_nt(12LL * n))
        sgd_kernel<true, true><<<blocks_for(n / 4), kTpb, 0, s>>>(p, g, lr, n);
    else if (aligned16(p) && aligned16(g))
        sgd_kernel<true, false><<<blocks_for(n / 4), kTpb, 0, s>>>(p, g, lr, n);
    else
        sgd_kernel<false, false><<<blocks_for(n), kTpb, 0, s>>>(p, g, lr, n);
    nnk_after_launch("launch_sgd_step", s);
}

void launch_add_bias(float* Y, const float* b, int M, int N, hipStream_t s) {
    NNK_REQUIRE(M >= 0 && N > 0, "bias", "launch_add_bias: bad shape M=%d N=%d", M, N);
    const long long total = (long long)M * N;
    NNK_REQUIRE(fits_i32(total), "bias", "launch_add_bias: %lld elements exceed 2^31", total);
    if (total == 0) return;
    NNK_REQUIRE(Y && b, "bias", "launch_add_bias: null pointer");
    if (N % 4 == 0 && aligned16(Y) && aligned16(b) && use_nt(8 * total))
        add_bias_vec_kernel<true><<<blocks_for(total / 4), kTpb, 0, s>>>(Y, b, total / 4, FastDiv((uint32_t)(N / 4)));
    else if (N % 4 == 0 && aligned16(Y) && aligned16(b))
        add_bias_vec_kernel<false><<<blocks_for(total / 4), kTpb, 0, s>>>(Y, b, total / 4, FastDiv((uint32_t)(N / 4)));
    else
        add_bias_kernel<<<blocks_for(total), kTpb, 0, s>>>(Y, b, total, FastDiv((uint32_t)N));
    nnk_after_launch("launch_add_bias", s);
}

void launch_bias_grad(float* gb, const float* grad_out, int batch, int N, hipStream_t s) {
    NNK_REQUIRE(batch >= 0 && N > 0, "bias_grad", "launch_bias_grad: bad shape batch=%d N=%d", batch, N);
    NNK_REQUIRE(gb, "bias_grad", "launch_bias_grad: null pointer");
    const int chunks = batch > 0 ? (batch + kBgRows - 1) / kBgRows : 0;
    if (chunks == 0) {
        // an empty sum is 0, as the reference's loop leaves it
        fill_kernel<<<dim3((unsigned)((N + kTpb - 1) / kTpb)), kTpb, 0, s>>>(gb, 0.0f, N);
        nnk_after_launch("launch_bias_grad", s);
        return;
    }
    NNK_REQUIRE(grad_out, "bias_grad", "launch_bias_grad: null pointer");
    float* part = nnk_scratch_acquire((size_t)chunks * N, s, "launch_bias_grad");
    if (!part) return;
    bias_grad_partial<<<dim3((unsigned)((N + kWave - 1) / kWave), (unsigned)chunks), kTpb, 0, s>>>(part, grad_out, batch, N);
    bias_grad_final<<<dim3((unsigned)((N + kTpb - 1) / kTpb)), kTpb, 0, s>>>(gb, part, chunks, N);
    nnk_scratch_release(part, s);
    nnk_after_launch("launch_bias_grad", s);
}

void launch_mp_cat(float* out, const float* a, const float* b, float t, int batch, int Na, int Nb,
    hipStream_t s) {
    float wa, wb;
    mp_cat_weights(t, Na, Nb, &wa, &wb);
    mp_cat_impl("launch_mp_cat", out, a, b, wa, wb, batch, Na, Nb, s);
}

void launch_mp_channel_cat(float* out, const float* a, const float* b, float t, int spatial, int Ca,
    int Cb, hipStream_t s) {
    float wa, wb;
    mp_cat_weights(t, Ca, Cb, &wa, &wb);
    mp_cat_impl("launch_mp_channel_cat", out, a, b, wa, wb, spatial, Ca, Cb, s);
}

void launch_mp_channel_split(float* grad_a, float* grad_b, const float* grad_out, float t,
    int spatial, int Ca, int Cb, hipStream_t s) {
    const char* what = "launch_mp_channel_split";
    NNK_REQUIRE(spatial >= 0 && Ca > 0 && Cb > 0, what, "%s: bad shape spatial=%d Ca=%d Cb=%d", what, spatial, Ca, Cb);
    const long long total = (long long)spatial * (Ca + Cb);
    NNK_REQUIRE(fits_i32(total), what, "%s: %lld elements exceed 2^31", what, total);
    if (total == 0) return;
    NNK_REQUIRE(grad_a && grad_b && grad_out, what, "%s: null pointer", what);
    float wa, wb;
    mp_cat_weights(t, Ca, Cb, &wa, &wb);
    if (Ca % 4 == 0 && Cb % 4 == 0 && aligned16(grad_a) && aligned16(grad_b) && aligned16(grad_out)) {
        const long long total4 = total / 4;
        if (use_nt(8 * total))
            mp_split_vec_kernel<true><<<blocks_for(total4), kTpb, 0, s>>>(grad_a, grad_b, grad_out, wa, wb,
                total4, Ca / 4, Cb / 4, FastDiv((uint32_t)((Ca + Cb) / 4)));
        else
            mp_split_vec_kernel<false><<<blocks_for(total4), kTpb, 0, s>>>(grad_a, grad_b, grad_out, wa, wb,
                total4, Ca / 4, Cb / 4, FastDiv((uint32_t)((Ca + Cb) / 4)));
    } else {
        mp_split_kernel<<<blocks_for(total), kTpb, 0, s>>>(grad_a, grad_b, grad_out, wa, wb, total,
            Ca, Cb, FastDiv((uint32_t)(Ca + Cb)));
    }
    nnk_after_launch(what, s);
}

}  // extern "C"
