// k_optim.hip -- Adam (single tensor, the reference launcher) and the
// multi-tensor Adam + EMA update.
// Reference maths: adam_step_kernel src/kernels.cu:170-183 (launcher 241-248)
// with the host bias corrections of src/optimizer.c:62-64, and the EMA update
// src/ema.c:29-35 (weighted_sum with decay, 1-decay).
//
// Multi-tensor form: the plan holds a device table of tensors and a list of
// 1024-element chunks (tensor, chunk index); one workgroup updates one chunk,
// so a whole parameter list is one launch instead of one per tensor.  Per
// parameter the fused step moves 36 bytes (read p, g, m, v, shadow; write p,
// m, v, shadow); p_new feeds the EMA from registers.  Large plans stream all
// five tensors with nontemporal loads and stores (use_nt).
#include <stdlib.h>
#include <string.h>

#include "nnk_common.h"

namespace {

using namespace nnk;

constexpr int kTpb = 256;
constexpr int kChunk = 1024;  // elements per workgroup: one float4 per thread
static_assert(kChunk % (4 * kTpb) == 0, "a full chunk is whole float4 slices of the workgroup");

struct DevSlot {
    float* p;
    float* m;
    float* v;
    const float* g;
    float* shadow;
    long long n;
    int vec;  // all pointers 16-byte aligned
    int pad;
};

struct AdamArgs {
    float lr, b1, b2, eps, bc1, bc2;
};

__device__ __forceinline__ float adam_one(float& p, float& m, float& v, float g, const AdamArgs& a) {
    const float mi = a.b1 * m + (1.0f - a.b1) * g;
    const float vi = a.b2 * v + (1.0f - a.b2) * g * g;
    m = mi;
    v = vi;
    p -= a.lr * (mi / a.bc1) / (sqrtf(vi / a.bc2) + a.eps);
    return p;
}

// One full chunk (kChunk elements, 16-byte aligned): every thread loads its
// U float4 of each tensor before any arithmetic, so all of the chunk's loads
// are in flight at once (a loop that stores p, m, v before loading the next
// slice keeps one slice in flight, since the tensors may alias as far as the
// compiler knows).  p_new feeds the EMA from registers.
template <int MODE, bool NT, bool EMA>
__device__ __forceinline__ void chunk_full(const DevSlot& t, long long start, const AdamArgs& a, float w0, float w1) {
    constexpr int U = kChunk / 4 / kTpb;
    float4 pp[U], mm[U], vv[U], gg[U], sh[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const long long i = start + 4LL * (threadIdx.x + u * kTpb);
        pp[u] = ldS<NT>(t.p + i);
        if constexpr (MODE != 2) {
            mm[u] = ldS<NT>(t.m + i);
            vv[u] = ldS<NT>(t.v + i);
            gg[u] = ldS<NT>(t.g + i);
        }
        if constexpr (EMA) sh[u] = ldS<NT>(t.shadow + i);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const long long i = start + 4LL * (threadIdx.x + u * kTpb);
        if constexpr (MODE != 2) {
            adam_one(pp[u].x, mm[u].x, vv[u].x, gg[u].x, a);
            adam_one(pp[u].y, mm[u].y, vv[u].y, gg[u].y, a);
            adam_one(pp[u].z, mm[u].z, vv[u].z, gg[u].z, a);
            adam_one(pp[u].w, mm[u].w, vv[u].w, gg[u].w, a);
            stS<NT>(t.p + i, pp[u]);
            stS<NT>(t.m + i, mm[u]);
            stS<NT>(t.v + i, vv[u]);
        }
        if constexpr (EMA) {
            sh[u].x = w0 * sh[u].x + w1 * pp[u].x;
            sh[u].y = w0 * sh[u].y + w1 * pp[u].y;
            sh[u].z = w0 * sh[u].z + w1 * pp[u].z;
            sh[u].w = w0 * sh[u].w + w1 * pp[u].w;
            stS<NT>(t.shadow + i, sh[u]);
        }
    }
}

// A chunk that is a tensor's last and partial, or of a tensor that is not
// 16-byte aligned.
template <int MODE, bool NT>
__device__ __forceinline__ void chunk_any(const DevSlot& t, long long start, long long end, bool ema,
    const AdamArgs& a, float w0, float w1) {
    if (t.vec) {
        const long long nv = (end - start) / 4;
        for (long long q = threadIdx.x; q < nv; q += kTpb) {
            const long long i = start + 4 * q;
            float4 pp = ldS<NT>(t.p + i);
            if constexpr (MODE != 2) {
                float4 mm = ldS<NT>(t.m + i), vv = ldS<NT>(t.v + i);
                const float4 gg = ldS<NT>(t.g + i);
                adam_one(pp.x, mm.x, vv.x, gg.x, a);
                adam_one(pp.y, mm.y, vv.y, gg.y, a);
                adam_one(pp.z, mm.z, vv.z, gg.z, a);
                adam_one(pp.w, mm.w, vv.w, gg.w, a);
                stS<NT>(t.p + i, pp);
                stS<NT>(t.m + i, mm);
                stS<NT>(t.v + i, vv);
            }
            if (ema) {
                float4 sh = ldS<NT>(t.shadow + i);
                sh.x = w0 * sh.x + w1 * pp.x;
                sh.y = w0 * sh.y + w1 * pp.y;
                sh.z = w0 * sh.z + w1 * pp.z;
                sh.w = w0 * sh.w + w1 * pp.w;
                stS<NT>(t.shadow + i, sh);
            }
        }
        const long long i = start + 4 * nv + threadIdx.x;
        if (i < end) {
            float pn = t.p[i];
            if constexpr (MODE != 2) pn = adam_one(t.p[i], t.m[i], t.v[i], t.g[i], a);
            if (ema) t.shadow[i] = w0 * t.shadow[i] + w1 * pn;
        }
    } else {
        for (long long i = start + threadIdx.x; i < end; i += kTpb) {
            float pn = t.p[i];
            if constexpr (MODE != 2) pn = adam_one(t.p[i], t.m[i], t.v[i], t.g[i], a);
            if (ema) t.shadow[i] = w0 * t.shadow[i] + w1 * pn;
        }
    }
}

// Single tensor (the reference launcher): one chunk per workgroup.
template <bool NT>
__global__ __launch_bounds__(kTpb) void adam_kernel(float* __restrict__ p, float* __restrict__ m,
    float* __restrict__ v, const float* __restrict__ g, AdamArgs a, long long n, int vec) {
    const DevSlot t{p, m, v, g, nullptr, n, vec, 0};
    const long long start = (long long)blockIdx.x * kChunk;
    const long long end = min(start + (long long)kChunk, n);
    if (vec && end - start == kChunk) chunk_full<0, NT, false>(t, start, a, 0.0f, 0.0f);
    else chunk_any<0, NT>(t, start, end, false, a, 0.0f, 0.0f);
}

// mode 0: Adam only, 1: Adam then EMA, 2: EMA only (shadow = w0*shadow + w1*p)
template <int MODE, bool NT>
__global__ __launch_bounds__(kTpb) void multi_tensor_kernel(const DevSlot* __restrict__ slots,
    const int2* __restrict__ chunks, AdamArgs a, float w0, float w1) {
    const int2 ch = chunks[blockIdx.x];
    const DevSlot t = slots[ch.x];
    const long long start = (long long)ch.y * kChunk;
    const long long end = min(start + (long long)kChunk, t.n);
    const bool ema = MODE != 0 && t.shadow != nullptr;
    if (t.vec && end - start == kChunk) {
        if (ema) chunk_full<MODE, NT, MODE != 0>(t, start, a, w0, w1);
        else if constexpr (MODE != 2) chunk_full<MODE, NT, false>(t, start, a, w0, w1);
    } else {
        chunk_any<MODE, NT>(t, start, end, ema, a, w0, w1);
    }
}

}  // namespace

struct NnMultiTensorPlan {
    DevSlot* d_slots;
    int2* d_chunks;
    int count;
    int nchunks;
    int has_adam;  // every slot carries p, m, v, g
    int has_ema;   // every slot carries p and shadow
};

extern "C" {

void launch_adam_step(float* p, float* m, float* v, const float* g, float lr, float beta1,
    float beta2, float eps, float bc1, float bc2, int n, hipStream_t s) {
    const char* what = "launch_adam_step";
    NNK_REQUIRE(n >= 0, what, "%s: n=%d", what, n);
    if (n == 0) return;
    NNK_REQUIRE(p && m && v && g, what, "%s: null pointer", what);
    const AdamArgs a{lr, beta1, beta2, eps, bc1, bc2};
    const int vec = aligned16(p) && aligned16(m) && aligned16(v) && aligned16(g);
    if (use_nt(28LL * n))
        adam_kernel<true><<<(unsigned)((n + kChunk - 1) / kChunk), kTpb, 0, s>>>(p, m, v, g, a, n, vec);
    else
        adam_kernel<false><<<(unsigned)((n + kChunk - 1) / kChunk), kTpb, 0, s>>>(p, m, v, g, a, n, vec);
    nnk_after_launch(what, s);
}

NnMultiTensorPlan* nnhip_multi_tensor_plan_create(const NnTensorSlot* slots, int count) {
    const char* what = "nnhip_multi_tensor_plan_create";
    if (count < 0 || (count > 0 && !slots)) {
        nnk_set_error(hipErrorInvalidValue, "%s: bad tensor list", what);
        return nullptr;
    }
    DevSlot* hs = (DevSlot*)calloc((size_t)(count > 0 ? count : 1), sizeof(DevSlot));
    long long nchunks = 0;
    int has_adam = 1, has_ema = 1;
    for (int i = 0; i < count; ++i) {
        const NnTensorSlot& t = slots[i];
        if (t.n < 0 || (t.n > 0 && !t.p)) {
            free(hs);
            nnk_set_error(hipErrorInvalidValue, "%s: tensor %d has n=%lld or no p", what, i, t.n);
            return nullptr;
        }
        hs[i] = DevSlot{t.p, t.m, t.v, t.g, t.shadow, t.n,
            aligned16(t.p) && aligned16(t.m) && aligned16(t.v) && aligned16(t.g) && aligned16(t.shadow), 0};
        if (!t.m || !t.v || !t.g) has_adam = 0;
        if (!t.shadow) has_ema = 0;
        nchunks += (t.n + kChunk - 1) / kChunk;
    }
    if (nchunks >= (1LL << 31)) {
        free(hs);
        nnk_set_error(hipErrorInvalidValue, "%s: too many chunks", what);
        return nullptr;
    }
    int2* hc = (int2*)malloc((size_t)(nchunks > 0 ? nchunks : 1) * sizeof(int2));
    long long k = 0;
    for (int i = 0; i < count; ++i) {
        const long long nc = (slots[i].n + kChunk - 1) / kChunk;
        for (long long c = 0; c < nc; ++c) hc[k++] = make_int2(i, (int)c);
    }
    NnMultiTensorPlan* plan = (NnMultiTensorPlan*)calloc(1, sizeof(NnMultiTensorPlan));
    plan->count = count;
    plan->nchunks = (int)nchunks;
    plan->has_adam = has_adam;
    plan->has_ema = has_ema;
    hipError_t e = hipMalloc((void**)&plan->d_slots, sizeof(DevSlot) * (size_t)(count > 0 ? count : 1));
    if (e == hipSuccess) e = hipMalloc((void**)&plan->d_chunks, sizeof(int2) * (size_t)(nchunks > 0 ? nchunks : 1));
    if (e == hipSuccess && count > 0) e = hipMemcpy(plan->d_slots, hs, sizeof(DevSlot) * (size_t)count, hipMemcpyHostToDevice);
    if (e == hipSuccess && nchunks > 0) e = hipMemcpy(plan->d_chunks, hc, sizeof(int2) * (size_t)nchunks, hipMemcpyHostToDevice);
    free(hs);
    free(hc);
    if (e != hipSuccess) {
        nnk_set_error((int)e, "%s: %s", what, hipGetErrorString(e));
        nnhip_multi_tensor_plan_destroy(plan);
        return nullptr;
    }
    return plan;
}

void nnhip_multi_tensor_plan_destroy(NnMultiTensorPlan* plan) {
    if (!plan) return;
    if (plan->d_slots) (void)hipFree(plan->d_slots);
    if (plan->d_chunks) (void)hipFree(plan->d_chunks);
    free(plan);
}

void launch_adam_ema_step(const NnMultiTensorPlan* plan, float lr, float beta1, float beta2,
    float eps, float bc1, float bc2, float ema_w0, float ema_w1, hipStream_t s) {
    const char* what = "launch_adam_ema_step";
    NNK_REQUIRE(plan, what, "%s: null plan", what);
    NNK_REQUIRE(plan->has_adam, what, "%s: plan lacks m/v/g for some tensor", what);
    if (plan->nchunks == 0) return;
    const AdamArgs a{lr, beta1, beta2, eps, bc1, bc2};
    const long long elems = (long long)plan->nchunks * kChunk;  // upper bound of the plan's parameters
    const unsigned grid = (unsigned)plan->nchunks;
    if (ema_w1 != 0.0f || ema_w0 != 1.0f) {
        if (use_nt(36 * elems))
            multi_tensor_kernel<1, true><<<grid, kTpb, 0, s>>>(plan->d_slots, plan->d_chunks, a, ema_w0, ema_w1);
        else
            multi_tensor_kernel<1, false><<<grid, kTpb, 0, s>>>(plan->d_slots, plan->d_chunks, a, ema_w0, ema_w1);
    } else {
        if (use_nt(28 * elems))
            multi_tensor_kernel<0, true><<<grid, kTpb, 0, s>>>(plan->d_slots, plan->d_chunks, a, ema_w0, ema_w1);
        else
            multi_tensor_kernel<0, false><<<grid, kTpb, 0, s>>>(plan->d_slots, plan->d_chunks, a, ema_w0, ema_w1);
    }
    nnk_after_launch(what, s);
}

void launch_ema_update(const NnMultiTensorPlan* plan, float w0, float w1, hipStream_t s) {
    const char* what = "launch_ema_update";
    NNK_REQUIRE(plan, what, "%s: null plan", what);
    NNK_REQUIRE(plan->has_ema, what, "%s: plan lacks a shadow for some tensor", what);
    if (plan->nchunks == 0) return;
    const AdamArgs a{0, 0, 0, 0, 1, 1};
    if (use_nt(12LL * plan->nchunks * kChunk))
        multi_tensor_kernel<2, true><<<(unsigned)plan->nchunks, kTpb, 0, s>>>(plan->d_slots, plan->d_chunks, a, w0, w1);
    else
        multi_tensor_kernel<2, false><<<(unsigned)plan->nchunks, kTpb, 0, s>>>(plan->d_slots, plan->d_chunks, a, w0, w1);
    nnk_after_launch(what, s);
}

}  // extern "C"
