// nnk_common.h -- device helpers shared by the gfx950 kernels of the launch layer.
//
// Numerical conventions (all kernels):
//   * fp32 storage and arithmetic; the library is compiled with
//     -ffp-contract=off, so a*b+c is a multiply and an add unless a function
//     opts in with `#pragma clang fp contract(fast)` (the fast Pade tanh and
//     the GroupNorm/LayerNorm bodies do).  Copies, single products and the
//     optimizer updates stay uncontracted, so they are bit-identical to the
//     CPU oracle, which is compiled with -ffp-contract=off.
//   * Division and sqrt are the correctly rounded IEEE operations (hipcc's
//     default) except in the fast form of the Pade activations (reciprocal,
//     see below);
//     rsqrtf maps to the hardware reciprocal square root.
//   * Reductions are fixed-shape trees (DPP within a row of 16 lanes, lane
//     reads across the 4 rows, LDS across waves), so every result is
//     reproducible run to run.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "nn_hip.h"

namespace nnk {

// ---------------------------------------------------------------------------
// Activation family.  Reference: src/kernels.cu:6-68.
// The tanh is the Pade [7/6] approximant of the Lambert continued fraction
// x/(1+x^2/(3+x^2/(5+...+x^2/13))), clamped to [-1,1]; the sigmoid is built
// on it as (tanh(x/2)+1)/2.  Backward formulas are the reference's (the SiLU
// derivative uses the approximate sigmoid, it is not the derivative of the
// approximate SiLU).
//
// Arithmetic, two forms (the reference build, Makefile:11, uses --use_fast_math,
// so its own quotient is approximate and its multiply-adds are contracted):
//   exact (FAST = false): the reference's operation order, no contraction,
//     correctly rounded division -- bit-identical to the CPU restatement;
//     used by the standalone activation kernels, which are HBM-bound.
//   fast (FAST = true): multiply-adds as FMAs and the quotient as numerator
//     times the hardware reciprocal (v_rcp_f32, 1 ulp); within a few ulp of
//     the exact form.  Used inside the fused GroupNorm kernels,
//     where the activation is most of the VALU work.  Near |tanh| = 1 the
//     terms 1 - t*t and 1 +- t cancel, so there the difference is relative to
//     the upstream gradient / input scale, not to the (tiny) result.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float pade_tanh_exact(float x) {
    const float x2 = x * x;
    const float p = x * (135135.0f + x2 * (17325.0f + x2 * (378.0f + x2)));
    const float q = 135135.0f + x2 * (62370.0f + x2 * (3150.0f + x2 * 28.0f));
    return fmaxf(-1.0f, fminf(1.0f, p / q));
}

__device__ __forceinline__ float pade_tanh_fast(float x) {
    const float x2 = x * x;
    const float p = x * fmaf(x2, fmaf(x2, x2 + 378.0f, 17325.0f), 135135.0f);
    const float q = fmaf(x2, fmaf(x2, fmaf(x2, 28.0f, 3150.0f), 62370.0f), 135135.0f);
    return fmaxf(-1.0f, fminf(1.0f, p * __builtin_amdgcn_rcpf(q)));
}

template <bool FAST>
__device__ __forceinline__ float pade_tanh(float x) {
    if constexpr (FAST) return pade_tanh_fast(x);
    else return pade_tanh_exact(x);
}

// sigmoid(z) = (tanh(z / 2) + 1) / 2 with the Pade tanh above, fast form.
// Substituting x = z / 2 (w = z^2 = 4 x^2) and halving the numerator scales
// every coefficient by a power of two (exact in float), so p / q = tanh(z/2) / 2;
// the + 1/2 is the addend of the multiply-add with the reciprocal, and the
// clamp of tanh to [-1, 1] becomes a clamp of the sigmoid to [0, 1], upper
// bound first as in the reference (a NaN quotient, for |z| beyond ~3e6,
// gives 1).  Within an ulp of halving the clamped tanh.
__device__ __forceinline__ float pade_sigmoid_fast(float z) {
    const float w = z * z;
    const float p = z * fmaf(w, fmaf(w, fmaf(w, 0.00390625f, 5.90625f), 1082.8125f), 33783.75f);
    const float q = fmaf(w, fmaf(w, fmaf(w, 0.4375f, 196.875f), 15592.5f), 135135.0f);
    return fmaxf(0.0f, fminf(1.0f, fmaf(p, __builtin_amdgcn_rcpf(q), 0.5f)));
}

template <bool FAST>
__device__ __forceinline__ float pade_sigmoid(float x) {
    // pade_tanh is clamped to [-1, 1], so (t + 1) * 0.5 already lies in [0, 1]:
    // the reference's outer clamp (kernels.cu:16) never changes the value and
    // is not evaluated.
    if constexpr (FAST) return pade_sigmoid_fast(x);
    else return (pade_tanh_exact(x * 0.5f) + 1.0f) * 0.5f;
}

constexpr float kGeluC = 0.7978845608f;
constexpr float kGeluA = 0.044715f;
constexpr float kMpSiluScale = 1.0f / 0.596f;

// Fast forms of the activation and its derivative: the reference formulas
// with the multiply-adds written as FMAs.
template <int ACT>
__device__ __forceinline__ float act_fwd_fast(float v) {
    if constexpr (ACT == ACT_RELU) {
        return v > 0.0f ? v : 0.0f;
    } else if constexpr (ACT == ACT_GELU) {
        const float t = pade_tanh_fast(kGeluC * fmaf(kGeluA * v, v * v, v));
        const float hv = 0.5f * v;
        return fmaf(hv, t, hv);
    } else if constexpr (ACT == ACT_SILU) {
        return v * pade_sigmoid<true>(v);
    } else if constexpr (ACT == ACT_MP_SILU) {
        return v * pade_sigmoid<true>(v) * kMpSiluScale;
    } else if constexpr (ACT == ACT_TANH) {
        return pade_tanh_fast(v);
    } else {
        return v;
    }
}

template <int ACT>
__device__ __forceinline__ float act_grad_fast(float z) {
    if constexpr (ACT == ACT_RELU) {
        return z > 0.0f ? 1.0f : 0.0f;
    } else if constexpr (ACT == ACT_TANH) {
        const float t = pade_tanh_fast(z);
        return fmaf(-t, t, 1.0f);
    } else if constexpr (ACT == ACT_SILU) {
        const float s = pade_sigmoid<true>(z);
        return s * fmaf(z, 1.0f - s, 1.0f);
    } else if constexpr (ACT == ACT_MP_SILU) {
        const float s = pade_sigmoid<true>(z);
        return s * fmaf(z, 1.0f - s, 1.0f) * kMpSiluScale;
    } else if constexpr (ACT == ACT_GELU) {
        const float t = pade_tanh_fast(kGeluC * fmaf(kGeluA * z, z * z, z));
        const float du = kGeluC * fmaf(3.0f * kGeluA * z, z, 1.0f);
        return fmaf(0.5f, 1.0f + t, 0.5f * z * fmaf(-t, t, 1.0f) * du);
    } else {
        return 1.0f;
    }
}

template <int ACT, bool FAST = true>
__device__ __forceinline__ float act_fwd(float v) {
    if constexpr (FAST) return act_fwd_fast<ACT>(v);
    if constexpr (ACT == ACT_RELU) {
        return v > 0.0f ? v : 0.0f;
    } else if constexpr (ACT == ACT_GELU) {
        return 0.5f * v * (1.0f + pade_tanh<FAST>(kGeluC * (v + kGeluA * v * v * v)));
    } else if constexpr (ACT == ACT_SILU) {
        return v * pade_sigmoid<FAST>(v);
    } else if constexpr (ACT == ACT_MP_SILU) {
        return v * pade_sigmoid<FAST>(v) * kMpSiluScale;
    } else if constexpr (ACT == ACT_TANH) {
        return pade_tanh<FAST>(v);
    } else {
        return v;
    }
}

template <int ACT, bool FAST = true>
__device__ __forceinline__ float act_grad(float z) {
    if constexpr (FAST) return act_grad_fast<ACT>(z);
    if constexpr (ACT == ACT_RELU) {
        return z > 0.0f ? 1.0f : 0.0f;
    } else if constexpr (ACT == ACT_TANH) {
        const float t = pade_tanh<FAST>(z);
        return 1.0f - t * t;
    } else if constexpr (ACT == ACT_SILU) {
        const float s = pade_sigmoid<FAST>(z);
        return s * (1.0f + z * (1.0f - s));
    } else if constexpr (ACT == ACT_MP_SILU) {
        const float s = pade_sigmoid<FAST>(z);
        return s * (1.0f + z * (1.0f - s)) * kMpSiluScale;
    } else if constexpr (ACT == ACT_GELU) {
        const float u = kGeluC * (z + kGeluA * z * z * z);
        const float t = pade_tanh<FAST>(u);
        const float du = kGeluC * (1.0f + 3.0f * kGeluA * z * z);
        return 0.5f * (1.0f + t) + 0.5f * z * (1.0f - t * t) * du;
    } else {
        return 1.0f;
    }
}

// Instantiate `F<ACT>` for a runtime activation; returns false for an unknown kind.
#define NNK_ACT_DISPATCH(act, ACTV, ...)                              \
    [&]() -> bool {                                                   \
        switch (act) {                                                \
        case ACT_IDENTITY: { constexpr int ACTV = ACT_IDENTITY; __VA_ARGS__; return true; } \
        case ACT_RELU:     { constexpr int ACTV = ACT_RELU;     __VA_ARGS__; return true; } \
        case ACT_GELU:     { constexpr int ACTV = ACT_GELU;     __VA_ARGS__; return true; } \
        case ACT_SILU:     { constexpr int ACTV = ACT_SILU;     __VA_ARGS__; return true; } \
        case ACT_TANH:     { constexpr int ACTV = ACT_TANH;     __VA_ARGS__; return true; } \
        case ACT_MP_SILU:  { constexpr int ACTV = ACT_MP_SILU;  __VA_ARGS__; return true; } \
        default: return false;                                        \
        }                                                             \
    }()

// ---------------------------------------------------------------------------
// Wave64 reductions.
// ---------------------------------------------------------------------------
constexpr int kWave = 64;

// DPP controls (CDNA ISA): quad_perm [1,0,3,2], quad_perm [2,3,0,1],
// row_half_mirror, row_mirror.
constexpr int kDppQuadXor1 = 0xb1;
constexpr int kDppQuadXor2 = 0x4e;
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __builtin_bit_cast(float,
        __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xf, 0xf, true));
}

__device__ __forceinline__ float lane_read(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Sum over the 64 lanes of a full wave; the result is wave-uniform.
// Every lane of the wave must be active.
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_mov<kDppQuadXor1>(v);
    v += dpp_mov<kDppQuadXor2>(v);
    v += dpp_mov<kDppRowHalfMirror>(v);
    v += dpp_mov<kDppRowMirror>(v);
    return ((lane_read(v, 0) + lane_read(v, 16)) + lane_read(v, 32)) + lane_read(v, 48);
}

// Sum over the lanes whose index agrees with this lane's modulo STRIDE
// (STRIDE a power of two < 64); the result lands in every such lane.
template <int STRIDE>
__device__ __forceinline__ float wave_sum_strided(float v) {
#pragma unroll
    for (int m = STRIDE; m < kWave; m <<= 1) v += __shfl_xor(v, m, kWave);
    return v;
}

// Block-wide sum of one value per thread.  `slots` is an LDS array of NW floats
// used by this call only (a second reduction in the same kernel needs other
// slots).  Every thread of the block must call it.
template <int NW>
__device__ __forceinline__ float block_sum(float v, float* slots) {
    const float w = wave_sum(v);
    if ((threadIdx.x & (kWave - 1)) == 0) slots[threadIdx.x / kWave] = w;
    __syncthreads();
    float s = slots[0];
#pragma unroll
    for (int i = 1; i < NW; ++i) s += slots[i];
    return s;
}

// Two block sums sharing one barrier; slots holds 2*NW floats.
template <int NW>
__device__ __forceinline__ void block_sum2(float& a, float& b, float* slots) {
    const float wa = wave_sum(a);
    const float wb = wave_sum(b);
    if ((threadIdx.x & (kWave - 1)) == 0) {
        slots[threadIdx.x / kWave] = wa;
        slots[NW + threadIdx.x / kWave] = wb;
    }
    __syncthreads();
    float sa = slots[0], sb = slots[NW];
#pragma unroll
    for (int i = 1; i < NW; ++i) {
        sa += slots[i];
        sb += slots[NW + i];
    }
    a = sa;
    b = sb;
}

// ---------------------------------------------------------------------------
// XCD-aware block order.  The dispatcher deals consecutive workgroup ids to
// the 8 XCDs of an MI355X in turn, and each XCD has its own L2.  Remapping
// makes each XCD walk a contiguous range of work items in dispatch order, so
// neighbouring items (which share cache lines, e.g. the 4 GroupNorm groups of
// one 128-byte pixel slice) meet in the same L2.  A bijection on [0, n).
// ---------------------------------------------------------------------------
constexpr int kNumXcd = 8;

__device__ __forceinline__ int xcd_swizzle(int bid, int n) {
    const int xcd = bid % kNumXcd;
    const int k = bid / kNumXcd;
    const int per = n / kNumXcd;
    const int rem = n % kNumXcd;
    const int start = xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per;
    return start + k;
}

// ---------------------------------------------------------------------------
// Division by a runtime constant d (1 <= d < 2^31) for numerators < 2^31:
// q = (umulhi(n, magic) + n) >> shift  (round-up magic-number method of
// Granlund and Montgomery, "Division by invariant integers using
// multiplication", PLDI 1994).
// ---------------------------------------------------------------------------
struct FastDiv {
    uint32_t d;
    uint32_t magic;
    uint32_t shift;

    __host__ __device__ FastDiv() : d(1), magic(0), shift(0) {}
    __host__ explicit FastDiv(uint32_t divisor) : d(divisor) {
        uint32_t s = 0;
        while ((1ull << s) < divisor) ++s;
        shift = s;
        magic = (uint32_t)(((1ull << 32) * ((1ull << s) - divisor)) / divisor + 1ull);
        if (divisor == 1) magic = 0;
    }
    __device__ __forceinline__ uint32_t div(uint32_t n) const {
        const uint32_t t = __umulhi(n, magic);
        return (uint32_t)(((uint64_t)t + n) >> shift);
    }
    __device__ __forceinline__ void divmod(uint32_t n, uint32_t& q, uint32_t& r) const {
        q = div(n);
        r = n - q * d;
    }
};

// ---------------------------------------------------------------------------
// 128-bit global accesses.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }
__device__ __forceinline__ void st4(float* p, float4 v) { *reinterpret_cast<float4*>(p) = v; }
typedef float f32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 ld4_stream(const float* p) {
    const f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
    return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void st4_stream(float* p, float4 v) {
    const f32x4 w = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(w, reinterpret_cast<f32x4*>(p));
}

// Cache policy of the streaming kernels.  A launch that touches at least
// kNtBytes (twice the MI355X's 256 MB Infinity Cache) streams its tensors
// with nontemporal loads and stores; smaller launches keep ordinary accesses
// so that operands a previous kernel just wrote can be served from that
// cache.  Measured here: nt saves 5-25 % on the 0.7-3 GB rows and costs the
// 67-268 MB rows 8-25 %.
constexpr long long kNtBytes = 512LL << 20;
inline bool use_nt(long long bytes) { return bytes >= kNtBytes; }

template <bool NT>
__device__ __forceinline__ float4 ldS(const float* p) {
    if constexpr (NT) return ld4_stream(p);
    else return ld4(p);
}
template <bool NT>
__device__ __forceinline__ void stS(float* p, float4 v) {
    if constexpr (NT) st4_stream(p, v);
    else st4(p, v);
}

__host__ __device__ __forceinline__ bool aligned16(const void* p) {
    return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

// ---------------------------------------------------------------------------
// Epoch-tagged 64-bit records: the exchange between workgroups of one launch.
// A record is (launch epoch << 32 | float bits), stored and loaded with
// relaxed agent-scope atomics (coherent across the XCDs' L2s).  A reader
// accepts a record only when it carries its own launch's epoch, so no fence
// has to order the writer's record before the writer's arrival count (an
// agent-scope release writes back the whole L2).  The epoch is never 0 and
// differs from every earlier launch's on the same workspace, so a
// zero-filled workspace, or one holding records of earlier launches only,
// never passes for this launch's data.
// ---------------------------------------------------------------------------
__device__ __forceinline__ unsigned long long tagged(unsigned long long tag, float v) {
    return tag | (unsigned long long)__builtin_bit_cast(unsigned, v);
}
__device__ __forceinline__ void rec_store(unsigned long long* p, unsigned long long v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned long long rec_load(const unsigned long long* p) {
    return __hip_atomic_load(const_cast<unsigned long long*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Where a bounded wait that gives up leaves its mark: the sticky word of the
// launch's workspace (nnhip_groupnorm_workspace_status reads it) and a
// process-wide word in host-mapped memory, which nnhip_get_last_error reads
// without synchronising the device.  Written only on that failure path.
struct WaitFail {
    unsigned* ws;
    unsigned* host;
};
__device__ __forceinline__ void wait_failed(const WaitFail& f) {
    atomicOr(f.ws, 1u);
    __hip_atomic_store(f.host, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Poll one record until it carries `epoch`, at most spin_limit times (each
// poll sleeps first); past that flag the failure and return what is there.
__device__ __forceinline__ float rec_wait(const unsigned long long* p, unsigned long long r, unsigned epoch,
    unsigned spin_limit, const WaitFail& fail) {
    unsigned n = 0;
    while ((unsigned)(r >> 32) != epoch) {
        if (++n > spin_limit) {
            wait_failed(fail);
            break;
        }
        __builtin_amdgcn_s_sleep(1);
        r = rec_load(p);
    }
    return __builtin_bit_cast(float, (unsigned)r);
}

// Sum of the n tagged records p[0], p[stride], ... in index order, KB loads
// in flight.  The records of a batch that do not carry `epoch` yet are loaded
// again together, so a batch costs one round trip per poll rather than one
// per late record; past spin_limit polls the failure is flagged and the sum
// is taken as it stands.  n must be uniform over the wave.
template <int KB>
__device__ __forceinline__ float rec_sum(const unsigned long long* p, size_t stride, int n, unsigned epoch,
    unsigned spin_limit, const WaitFail& fail) {
    float acc = 0.0f;
    for (int m = 0; m < n; m += KB) {
        const int nb = n - m < KB ? n - m : KB;
        unsigned long long r[KB];
#pragma unroll
        for (int u = 0; u < KB; ++u)
            if (u < nb) r[u] = rec_load(p + (size_t)(m + u) * stride);
        for (unsigned polls = 0;; ++polls) {
            bool late = false;
#pragma unroll
            for (int u = 0; u < KB; ++u) late |= u < nb && (unsigned)(r[u] >> 32) != epoch;
            if (!late) break;
            if (polls >= spin_limit) {
                wait_failed(fail);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
#pragma unroll
            for (int u = 0; u < KB; ++u)
                if (u < nb && (unsigned)(r[u] >> 32) != epoch) r[u] = rec_load(p + (size_t)(m + u) * stride);
        }
#pragma unroll
        for (int u = 0; u < KB; ++u)
            if (u < nb) acc += __builtin_bit_cast(float, (unsigned)r[u]);
    }
    return acc;
}


}  // namespace nnk

// ---------------------------------------------------------------------------
// Host side of the launch layer: error record and scratch.
// ---------------------------------------------------------------------------

// Record an error (first one wins until read by nnhip_get_last_error).
void nnk_set_error(int code, const char* fmt, ...);
// Check the launch just made on `s` (and, in NNHIP_CHECK=1 mode, synchronise
// the stream and abort on failure).  `what` names the launcher.
void nnk_after_launch(const char* what, hipStream_t s);
// Whether stream s is capturing a graph (no synchronisation or allocation then).
bool nnk_capturing(hipStream_t s);
// Compute units of the device that stream s (or, for the null stream, the
// current device) belongs to, cached per device; 0 if unknown.
int nnk_device_cus(hipStream_t s);
void nnk_path_note(const char* fmt, ...);
// Stream-ordered scratch for launchers that need partial sums.
float* nnk_scratch_acquire(size_t n_floats, hipStream_t s, const char* what);
void nnk_scratch_release(float* p, hipStream_t s);
void nnk_scratch_forget_stream(hipStream_t s);
// Zero n_floats words of a workspace drawn from the scratch pool (a fill
// kernel, so that the sequence can be captured in a graph).
void nnk_clear_workspace(float* ws, size_t n_floats, hipStream_t s);
// Device address of the process-wide host-mapped word that a streaming
// kernel's bounded wait sets when it gives up (see WaitFail).  It is
// allocated when the library is loaded, never by a launcher; nullptr when
// that allocation failed (no device at load time).
unsigned* nnk_wait_flag();

#define NNK_REQUIRE(cond, what, ...)                         \
    do {                                                     \
        if (!(cond)) {                                       \
            nnk_set_error(hipErrorInvalidValue, __VA_ARGS__);\
            return;                                          \
        }                                                    \
    } while (0)

// As NNK_REQUIRE, in a function returning `ret`.
#define NNK_REQUIRE_RET(cond, ret, what, ...)                \
    do {                                                     \
        if (!(cond)) {                                       \
            nnk_set_error(hipErrorInvalidValue, __VA_ARGS__);\
            return ret;                                      \
        }                                                    \
    } while (0)
