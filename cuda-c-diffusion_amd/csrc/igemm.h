// igemm.h -- the implicit-GEMM convolution kernels on the fp32 matrix cores,
// shared by k_igemm.hip (the plain launchers) and k_igemm_fused.hip (the
// launchers with a neighbouring pass folded into a kernel's operand loads or
// epilogue).  Design notes and the MFMA lane layout: k_igemm.hip.
#pragma once
#include "nn_hip_rt.h"
#include "nnk_common.h"

namespace {

using namespace nnk;

constexpr int kBM = 128, kBK = 32, kTpb = 256;
constexpr int kBNmin = 64;  // output-channel tiles of 128 or 64
typedef float f32x16 __attribute__((ext_vector_type(16)));

struct ConvShape {
    int B, H, W, Cin, Cout, K, stride, pad, Ho, Wo;
    int M;    // B * Ho * Wo
    int KKC;  // K * K * Cin
    FastDiv wo, ho;  // output pixel decode m -> (b, oh, ow)
};

// float4 slot of (row, chunk) in a [128][8] tile.  The xor spreads any 8
// consecutive rows of one chunk over the 8 chunk positions, and any 16
// consecutive rows over distinct (row parity, position) pairs, so 128-bit
// accesses whose lane groups cover 128 or 256 bytes of banks do not conflict.
__device__ __forceinline__ int slot(int row, int chunk) {
    return row * 8 + (chunk ^ (row & 7) ^ ((row >> 3) & 1));
}

// float offset of (k, n) in a [32][BN] B tile: rows 4..7 of every 8 rotated by 32
template <int BN>
__device__ __forceinline__ int kslot(int k, int n) {
    return k * BN + ((n + 32 * ((k >> 2) & 1)) & (BN - 1));
}

enum { kEpiNone = 0, kEpiBias = 1, kEpiGain = 2 };
// Fused neighbours of the forward / input-gradient kernel (bit flags), with v
// the output after bias or gain:
//   kXeRes : y = wa * res[m, n] + wb * v            (launch_weighted_sum(y, res, v, wa, wb))
//   kXeActG: v = v * act'(xa[m, n]) first            (launch_activation_backward)
//   kXeMod : y = v and y2 = act(v * (cond[b, n] + 1)) (launch_spatial_modulate_act_forward)
// each with the operation order of the pass it replaces, so the results are
// those of the separate passes bit for bit.
enum { kXeNone = 0, kXeRes = 1, kXeActG = 2, kXeMod = 4 };
struct ConvEpi {
    const float* res;   // kXeRes: [M][C_out]
    const float* xa;    // kXeActG: [M][C_out]
    const float* cond;  // kXeMod: [B][C_out]
    float* y2;          // kXeMod: [M][C_out]
    float wa, wb;       // kXeRes weights
    FastDiv hw;         // kXeMod: output pixels per sample
};
// Source of operand B: the forward's weight Wt[k][n], or the input gradient's
// flipped weight (sh is then the gradient's convolution: C_in = the layer's
// C_out, C_out = the layer's C_in, so Wt is [K*K*sh.Cout][sh.Cin]).
enum { kWFwd = 0, kWFlip = 1 };

template <int EPI, int BN, int WSRC, int XE = kXeNone, int ACT = 0>
__global__ __launch_bounds__(kTpb, 2) void igemm_fwd(float* __restrict__ Y, const float* __restrict__ X,
    const float* __restrict__ Wt, const float* __restrict__ bias, const float* __restrict__ gain, ConvShape sh,
    ConvEpi ep) {
    constexpr int UT = BN / 64;  // 32-column accumulator tiles per wave
    // weight float4 loaded per thread: a 4 x 4 block (forward) or BN / 32
    // rows of one chunk (flipped)
    constexpr int BQ = WSRC == kWFwd ? 4 : BN / 32;
    constexpr int NQ = BN / 4;   // forward: n quads of the tile
    __shared__ float4 As[2][kBM * 8];
    __shared__ float4 Bs[2][BN * 8];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int wm = w >> 1, wn = w & 1;
    const int m0 = blockIdx.x * kBM, n0 = blockIdx.y * BN;
    // loader role: chunk ch of rows r0 + 32 q
    const int ch = tid & 7, r0 = tid >> 3;
    int pix[4], ihb[4], iwb[4];
    bool rok[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int m = m0 + r0 + 32 * q;
        rok[q] = m < sh.M;
        const int mm = rok[q] ? m : 0;
        uint32_t t, ow, b, oh;
        sh.wo.divmod((uint32_t)mm, t, ow);
        sh.ho.divmod(t, b, oh);
        pix[q] = (int)b * sh.H * sh.W;
        ihb[q] = (int)oh * sh.stride - sh.pad;
        iwb[q] = (int)ow * sh.stride - sh.pad;
    }
    // forward weight roles: n quad n4, k rows 4 kq .. 4 kq + 3 of the slice
    // (with BN = 64 the second half of the workgroup repeats the first's
    // loads and stores nothing: every lane loads, see below)
    const int n4 = tid % NQ, kq = (tid / NQ) % 8;
    const bool bput = NQ * 8 >= kTpb || tid < NQ * 8;
    const float* wq = Wt + (size_t)(4 * kq) * sh.Cout + n0 + 4 * n4;
    // flipped weight: row n0 + r0 + 32 q of the tap's [C_in][C_out] block
    const float* wrow = Wt + (size_t)(n0 + r0) * sh.Cin + ch * 4;
    const int KK = sh.K * sh.K;

    // Every lane loads (a padding position reads channel ci of pixel 0 and is
    // zeroed when stored): a branch around a load would make the compiler's
    // later waits drain the whole vector-memory counter, i.e. wait for the
    // next slice's loads before the current slice's MFMAs.
    // Two register sets: the slice two ahead is loaded while the next one is
    // written to LDS, so a load has two slices of MFMA work to arrive.
    struct Regs {
        float4 a[4], b[BQ];
        bool ok[4];
    };
    Regs R0, R1;
    auto load = [&](int kt, Regs& R) {
        const int k0 = kt * kBK;
        const int khw = k0 / sh.Cin, cs = k0 - khw * sh.Cin, ci = cs + ch * 4;
        const int kh = khw / sh.K, kw = khw - kh * sh.K;
        // flipped weight: the slice's channels cs.. of tap KK-1-khw, a
        // uniform offset from each lane's row (held in a scalar register)
        const int wfo = __builtin_amdgcn_readfirstlane((KK - 1 - khw) * sh.Cout * sh.Cin + cs);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int ih = ihb[q] + kh, iw = iwb[q] + kw;
            R.ok[q] = rok[q] & ((unsigned)ih < (unsigned)sh.H) & ((unsigned)iw < (unsigned)sh.W);
            const int p = R.ok[q] ? pix[q] + ih * sh.W + iw : 0;
            R.a[q] = ld4(X + (size_t)p * sh.Cin + ci);
            if constexpr (WSRC == kWFwd) R.b[q] = ld4(wq + (size_t)(k0 + q) * sh.Cout);
            else if (q < BQ) R.b[q] = ld4(wrow + wfo + 32 * q * sh.Cin);
        }
    };
    // Padding is zeroed by masking the bits (a select of whole float4 values
    // becomes a select of their addresses, which puts them in scratch memory).
    auto store = [&](int buf, const Regs& R) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const unsigned mk = R.ok[q] ? 0xffffffffu : 0u;
            const float4 a = R.a[q];
            float4 v;
            v.x = __uint_as_float(__float_as_uint(a.x) & mk);
            v.y = __uint_as_float(__float_as_uint(a.y) & mk);
            v.z = __uint_as_float(__float_as_uint(a.z) & mk);
            v.w = __uint_as_float(__float_as_uint(a.w) & mk);
            As[buf][slot(r0 + 32 * q, ch)] = v;
            if constexpr (WSRC == kWFlip) {
                if (q < BQ) Bs[buf][slot(r0 + 32 * q, ch)] = R.b[q];
            }
        }
        // forward: k rows 4 kq + i, n 4 n4 .. 4 n4 + 3, as loaded
        if constexpr (WSRC == kWFwd) {
            if (bput) {
                float* bs = reinterpret_cast<float*>(&Bs[buf][0]);
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    *reinterpret_cast<float4*>(bs + kslot<BN>(4 * kq + i, 4 * n4)) = R.b[i];
            }
        }
    };

    f32x16 acc[2][UT];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int u = 0; u < UT; ++u) acc[t][u] = (f32x16){};
    const int nk = sh.KKC / kBK;
    const int fr = lane & 31, fh = lane >> 5;
    // epilogue operands, loaded before the pipeline
    float bn[UT], g = 1.0f;
#pragma unroll
    for (int u = 0; u < UT; ++u) bn[u] = 0.0f;
    if constexpr (EPI == kEpiBias) {
#pragma unroll
        for (int u = 0; u < UT; ++u) bn[u] = bias[n0 + wn * (BN / 2) + 32 * u + fr];
    }
    if constexpr (EPI == kEpiGain) g = gain[0];
    // Fragments of a k quarter (8 k: one 128-bit read per row tile) and the
    // 16 MFMAs on them.  The next quarter's reads are issued before the
    // current quarter's MFMAs (two fragment register sets; the scheduling
    // barriers keep the compiler from sinking the reads below the MFMAs, which
    // would leave the matrix core idle for the LDS latency of every quarter).
    auto frag = [&](int buf, int kq, float4 (&a)[2], float4 (&b)[UT]) {
        const int c = 2 * kq + fh;
#pragma unroll
        for (int t = 0; t < 2; ++t) a[t] = As[buf][slot(wm * 64 + 32 * t + fr, c)];
        if constexpr (WSRC == kWFwd) {
            // component j of b[u] = B[k = 4 c + j][n]: rows 8 kq + 4 fh + j
            const float* bs = reinterpret_cast<const float*>(&Bs[buf][0]);
#pragma unroll
            for (int u = 0; u < UT; ++u) {
                const int n = wn * (BN / 2) + 32 * u + fr;
                b[u].x = bs[kslot<BN>(4 * c + 0, n)];
                b[u].y = bs[kslot<BN>(4 * c + 1, n)];
                b[u].z = bs[kslot<BN>(4 * c + 2, n)];
                b[u].w = bs[kslot<BN>(4 * c + 3, n)];
            }
        } else {
#pragma unroll
            for (int u = 0; u < UT; ++u) b[u] = Bs[buf][slot(wn * (BN / 2) + 32 * u + fr, c)];
        }
    };
    auto mfmas = [&](const float4 (&a)[2], const float4 (&b)[UT]) {
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int u = 0; u < UT; ++u) acc[t][u] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[t].x, b[u].x, acc[t][u], 0, 0, 0);
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int u = 0; u < UT; ++u) acc[t][u] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[t].y, b[u].y, acc[t][u], 0, 0, 0);
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int u = 0; u < UT; ++u) acc[t][u] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[t].z, b[u].z, acc[t][u], 0, 0, 0);
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int u = 0; u < UT; ++u) acc[t][u] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[t].w, b[u].w, acc[t][u], 0, 0, 0);
    };
    auto compute = [&](int buf) {
        float4 a0[2], b0[UT], a1[2], b1[UT];
        frag(buf, 0, a0, b0);
        frag(buf, 1, a1, b1);
        __builtin_amdgcn_sched_barrier(0);
        mfmas(a0, b0);
        __builtin_amdgcn_sched_barrier(0);
        frag(buf, 2, a0, b0);
        __builtin_amdgcn_sched_barrier(0);
        mfmas(a1, b1);
        __builtin_amdgcn_sched_barrier(0);
        frag(buf, 3, a1, b1);
        __builtin_amdgcn_sched_barrier(0);
        mfmas(a0, b0);
        __builtin_amdgcn_sched_barrier(0);
        mfmas(a1, b1);
    };
    // Slices: prologue, a branch-free steady loop over pairs of slices (slice
    // kt computes from LDS buffer kt % 2 while R[kt % 2] receives slice kt + 2
    // and R[(kt + 1) % 2] goes to the other buffer; the second load of a pair
    // is clamped to the last slice, a harmless reload), then the one or two
    // slices left.
    load(0, R0);
    if (nk > 1) load(1, R1);
    store(0, R0);
    __syncthreads();
    int kt = 0;
    for (; kt + 2 < nk; kt += 2) {
        load(kt + 2, R0);
        compute(0);
        store(1, R1);
        __syncthreads();
        load(min(kt + 3, nk - 1), R1);
        compute(1);
        store(0, R0);
        __syncthreads();
    }
    // Fused epilogue operands: all of a lane's are loaded at the start of the
    // epilogue, one round trip (the main loop's registers are free by then).
    // A row past M reads row M - 1 (harmless) and stores nothing.  Offsets are
    // 32-bit (the launcher bounds the tensors below 2^31 elements).
    const int mrow = m0 + wm * 64 + 4 * fh, ncol = n0 + wn * (BN / 2) + fr;
    const int rowlim = sh.M - 1 - mrow;
    const uint32_t lofs = (uint32_t)(mrow * sh.Cout + ncol);
    float e1[UT][2][16], e2[UT][2][16];
    auto fetch = [&](int u) {
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int d = min(32 * t + 8 * (r >> 2) + (r & 3), rowlim);
                const uint32_t off = lofs + (uint32_t)(d * sh.Cout + 32 * u);
                if constexpr ((XE & kXeRes) != 0) e1[u][t][r] = ep.res[off];
                if constexpr ((XE & kXeActG) != 0) e2[u][t][r] = ep.xa[off];
                if constexpr ((XE & kXeMod) != 0) {
                    uint32_t bb, q;
                    ep.hw.divmod((uint32_t)(mrow + d), bb, q);
                    e2[u][t][r] = ep.cond[bb * (uint32_t)sh.Cout + (uint32_t)(ncol + 32 * u)];
                }
            }
    };
    compute(0);
    if (kt + 1 < nk) {
        store(1, R1);
        __syncthreads();
        compute(1);
    }

    // epilogue: lanes 0-31 and 32-63 each write 32 consecutive outputs of a
    // row.  A full row tile stores with no per-row test (a branch per store
    // would make every store wait for all earlier ones).
    auto out = [&](int t, int u, int r) {
        float v = acc[t][u][r];
        if constexpr (EPI == kEpiBias) v = v + bn[u];
        if constexpr (EPI == kEpiGain) v = v * g;
        return v;
    };
    float* yb = Y + (size_t)(m0 + wm * 64 + 4 * fh) * sh.Cout + n0 + wn * (BN / 2) + fr;
    if constexpr (XE != kXeNone) {
#pragma unroll
        for (int u = 0; u < UT; ++u) fetch(u);
#pragma unroll
        for (int u = 0; u < UT; ++u) {
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int dm = 32 * t + 8 * (r >> 2) + (r & 3);
                    if (mrow + dm >= sh.M) continue;
                    float v = out(t, u, r);
                    if constexpr ((XE & kXeActG) != 0) v = v * act_grad<ACT, false>(e2[u][t][r]);
                    if constexpr ((XE & kXeRes) != 0) v = ep.wa * e1[u][t][r] + ep.wb * v;
                    yb[(size_t)dm * sh.Cout + 32 * u] = v;
                    if constexpr ((XE & kXeMod) != 0)
                        ep.y2[(size_t)(mrow + dm) * sh.Cout + ncol + 32 * u] =
                            act_fwd<ACT, false>(v * (e2[u][t][r] + 1.0f));
                }
        }
    } else if (m0 + kBM <= sh.M) {
#pragma unroll
        for (int u = 0; u < UT; ++u)
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    yb[(size_t)(32 * t + 8 * (r >> 2) + (r & 3)) * sh.Cout + 32 * u] = out(t, u, r);
    } else {
#pragma unroll
        for (int u = 0; u < UT; ++u)
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int dm = 32 * t + 8 * (r >> 2) + (r & 3);
                    if (m0 + wm * 64 + 4 * fh + dm < sh.M) yb[(size_t)dm * sh.Cout + 32 * u] = out(t, u, r);
                }
    }
}

// ---------------------------------------------------------------------------
// Weight gradient: gW[k, n] = sum_m A[m, k] dY[m, n] (the reference's
// gemm_dW over the im2col matrix, src/conv2d.c:44-47), with A gathered from X
// as in the forward.  The m reduction (B * Ho * Wo rows) is split over S
// workgroups per 128 x 128 output tile; split z writes its fixed-order partial
// tile to part[z], and a second launch adds the S partials in split order.
//
// Per stage a workgroup stages 32 pixel rows m of A (its 128 k columns) and
// of dY (its BN n columns) in LDS transposed: per column, 8 float4 chunks of
// 4 consecutive m (tslot).  A lane's MFMA operands then run along the pixel
// reduction in one 128-bit read: in quad Q of the stage, lane l reads pixels
// 8 Q + 4 (l / 32) .. + 3 of its column (k, or n, = l % 32 of a 32-column
// block), and component c feeds the c-th MFMA, which pairs pixels 8 Q + c and
// 8 Q + 4 + c of the two half-waves (any pairing gives the same sum, as long
// as A and dY use the same one; this one is fixed).  Each loader thread
// gathers 4 consecutive pixel rows of one 4-column chunk (one pixel decode,
// then steps along the output row) and transposes them in registers into 4
// chunk writes.
// ---------------------------------------------------------------------------
constexpr int kWgM = 32;  // m rows per stage

// float4 slot of (column, chunk of 4 m) in a [columns][8] transposed tile.
// The xor with (col ^ col / 8) mod 8 puts the 16 columns that a 16-lane group
// reads (consecutive columns, one chunk) on 16 distinct bank quads, and the
// columns 4 ch + i that a loader instruction writes (ch = 16 consecutive
// lanes) on at most two lanes per quad.
__device__ __forceinline__ int tslot(int col, int mc) { return col * 8 + (mc ^ ((col ^ (col >> 3)) & 7)); }

// XCD-aware tile order.  Workgroups are dispatched round-robin over the
// device's 8 XCDs (workgroup L on XCD L % 8), each with its own L2.  Tile
// L' = xcd_order(L) gives XCD x a contiguous range of tiles, so the k tiles
// of one m split, which read the same X and dY rows, run in the same L2
// instead of on different XCDs.  A bijection of [0, total) for any total.
constexpr int kXcds = 8;
__device__ __forceinline__ int xcd_order(int L, int total) {
    const int x = L % kXcds, j = L / kXcds, q = total / kXcds, r = total % kXcds;
    return x * q + min(x, r) + j;
}

template <int BN>
__global__ __launch_bounds__(kTpb, 2) void igemm_wgrad(float* __restrict__ part, const float* __restrict__ X,
    const float* __restrict__ dY, ConvShape sh, int rows_per_split) {
    constexpr int UT = BN / 64;               // 32-column accumulator tiles per wave
    constexpr int DCH = BN / 4;               // float4 chunks per dY row
    constexpr int DTHR = DCH * (kWgM / 4);    // dY loader threads: (n chunk, group of 4 rows)
    static_assert(kWgM == 32 && DTHR <= kTpb && kTpb == 32 * (kWgM / 4), "loader roles");
    __shared__ float4 As[2][128 * 8];
    __shared__ float4 Ds[2][BN * 8];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int wk = w >> 1, wn = w & 1;
    // tile (k tile, n tile, split z), k tile fastest, in XCD-aware order
    const int KT = (sh.KKC + 127) / 128, NT = sh.Cout / BN;
    const int tl = xcd_order((int)blockIdx.x, (int)gridDim.x);
    const int k0 = (tl % KT) * 128, n0 = ((tl / KT) % NT) * BN, z = tl / (KT * NT);
    const int mbeg = z * rows_per_split;
    const int mend = min(sh.M, mbeg + rows_per_split);
    // loader roles: A chunk ch (k = k0 + 4 ch .. + 3) of the stage's pixel rows
    // 4 g .. 4 g + 3; dY chunk dch (n = n0 + 4 dch .. + 3) of rows 4 dg .. + 3
    const int ch = tid & 31, g = tid >> 5;
    const int dch = tid % DCH, dg = tid / DCH;
    const bool dld = tid < DTHR;
    const int kc = k0 + 4 * ch;
    const bool kok = kc < sh.KKC;
    const int tap = kok ? kc / sh.Cin : 0, ci = kok ? kc - tap * sh.Cin : 0;
    const int kh = tap / sh.K, kw = tap - kh * sh.K;
    const float* dcol = dY + n0 + 4 * dch;
    const uint32_t Wo = (uint32_t)sh.Wo, Ho = (uint32_t)sh.Ho;

    // Two register sets: the stage two ahead is loaded while the next one is
    // written to LDS, so a load has two stages of MFMA work to arrive.  Every
    // lane loads (rows past the end, padding and the idle dY loaders of a
    // 64-column tile read a valid address and are zeroed when stored): a
    // branch around a load would make the compiler's later waits drain the
    // whole vector-memory counter.
    struct Regs {
        float4 a[4], d[4];
        bool aok[4], dok[4];
    };
    Regs R0, R1;
    auto load = [&](int ms, Regs& R) {
        // decode the first of the 4 rows once, then step along the output row
        const int m0 = ms + 4 * g;
        uint32_t t, ow, b, oh;
        sh.wo.divmod((uint32_t)(m0 < sh.M ? m0 : 0), t, ow);
        sh.ho.divmod(t, b, oh);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int ih = (int)oh * sh.stride - sh.pad + kh, iw = (int)ow * sh.stride - sh.pad + kw;
            R.aok[q] = (m0 + q < mend) & kok & ((unsigned)ih < (unsigned)sh.H) & ((unsigned)iw < (unsigned)sh.W);
            const int p = R.aok[q] ? ((int)b * sh.H + ih) * sh.W + iw : 0;
            // 32-bit element offsets (the host bounds x and dy below 2^31
            // elements): same-box A/B 346.5 -> 343.7 us at cfg3 against 64-bit
            // products; the forward's loader measured slower with the same change
            R.a[q] = ld4(X + (uint32_t)(p * sh.Cin + ci));
            if (++ow == Wo) {
                ow = 0;
                if (++oh == Ho) {
                    oh = 0;
                    ++b;
                }
            }
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int m = ms + 4 * dg + q;
            R.dok[q] = dld & (m < mend);
            R.d[q] = ld4(dcol + (uint32_t)((R.dok[q] ? m : 0) * sh.Cout));
        }
    };
    auto mask4 = [](float4 v, bool ok) {
        const unsigned mk = ok ? 0xffffffffu : 0u;
        v.x = __uint_as_float(__float_as_uint(v.x) & mk);
        v.y = __uint_as_float(__float_as_uint(v.y) & mk);
        v.z = __uint_as_float(__float_as_uint(v.z) & mk);
        v.w = __uint_as_float(__float_as_uint(v.w) & mk);
        return v;
    };
    // 4 rows x 4 columns in registers -> 4 column chunks (rows 4 gg .. + 3)
    auto put = [&](float4* tile, int col0, int gg, const float4 (&v)[4], const bool (&ok)[4]) {
        const float4 r0 = mask4(v[0], ok[0]), r1 = mask4(v[1], ok[1]), r2 = mask4(v[2], ok[2]),
                     r3 = mask4(v[3], ok[3]);
        tile[tslot(col0 + 0, gg)] = make_float4(r0.x, r1.x, r2.x, r3.x);
        tile[tslot(col0 + 1, gg)] = make_float4(r0.y, r1.y, r2.y, r3.y);
        tile[tslot(col0 + 2, gg)] = make_float4(r0.z, r1.z, r2.z, r3.z);
        tile[tslot(col0 + 3, gg)] = make_float4(r0.w, r1.w, r2.w, r3.w);
    };
    auto store = [&](int buf, const Regs& R) {
        put(As[buf], 4 * ch, g, R.a, R.aok);
        if (dld) put(Ds[buf], 4 * dch, dg, R.d, R.dok);
    };
    f32x16 acc[2][UT];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int u = 0; u < UT; ++u) acc[t][u] = (f32x16){};
    const int fr = lane & 31, fh = lane >> 5;
    // Operands of quad Q (pixels 8 Q .. 8 Q + 7) and their MFMAs.  Two operand
    // register sets: the reads of quad Q + 2 are issued right after the MFMAs
    // of quad Q (the scheduling barriers keep them there), so each quad's
    // reads have the next quad's 4 x 2 x UT MFMAs to arrive.
    auto qfrag = [&](int buf, int Q, float4 (&a)[2], float4 (&d)[UT]) {
        const int mc = 2 * Q + fh;
#pragma unroll
        for (int t = 0; t < 2; ++t) a[t] = As[buf][tslot(wk * 64 + 32 * t + fr, mc)];
#pragma unroll
        for (int u = 0; u < UT; ++u) d[u] = Ds[buf][tslot(wn * (BN / 2) + 32 * u + fr, mc)];
    };
    // component-major: the 2 x UT accumulators in turn, so consecutive MFMAs
    // never wait for each other's result
    auto qmfma = [&](const float4 (&a)[2], const float4 (&d)[UT]) {
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int u = 0; u < UT; ++u) acc[t][u] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[t].x, d[u].x, acc[t][u], 0, 0, 0);
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int u = 0; u < UT; ++u) acc[t][u] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[t].y, d[u].y, acc[t][u], 0, 0, 0);
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int u = 0; u < UT; ++u) acc[t][u] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[t].z, d[u].z, acc[t][u], 0, 0, 0);
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int u = 0; u < UT; ++u) acc[t][u] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[t].w, d[u].w, acc[t][u], 0, 0, 0);
    };
    auto compute = [&](int buf) {
        float4 a0[2], d0[UT], a1[2], d1[UT];
        qfrag(buf, 0, a0, d0);
        qfrag(buf, 1, a1, d1);
        __builtin_amdgcn_sched_barrier(0);
        qmfma(a0, d0);
        __builtin_amdgcn_sched_barrier(0);
        qfrag(buf, 2, a0, d0);
        __builtin_amdgcn_sched_barrier(0);
        qmfma(a1, d1);
        __builtin_amdgcn_sched_barrier(0);
        qfrag(buf, 3, a1, d1);
        __builtin_amdgcn_sched_barrier(0);
        qmfma(a0, d0);
        __builtin_amdgcn_sched_barrier(0);
        qmfma(a1, d1);
        __builtin_amdgcn_sched_barrier(0);
    };
    // Stages: prologue, a branch-free steady loop over pairs of stages (stage
    // st computes from LDS buffer st % 2 while R[st % 2] receives stage st + 2
    // and R[(st + 1) % 2] goes to the other buffer; the second load of a pair
    // is clamped to the last stage, a harmless reload), then the one or two
    // stages left.
    const int nst = (mend - mbeg + kWgM - 1) / kWgM;
    if (nst > 0) {
        load(mbeg, R0);
        if (nst > 1) load(mbeg + kWgM, R1);
        store(0, R0);
        __syncthreads();
        int st = 0;
        for (; st + 2 < nst; st += 2) {
            load(mbeg + (st + 2) * kWgM, R0);
            compute(0);
            store(1, R1);
            __syncthreads();
            load(mbeg + min(st + 3, nst - 1) * kWgM, R1);
            compute(1);
            store(0, R0);
            __syncthreads();
        }
        compute(0);
        if (st + 1 < nst) {
            store(1, R1);
            __syncthreads();
            compute(1);
        }
    }
    // partial tile: D[k][n], rows k = k0 + wk 64 + 32 t + 8 (r / 4) + 4 h + r % 4
    float* pb = part + (size_t)z * sh.KKC * sh.Cout + (size_t)(k0 + wk * 64 + 4 * fh) * sh.Cout + n0 + wn * (BN / 2) + fr;
#pragma unroll
    for (int u = 0; u < UT; ++u)
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int dk = 32 * t + 8 * (r >> 2) + (r & 3);
                if (k0 + wk * 64 + 4 * fh + dk < sh.KKC) pb[(size_t)dk * sh.Cout + 32 * u] = acc[t][u][r];
            }
}

// gW[i] = part[0][i] + part[1][i] + ... (split order).
__global__ __launch_bounds__(256) void wgrad_reduce(float* __restrict__ gW, const float* __restrict__ part, int S,
    long long n) {
    const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    // kB slices in flight, added in slice order
    constexpr int kB = 8;
    float t = part[i];
    int z = 1;
    for (; z + kB <= S; z += kB) {
        float v[kB];
#pragma unroll
        for (int u = 0; u < kB; ++u) v[u] = part[(size_t)(z + u) * n + i];
#pragma unroll
        for (int u = 0; u < kB; ++u) t += v[u];
    }
    for (; z < S; ++z) t += part[(size_t)z * n + i];
    gW[i] = t;
}

struct WgradPlan {
    int S, rows;
};

int tile_n(int Cout) { return Cout % 128 == 0 ? 128 : 64; }

WgradPlan wgrad_plan(int M, int KKC, int Cout) {
    const int tiles = ((KKC + 127) / 128) * (Cout / tile_n(Cout));
    // one round of resident workgroups (two per CU on 256 CUs)
    int S = tiles >= 512 ? 1 : 512 / tiles;
    const int smax = (M + kWgM - 1) / kWgM;
    if (S > smax) S = smax;
    if (S < 1) S = 1;
    int rows = (M + S - 1) / S;
    rows = (rows + kWgM - 1) / kWgM * kWgM;
    WgradPlan p;
    p.rows = rows;
    p.S = (M + rows - 1) / rows;
    return p;
}


// Checks shared by the forward launchers (plain and fused): -1 after
// recording an error, 0 when there is nothing to do (batch 0), 1 with `sh`
// filled in.
inline int fwd_setup(const char* what, const float* Y, const float* X, const float* Wt, const float* bias,
    const float* gain, int batch, int H, int W, int C_in, int C_out, int K, int stride, int pad, int H_out,
    int W_out, ConvShape& sh) {
    NNK_REQUIRE_RET(batch >= 0 && H > 0 && W > 0 && K > 0 && stride > 0 && pad >= 0, -1, what,
        "%s: bad geometry", what);
    NNK_REQUIRE_RET(nnhip_conv2d_implicit_supported(C_in, C_out), -1, what,
        "%s: needs C_in %% %d == 0 and C_out %% %d == 0 (C_in=%d C_out=%d)", what, kBK, kBNmin, C_in, C_out);
    NNK_REQUIRE_RET(H_out == (H + 2 * pad - K) / stride + 1 && W_out == (W + 2 * pad - K) / stride + 1 &&
                        H_out > 0 && W_out > 0,
        -1, what, "%s: output size %dx%d does not match the geometry", what, H_out, W_out);
    NNK_REQUIRE_RET((long long)batch * H * W * C_in < (1LL << 31) &&
                        (long long)batch * H_out * W_out * C_out < (1LL << 31),
        -1, what, "%s: tensor exceeds the 32-bit index range", what);
    NNK_REQUIRE_RET(!(bias && gain), -1, what, "%s: bias and gain are exclusive", what);
    if (batch == 0) return 0;
    NNK_REQUIRE_RET(Y && X && Wt, -1, what, "%s: null pointer", what);
    NNK_REQUIRE_RET(aligned16(X) && aligned16(Wt), -1, what, "%s: x and the weight must be 16-byte aligned", what);
    sh = ConvShape{batch, H, W, C_in, C_out, K, stride, pad, H_out, W_out, batch * H_out * W_out, K * K * C_in,
        FastDiv((uint32_t)W_out), FastDiv((uint32_t)H_out)};
    return 1;
}

// Checks shared by the input-gradient launchers; `sh` is then the stride-1
// convolution of dy (Ho x Wo x C_out) with the flipped kernel and padding
// K-1-pad, whose output is H x W x C_in.
inline int dgrad_setup(const char* what, const float* dX, const float* dY, const float* Wt, int batch, int H, int W,
    int C_in, int C_out, int K, int pad, ConvShape& sh) {
    NNK_REQUIRE_RET(batch >= 0 && H > 0 && W > 0 && K > 0 && pad >= 0, -1, what, "%s: bad geometry", what);
    NNK_REQUIRE_RET(nnhip_conv2d_input_grad_implicit_supported(C_in, C_out, K, 1, pad), -1, what,
        "%s: needs pad <= K - 1, C_out %% %d == 0 and C_in %% %d == 0 (C_in=%d C_out=%d K=%d pad=%d)", what, kBK,
        kBNmin, C_in, C_out, K, pad);
    const int Ho = H + 2 * pad - K + 1, Wo = W + 2 * pad - K + 1;
    NNK_REQUIRE_RET(Ho > 0 && Wo > 0, -1, what, "%s: empty output for this geometry", what);
    NNK_REQUIRE_RET((long long)batch * H * W * C_in < (1LL << 31) && (long long)batch * Ho * Wo * C_out < (1LL << 31) &&
                        (long long)K * K * C_in * C_out < (1LL << 31),
        -1, what, "%s: tensor exceeds the 32-bit index range", what);
    if (batch == 0) return 0;
    NNK_REQUIRE_RET(dX && dY && Wt, -1, what, "%s: null pointer", what);
    NNK_REQUIRE_RET(aligned16(dY) && aligned16(Wt), -1, what, "%s: dy and the weight must be 16-byte aligned", what);
    sh = ConvShape{batch, Ho, Wo, C_out, C_in, K, 1, K - 1 - pad, H, W, batch * H * W, K * K * C_out,
        FastDiv((uint32_t)W), FastDiv((uint32_t)H)};
    return 1;
}

void wgrad_launch(const char* what, float* gW, const float* X, const float* dY, int batch, int H, int W, int C_in,
    int C_out, int K, int stride, int pad, int H_out, int W_out, float* workspace, hipStream_t s) {
    NNK_REQUIRE(batch >= 0 && H > 0 && W > 0 && K > 0 && stride > 0 && pad >= 0, what, "%s: bad geometry", what);
    NNK_REQUIRE(nnhip_conv2d_wgrad_implicit_supported(C_in, C_out), what,
        "%s: needs C_in %% 4 == 0 and C_out %% %d == 0 (C_in=%d C_out=%d)", what, kBNmin, C_in, C_out);
    NNK_REQUIRE(H_out == (H + 2 * pad - K) / stride + 1 && W_out == (W + 2 * pad - K) / stride + 1 && H_out > 0 &&
                    W_out > 0,
        what, "%s: output size %dx%d does not match the geometry", what, H_out, W_out);
    NNK_REQUIRE((long long)batch * H * W * C_in < (1LL << 31) && (long long)batch * H_out * W_out * C_out < (1LL << 31),
        what, "%s: tensor exceeds the 32-bit index range", what);
    NNK_REQUIRE(gW && (batch == 0 || (X && dY)), what, "%s: null pointer", what);
    const int KKC = K * K * C_in;
    if (batch == 0) {
        nnhip_fill_f32(gW, 0.0f, (size_t)KKC * C_out, s);
        return;
    }
    NNK_REQUIRE(aligned16(X) && aligned16(dY), what, "%s: X and dY must be 16-byte aligned", what);
    ConvShape sh{batch, H, W, C_in, C_out, K, stride, pad, H_out, W_out, batch * H_out * W_out, KKC,
        FastDiv((uint32_t)W_out), FastDiv((uint32_t)H_out)};
    const WgradPlan p = wgrad_plan(sh.M, KKC, C_out);
    float* part = gW;
    bool pooled = false;
    if (p.S > 1) {
        if (workspace) {
            part = workspace;
        } else {
            part = nnk_scratch_acquire((size_t)p.S * KKC * C_out, s, what);
            if (!part) return;
            pooled = true;
        }
    }
    const int BN = tile_n(C_out);
    const dim3 grid((unsigned)((KKC + 127) / 128) * (unsigned)(C_out / BN) * (unsigned)p.S);
    if (BN == 128) igemm_wgrad<128><<<grid, kTpb, 0, s>>>(part, X, dY, sh, p.rows);
    else igemm_wgrad<64><<<grid, kTpb, 0, s>>>(part, X, dY, sh, p.rows);
    if (p.S > 1) {
        const long long n = (long long)KKC * C_out;
        wgrad_reduce<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(gW, part, p.S, n);
    }
    if (pooled) nnk_scratch_release(part, s);
    nnk_after_launch(what, s);
}

}  // namespace

