// gn_kernels.h -- NHWC GroupNorm (+ fused activation) kernels for gfx950.
//
// Reference maths: src/kernels.cu:622-717 (forward, backward-x, backward-param)
// composed with the activation of src/kernels.cu:21-68 as the DDPM block does
// (src/conv_residual.c:28-29, 51-52).
//
// Layout: x, y, dx, dy are [B, HW, C] row-major (NHWC with H*W flattened);
// group g of sample b owns channels [g*cpg, (g+1)*cpg) of every pixel, i.e.
// cpg contiguous floats at a stride of C floats.  mu/rstd are [B*G].
//
// Register-resident path (gn_fwd_reg / gn_bwd_reg): one workgroup per (b, g)
// holds the whole group in VGPRs, so x (and dy) cross HBM exactly once:
//   forward  : read x, write y                    =  8 B/elem
//   backward : read x and dy, write dx            = 12 B/elem
// (+ B*C*2 floats of per-sample channel partials for dgamma/dbeta, reduced
// over the batch by gn_param_reduce in a fixed order).
// Thread t owns float4 slot `sub = t % V4PP` of pixels p0 + k*PSTEP.
#pragma once

#include "nnk_common.h"

namespace nnk {
namespace gn {

// ---------------------------------------------------------------------------
// Forward, register resident.
// ---------------------------------------------------------------------------
template <int TPB, int NV, int V4PP, int ACT>
__global__ __launch_bounds__(TPB) void gn_fwd_reg(float* __restrict__ y,
    float* __restrict__ mu_out, float* __restrict__ rstd_out,
    const float* __restrict__ x, const float* __restrict__ gamma,
    const float* __restrict__ beta, int G, int HW, int C, float eps) {
    constexpr int NW = TPB / kWave;
    constexpr int PSTEP = TPB / V4PP;
    constexpr int CPG = 4 * V4PP;
    __shared__ float red[2 * NW];

    const int work = xcd_swizzle(blockIdx.x, gridDim.x);
    const int b = work / G;
    const int g = work - b * G;
    const int tid = threadIdx.x;
    const int sub = tid % V4PP;
    const int p0 = tid / V4PP;
    const size_t off = (size_t)b * HW * C + (size_t)g * CPG + (size_t)sub * 4;
    const float* xb = x + off;
    float* yb = y + off;

    float4 v[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int p = p0 + k * PSTEP;
        if (p < HW) v[k] = ld4(xb + (size_t)p * C);
        else v[k] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }

    // mean: padded slots hold 0 and add nothing
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k) s += (v[k].x + v[k].y) + (v[k].z + v[k].w);
    const float nf = (float)(HW * CPG);
    const float mean = block_sum<NW>(s, red) / nf;

    // variance about the mean, from the registers (no second HBM pass)
    float q = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        if (p0 + k * PSTEP < HW) {
            const float a = v[k].x - mean, bb = v[k].y - mean;
            const float c = v[k].z - mean, d = v[k].w - mean;
            q += (a * a + bb * bb) + (c * c + d * d);
        }
    }
    const float var = block_sum<NW>(q, red + NW) / nf;
    const float rs = rsqrtf(var + eps);
    if (tid == 0) {
        mu_out[work] = mean;
        rstd_out[work] = rs;
    }

    const float4 gm = ld4(gamma + g * CPG + sub * 4);
    const float4 bt = ld4(beta + g * CPG + sub * 4);
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int p = p0 + k * PSTEP;
        if (p < HW) {
            float4 o;
            o.x = act_fwd<ACT>(gm.x * ((v[k].x - mean) * rs) + bt.x);
            o.y = act_fwd<ACT>(gm.y * ((v[k].y - mean) * rs) + bt.y);
            o.z = act_fwd<ACT>(gm.z * ((v[k].z - mean) * rs) + bt.z);
            o.w = act_fwd<ACT>(gm.w * ((v[k].w - mean) * rs) + bt.w);
            st4(yb + (size_t)p * C, o);
        }
    }
}

// ---------------------------------------------------------------------------
// Backward, register resident.  dy is the gradient of act(GN(x)); the
// pre-activation h = gamma*xhat + beta is recomputed.  Writes dx and the
// per-(b, channel) partials  part_g[b*C+c] = sum_hw d*xhat,
// part_b[b*C+c] = sum_hw d, with d = dy * act'(h).
// ---------------------------------------------------------------------------
template <int TPB, int NV, int V4PP, int ACT>
__global__ __launch_bounds__(TPB) void gn_bwd_reg(float* __restrict__ dx,
    float* __restrict__ part_g, float* __restrict__ part_b,
    const float* __restrict__ dy, const float* __restrict__ x,
    const float* __restrict__ gamma, const float* __restrict__ beta,
    const float* __restrict__ mu, const float* __restrict__ rstd,
    int G, int HW, int C) {
    constexpr int NW = TPB / kWave;
    constexpr int PSTEP = TPB / V4PP;
    constexpr int CPG = 4 * V4PP;
    __shared__ float red[2 * NW];
    __shared__ float cred[NW][V4PP][8];

    const int work = xcd_swizzle(blockIdx.x, gridDim.x);
    const int b = work / G;
    const int g = work - b * G;
    const int tid = threadIdx.x;
    const int sub = tid % V4PP;
    const int p0 = tid / V4PP;
    const size_t off = (size_t)b * HW * C + (size_t)g * CPG + (size_t)sub * 4;

    float4 xv[NV], gv[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int p = p0 + k * PSTEP;
        if (p < HW) {
            xv[k] = ld4(x + off + (size_t)p * C);
            gv[k] = ld4(dy + off + (size_t)p * C);
        } else {
            xv[k] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            gv[k] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
    }

    const float mean = mu[work];
    const float rs = rstd[work];
    const float4 gm = ld4(gamma + g * CPG + sub * 4);
    float4 bt = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if constexpr (ACT != ACT_IDENTITY) bt = ld4(beta + g * CPG + sub * 4);

    float pg = 0.0f, pgx = 0.0f;
    float4 cg = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    float4 cb = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        if (p0 + k * PSTEP < HW) {
            float4 xh, d, gg;
            xh.x = (xv[k].x - mean) * rs;
            xh.y = (xv[k].y - mean) * rs;
            xh.z = (xv[k].z - mean) * rs;
            xh.w = (xv[k].w - mean) * rs;
            d = gv[k];
            if constexpr (ACT != ACT_IDENTITY) {
                d.x = d.x * act_grad<ACT>(gm.x * xh.x + bt.x);
                d.y = d.y * act_grad<ACT>(gm.y * xh.y + bt.y);
                d.z = d.z * act_grad<ACT>(gm.z * xh.z + bt.z);
                d.w = d.w * act_grad<ACT>(gm.w * xh.w + bt.w);
            }
            cg.x += d.x * xh.x;
            cg.y += d.y * xh.y;
            cg.z += d.z * xh.z;
            cg.w += d.w * xh.w;
            cb.x += d.x;
            cb.y += d.y;
            cb.z += d.z;
            cb.w += d.w;
            gg.x = d.x * gm.x;
            gg.y = d.y * gm.y;
            gg.z = d.z * gm.z;
            gg.w = d.w * gm.w;
            pg += (gg.x + gg.y) + (gg.z + gg.w);
            pgx += (gg.x * xh.x + gg.y * xh.y) + (gg.z * xh.z + gg.w * xh.w);
            xv[k] = xh;
            gv[k] = gg;
        }
    }

    block_sum2<NW>(pg, pgx, red);
    const float nf = (float)(HW * CPG);
    const float inv_n = 1.0f / nf;
    const float m1 = pg * inv_n;

#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int p = p0 + k * PSTEP;
        if (p < HW) {
            float4 o;
            o.x = rs * ((gv[k].x - m1) - xv[k].x * pgx * inv_n);
            o.y = rs * ((gv[k].y - m1) - xv[k].y * pgx * inv_n);
            o.z = rs * ((gv[k].z - m1) - xv[k].z * pgx * inv_n);
            o.w = rs * ((gv[k].w - m1) - xv[k].w * pgx * inv_n);
            st4(dx + off + (size_t)p * C, o);
        }
    }

    // per-channel partials: lanes with equal `sub` own the same 4 channels
    float c8[8] = {cg.x, cg.y, cg.z, cg.w, cb.x, cb.y, cb.z, cb.w};
#pragma unroll
    for (int j = 0; j < 8; ++j) c8[j] = wave_sum_strided<V4PP>(c8[j]);
    const int lane = tid & (kWave - 1);
    const int wid = tid / kWave;
    if (lane < V4PP) {
#pragma unroll
        for (int j = 0; j < 8; ++j) cred[wid][lane][j] = c8[j];
    }
    __syncthreads();
    if (tid < V4PP * 8) {
        const int s2 = tid / 8;
        const int j = tid % 8;
        float acc = cred[0][s2][j];
#pragma unroll
        for (int w = 1; w < NW; ++w) acc += cred[w][s2][j];
        const size_t ch = (size_t)b * C + (size_t)g * CPG + s2 * 4 + (j & 3);
        if (j < 4) part_g[ch] = acc;
        else part_b[ch] = acc;
    }
}

// Launch-shape table of the register-resident path: TPB threads x NV float4
// per thread covers groups of up to TPB*NV float4.
struct RegConfig {
    int tpb;
    int nv;
};
constexpr RegConfig kRegConfigs[] = {{256, 1}, {256, 4}, {512, 4}, {1024, 4}, {1024, 8}};
constexpr int kNumRegConfigs = sizeof(kRegConfigs) / sizeof(kRegConfigs[0]);

// Index into kRegConfigs for a group of nf4 float4, or -1 when too large.
inline int pick_reg_config(long long nf4) {
    for (int i = 0; i < kNumRegConfigs; ++i)
        if ((long long)kRegConfigs[i].tpb * kRegConfigs[i].nv >= nf4) return i;
    return -1;
}

}  // namespace gn
}  // namespace nnk

// Dispatchers (one translation unit each); return false when no variant fits.
bool nnk_gn_fwd_reg_dispatch(int cfg, int v4pp, int act, float* y, float* mu, float* rstd,
    const float* x, const float* gamma, const float* beta,
    int B, int G, int HW, int C, float eps, hipStream_t s);
bool nnk_gn_bwd_reg_dispatch(int cfg, int v4pp, int act, float* dx, float* part_g, float* part_b,
    const float* dy, const float* x, const float* gamma, const float* beta,
    const float* mu, const float* rstd, int B, int G, int HW, int C, hipStream_t s);
