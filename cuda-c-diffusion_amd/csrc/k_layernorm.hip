// k_layernorm.hip -- per-row LayerNorm forward/backward.
// Reference maths: src/kernels.cu:491-567 (two-pass mean/variance, eps inside
// the rsqrt; dx = rstd*(g - mean(g) - xhat*mean(g*xhat)), g = dy*gamma;
// dgamma/dbeta are column sums over the rows) with launchers 594-616.
//
// Fast path (C % 4 == 0, C <= 1024, 16-byte aligned): one wave per row, lane
// l owns float4 slots l, l+64, ...; each wave keeps RB rows in flight.
//   forward : read x, write y           =  8 B/elem
//   backward: read x, dy, write dx      = 12 B/elem
//             + per-workgroup channel partials (2*C floats per 64 rows with
//               4-wave workgroups; per 256 rows with 16-wave workgroups, which
//               C <= 256 takes when the rows give every CU one), stored in
//               16-channel chunks and summed in a fixed order by one more
//               launch (one workgroup per chunk and kind, reading its chunk
//               as one contiguous run): ln_colsum_small up to 256 partial
//               rows, ln_colsum_chunk above.
// Generic path: one 256-thread block per row plus a coalesced partial kernel.
// The fast path streams x, dy, y, dx with nontemporal loads and stores when
// the launch is large (use_nt).
#include "nnk_common.h"

namespace {

using namespace nnk;

constexpr int kTpb = 256;
constexpr int kNw = kTpb / kWave;
constexpr int kRowsPerWave = 16;  // fast backward: rows per wave
constexpr int kWideWaves = 16;    // fast backward: waves of a 1024-thread workgroup
// Backward partial granularity: 64 rows per partial row on the generic path
// and the fast path's 4-wave workgroups, NWV * 16 with NWV waves; 64 is the
// smallest, so the workspace is sized by it.
constexpr int kRowsPerWg = 64;
static_assert(kRowsPerWg == 4 * kRowsPerWave, "a 4-wave workgroup writes one partial row per kRowsPerWg rows");
// The dgamma/dbeta partials of partial row p lie in
// chunks of kCw channels: channel c at part[((c / kCw) * P + p) * kCw + c % kCw],
// P partial rows.  A chunk's P rows are one contiguous run of P * 64 bytes.
constexpr int kCw = 16;
__device__ __forceinline__ size_t part_index(int c, int p, int P) {
    return ((size_t)(c / kCw) * P + p) * kCw + (c % kCw);
}

// ----------------------------------------------------------------------------
// Fast forward: NV float4 per lane per row, RB rows per wave at a time.
// ----------------------------------------------------------------------------
template <int NV, int RB, bool NT>
__global__ __launch_bounds__(kTpb) void ln_fwd_wave(float* __restrict__ y,
    float* __restrict__ mu, float* __restrict__ rstd, const float* __restrict__ x,
    const float* __restrict__ gamma, const float* __restrict__ beta, int rows, int C, float eps) {
    const int lane = threadIdx.x & (kWave - 1);
    const int wid = threadIdx.x / kWave;
    const int C4 = C / 4;
    const int r0 = (blockIdx.x * kNw + wid) * RB;
    const float cf = (float)C;

    float4 v[RB][NV];
#pragma unroll
    for (int r = 0; r < RB; ++r) {
        const int row = r0 + r;
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const int c4 = lane + k * kWave;
            if (row < rows && c4 < C4) v[r][k] = ldS<NT>(x + (size_t)row * C + 4 * c4);
            else v[r][k] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
    }
    // gamma and beta once per wave, after the rows' loads are out
    float4 gmv[NV], btv[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int c4 = lane + k * kWave;
        gmv[k] = c4 < C4 ? ld4(gamma + 4 * c4) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        btv[k] = c4 < C4 ? ld4(beta + 4 * c4) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
#pragma unroll
    for (int r = 0; r < RB; ++r) {
        const int row = r0 + r;
        float s = 0.0f;
#pragma unroll
        for (int k = 0; k < NV; ++k) s += (v[r][k].x + v[r][k].y) + (v[r][k].z + v[r][k].w);
        const float m = wave_sum(s) / cf;
        float q = 0.0f;
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            if (lane + k * kWave < C4) {
                const float a = v[r][k].x - m, b = v[r][k].y - m;
                const float c = v[r][k].z - m, d = v[r][k].w - m;
                q += (a * a + b * b) + (c * c + d * d);
            }
        }
        const float rs = rsqrtf(wave_sum(q) / cf + eps);
        if (row < rows) {
            if (lane == 0) {
                mu[row] = m;
                rstd[row] = rs;
            }
#pragma unroll
            for (int k = 0; k < NV; ++k) {
                const int c4 = lane + k * kWave;
                if (c4 < C4) {
                    const float4 gm = gmv[k], bt = btv[k];
                    float4 o;
                    o.x = gm.x * ((v[r][k].x - m) * rs) + bt.x;
                    o.y = gm.y * ((v[r][k].y - m) * rs) + bt.y;
                    o.z = gm.z * ((v[r][k].z - m) * rs) + bt.z;
                    o.w = gm.w * ((v[r][k].w - m) * rs) + bt.w;
                    stS<NT>(y + (size_t)row * C + 4 * c4, o);
                }
            }
        }
    }
}

// ----------------------------------------------------------------------------
// Fast backward: each of the NWV waves of workgroup b walks 16 rows, RB at a
// time (PIPE: the next RB rows' loads are issued before the current rows'
// maths), then the waves' channel sums are added in LDS in wave order into
// partial row b of part_g/part_b (part_index, P = gridDim.x).  The rows of
// wave w: with CYC, i * (waves of the grid) + (b NWV + w) for i = 0..15, so
// that each step of the grid reads one contiguous band of rows; otherwise the
// block [NWV 16 b + 16 w, + 16).
// ----------------------------------------------------------------------------
template <int NV, int RB, int NWV, bool PIPE, bool CYC, bool NT>
__global__ __launch_bounds__(NWV * kWave) void ln_bwd_wave(float* __restrict__ dx,
    float* __restrict__ part_g, float* __restrict__ part_b, const float* __restrict__ dy,
    const float* __restrict__ x, const float* __restrict__ gamma,
    const float* __restrict__ mu, const float* __restrict__ rstd, int rows, int C) {
    constexpr int TPB = NWV * kWave;
    constexpr int kSteps = kRowsPerWave / RB;
    static_assert(kRowsPerWave % RB == 0, "whole steps");
    __shared__ float4 lds[NWV][2][NV][kWave];
    const int lane = threadIdx.x & (kWave - 1);
    const int wid = threadIdx.x / kWave;
    const int C4 = C / 4;
    const float invC = 1.0f / (float)C;

    float4 gm[NV];
    float4 cg[NV], cb[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int c4 = lane + k * kWave;
        gm[k] = c4 < C4 ? ld4(gamma + 4 * c4) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        cg[k] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        cb[k] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }

    const int wrow0 = blockIdx.x * (NWV * kRowsPerWave) + wid * kRowsPerWave;
    const int gw = blockIdx.x * NWV + wid, nwt = gridDim.x * NWV;
    auto row_of = [&](int i) { return CYC ? i * nwt + gw : wrow0 + i; };
    constexpr int NB = PIPE ? 2 : 1;  // row buffers
    float4 xv[NB][RB][NV], gv[NB][RB][NV];
    auto load = [&](int buf, int it) {
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            const int row = row_of(it + r);
#pragma unroll
            for (int k = 0; k < NV; ++k) {
                const int c4 = lane + k * kWave;
                if (row < rows && c4 < C4) {
                    xv[buf][r][k] = ldS<NT>(x + (size_t)row * C + 4 * c4);
                    gv[buf][r][k] = ldS<NT>(dy + (size_t)row * C + 4 * c4);
                } else {
                    xv[buf][r][k] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                    gv[buf][r][k] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                }
            }
        }
    };
    auto compute = [&](int buf, int it) {
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            const int row = row_of(it + r);
            if (row >= rows) break;  // wave-uniform
            const float m = mu[row], rs = rstd[row];
            float pg = 0.0f, pgx = 0.0f;
#pragma unroll
            for (int k = 0; k < NV; ++k) {
                if (lane + k * kWave < C4) {
                    float4 xh, g;
                    xh.x = (xv[buf][r][k].x - m) * rs;
                    xh.y = (xv[buf][r][k].y - m) * rs;
                    xh.z = (xv[buf][r][k].z - m) * rs;
                    xh.w = (xv[buf][r][k].w - m) * rs;
                    const float4 d = gv[buf][r][k];
                    cg[k].x += d.x * xh.x;
                    cg[k].y += d.y * xh.y;
                    cg[k].z += d.z * xh.z;
                    cg[k].w += d.w * xh.w;
                    cb[k].x += d.x;
                    cb[k].y += d.y;
                    cb[k].z += d.z;
                    cb[k].w += d.w;
                    g.x = d.x * gm[k].x;
                    g.y = d.y * gm[k].y;
                    g.z = d.z * gm[k].z;
                    g.w = d.w * gm[k].w;
                    pg += (g.x + g.y) + (g.z + g.w);
                    pgx += (g.x * xh.x + g.y * xh.y) + (g.z * xh.z + g.w * xh.w);
                    xv[buf][r][k] = xh;
                    gv[buf][r][k] = g;
                }
            }
            const float S1 = wave_sum(pg), S2 = wave_sum(pgx);
            const float m1 = S1 * invC;
#pragma unroll
            for (int k = 0; k < NV; ++k) {
                const int c4 = lane + k * kWave;
                if (c4 < C4) {
                    float4 o;
                    o.x = rs * ((gv[buf][r][k].x - m1) - xv[buf][r][k].x * S2 * invC);
                    o.y = rs * ((gv[buf][r][k].y - m1) - xv[buf][r][k].y * S2 * invC);
                    o.z = rs * ((gv[buf][r][k].z - m1) - xv[buf][r][k].z * S2 * invC);
                    o.w = rs * ((gv[buf][r][k].w - m1) - xv[buf][r][k].w * S2 * invC);
                    stS<NT>(dx + (size_t)row * C + 4 * c4, o);
                }
            }
        }
    };
    if constexpr (PIPE) {
        load(0, 0);
#pragma unroll
        for (int st = 0; st < kSteps; ++st) {
            if (st + 1 < kSteps) load((st + 1) & 1, (st + 1) * RB);
            compute(st & 1, st * RB);
        }
    } else {
#pragma unroll
        for (int st = 0; st < kSteps; ++st) {
            load(0, st * RB);
            compute(0, st * RB);
        }
    }

#pragma unroll
    for (int k = 0; k < NV; ++k) {
        lds[wid][0][k][lane] = cg[k];
        lds[wid][1][k][lane] = cb[k];
    }
    __syncthreads();
    // thread t < 2*NV*64 adds one (kind, k, lane) float4 over the waves in order
    for (int t = threadIdx.x; t < 2 * NV * kWave; t += TPB) {
        const int kind = t / (NV * kWave);
        const int k = (t / kWave) % NV;
        const int l = t % kWave;
        const int c4 = l + k * kWave;
        if (c4 < C4) {
            float4 a = lds[0][kind][k][l];
#pragma unroll
            for (int w = 1; w < NWV; ++w) {
                const float4 b = lds[w][kind][k][l];
                a.x += b.x;
                a.y += b.y;
                a.z += b.z;
                a.w += b.w;
            }
            st4((kind == 0 ? part_g : part_b) + part_index(4 * c4, blockIdx.x, gridDim.x), a);
        }
    }
}

// ----------------------------------------------------------------------------
// Generic path.
// ----------------------------------------------------------------------------
__global__ __launch_bounds__(kTpb) void ln_fwd_generic(float* __restrict__ y,
    float* __restrict__ mu, float* __restrict__ rstd, const float* __restrict__ x,
    const float* __restrict__ gamma, const float* __restrict__ beta, int C, float eps) {
    __shared__ float red[2 * kNw];
    const int row = blockIdx.x;
    const float* xr = x + (size_t)row * C;
    float s = 0.0f;
    for (int c = threadIdx.x; c < C; c += kTpb) s += xr[c];
    const float m = block_sum<kNw>(s, red) / (float)C;
    float q = 0.0f;
    for (int c = threadIdx.x; c < C; c += kTpb) {
        const float d = xr[c] - m;
        q += d * d;
    }
    const float rs = rsqrtf(block_sum<kNw>(q, red + kNw) / (float)C + eps);
    if (threadIdx.x == 0) {
        mu[row] = m;
        rstd[row] = rs;
    }
    float* yr = y + (size_t)row * C;
    for (int c = threadIdx.x; c < C; c += kTpb) yr[c] = gamma[c] * ((xr[c] - m) * rs) + beta[c];
}

__global__ __launch_bounds__(kTpb) void ln_bwd_dx_generic(float* __restrict__ dx,
    const float* __restrict__ dy, const float* __restrict__ x, const float* __restrict__ gamma,
    const float* __restrict__ mu, const float* __restrict__ rstd, int C) {
    __shared__ float red[2 * kNw];
    const int row = blockIdx.x;
    const size_t base = (size_t)row * C;
    const float m = mu[row], rs = rstd[row];
    float pg = 0.0f, pgx = 0.0f;
    for (int c = threadIdx.x; c < C; c += kTpb) {
        const float xh = (x[base + c] - m) * rs;
        const float g = dy[base + c] * gamma[c];
        pg += g;
        pgx += g * xh;
    }
    block_sum2<kNw>(pg, pgx, red);
    const float invC = 1.0f / (float)C;
    for (int c = threadIdx.x; c < C; c += kTpb) {
        const float xh = (x[base + c] - m) * rs;
        const float g = dy[base + c] * gamma[c];
        dx[base + c] = rs * ((g - pg * invC) - xh * pgx * invC);
    }
}

// partial row y (rows [64 y, 64 y + 64)) of part_g/part_b, stored at
// part_index(c, y, P = gridDim.y): lanes walk 64 channels.
__global__ __launch_bounds__(kTpb) void ln_param_partial_generic(float* __restrict__ part_g,
    float* __restrict__ part_b, const float* __restrict__ dy, const float* __restrict__ x,
    const float* __restrict__ mu, const float* __restrict__ rstd, int rows, int C) {
    __shared__ float lg[kNw][kWave];
    __shared__ float lb[kNw][kWave];
    const int lane = threadIdx.x & (kWave - 1);
    const int wid = threadIdx.x / kWave;
    const int c = blockIdx.x * kWave + lane;
    const int r0 = blockIdx.y * kRowsPerWg;
    const int r1 = min(rows, r0 + kRowsPerWg);
    float sg = 0.0f, sb = 0.0f;
    if (c < C) {
        for (int r = r0 + wid; r < r1; r += kNw) {
            const float xh = (x[(size_t)r * C + c] - mu[r]) * rstd[r];
            const float d = dy[(size_t)r * C + c];
            sg += d * xh;
            sb += d;
        }
    }
    lg[wid][lane] = sg;
    lb[wid][lane] = sb;
    __syncthreads();
    if (wid == 0 && c < C) {
        const size_t o = part_index(c, blockIdx.y, gridDim.y);
        part_g[o] = ((lg[0][lane] + lg[1][lane]) + lg[2][lane]) + lg[3][lane];
        part_b[o] = ((lb[0][lane] + lb[1][lane]) + lb[2][lane]) + lb[3][lane];
    }
}

// dgamma/dbeta column sums over the P partial rows, in one launch: workgroup
// (chunk, kind) sums the kCw channels of its chunk.  Fixed order, in two
// levels:
//   segment s (partial rows [64 s, 64 s + 64)): four chains, chain w adding
//     rows 64 s + w, + 4, ... in row order from 0 (a row past P adds 0), then
//     ((chain 0 + chain 1) + chain 2) + chain 3;
//   total: four chains, chain w adding segments w, w + 4, ... in order from 0,
//     then ((chain 0 + chain 1) + chain 2) + chain 3.
// Segments are taken kSegB at a time: thread (s, w, q) of a batch runs one
// first-level chain over channel quad q with its 16 loads in flight; the
// chains are combined in LDS, and threads (w, j) < 64 carry the second-level
// chains across the batches.
constexpr int kSeg = 64;
constexpr int kPer = kSeg / 4;                  // rows per first-level chain
constexpr int kSegB = kTpb / (4 * (kCw / 4));   // segments per batch (16)
__global__ __launch_bounds__(kTpb) void ln_colsum_chunk(float* __restrict__ og, float* __restrict__ ob,
    const float* __restrict__ pg, const float* __restrict__ pb, int P, int C) {
    // chain sums [segment][chain][channel], each segment's row padded by 16
    // floats: a wave's 128-bit stores (one segment) cover the 64 banks once,
    // and the segment step's reads of four segments fall in different banks
    constexpr int kLp = 4 * kCw + 16;
    __shared__ __align__(16) float lchain[kSegB][kLp];
    __shared__ float lseg[kSegB][kCw];
    __shared__ float lfin[4][kCw];
    const int t = threadIdx.x;
    const int q = t % (kCw / 4), w = (t / (kCw / 4)) % 4, sl = t / kCw;
    const float* part = (blockIdx.y ? pb : pg) + (size_t)blockIdx.x * P * kCw;
    const int S = (P + kSeg - 1) / kSeg;
    float acc = 0.0f;  // second-level chain t / kCw, channel t % kCw (t < 4 kCw)
    for (int s0 = 0; s0 < S; s0 += kSegB) {
        const int s = s0 + sl;
        if (s < S) {
            const int p0 = s * kSeg, p1 = min(P, p0 + kSeg);
            float4 v[kPer];
#pragma unroll
            for (int u = 0; u < kPer; ++u) {
                const int p = p0 + w + 4 * u;
                v[u] = p < p1 ? ld4(part + (size_t)p * kCw + 4 * q) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            }
            float4 a = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
            for (int u = 0; u < kPer; ++u) {
                a.x += v[u].x;
                a.y += v[u].y;
                a.z += v[u].z;
                a.w += v[u].w;
            }
            *reinterpret_cast<float4*>(&lchain[sl][w * kCw + 4 * q]) = a;
        }
        __syncthreads();
        {
            const int ss = t / kCw, j = t % kCw;
            if (s0 + ss < S) {
                const float* ch = lchain[ss];
                lseg[ss][j] = ((ch[j] + ch[kCw + j]) + ch[2 * kCw + j]) + ch[3 * kCw + j];
            }
        }
        __syncthreads();
        if (t < 4 * kCw) {
            const int w2 = t / kCw, j = t % kCw;
#pragma unroll
            for (int u = 0; u < kSegB / 4; ++u) {
                if (s0 + w2 + 4 * u < S) acc += lseg[w2 + 4 * u][j];
            }
        }
    }
    if (t < 4 * kCw) lfin[t / kCw][t % kCw] = acc;
    __syncthreads();
    if (t < kCw) {
        const int c = blockIdx.x * kCw + t;
        if (c < C) (blockIdx.y ? ob : og)[c] = ((lfin[0][t] + lfin[1][t]) + lfin[2][t]) + lfin[3][t];
    }
}

// The same column sums for P <= 256 partial rows, in one short step: thread
// (r = t / 4, channel quad q = t % 4) adds partial rows r, r + 64, r + 128,
// r + 192 in that order (rows past P add nothing); lanes (group g, channel j)
// then add the chains 4g .. 4g + 3 in order, and one lane per channel the 16
// groups in order.  Every thread loads: one round trip instead of the general
// kernel's per-segment chains.
constexpr int kSmallP = 256;
__global__ __launch_bounds__(kTpb) void ln_colsum_small(float* __restrict__ og, float* __restrict__ ob,
    const float* __restrict__ pg, const float* __restrict__ pb, int P, int C) {
    static_assert(kTpb == 4 * 64 && kCw == 16, "64 row lanes x 4 channel quads; 16 groups x 16 channels");
    // chain sums of rows 4g .. 4g + 3 in lchain[g], each group padded by 16
    // floats: the 16 lanes of a 128-bit store (four rows of one group) cover
    // the 64 banks once, and a wave's reads (four groups, one row each) fall
    // in four disjoint 16-bank ranges
    __shared__ __align__(16) float lchain[16][4 * kCw + 16];
    __shared__ float lgrp[16][kCw];
    const int t = threadIdx.x;
    const int q = t % 4, r = t / 4;
    const float* part = (blockIdx.y ? pb : pg) + (size_t)blockIdx.x * P * kCw;
    float4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int p = r + 64 * u;
        v[u] = p < P ? ld4(part + (size_t)p * kCw + 4 * q) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    float4 a = v[0];
#pragma unroll
    for (int u = 1; u < 4; ++u) {
        a.x += v[u].x;
        a.y += v[u].y;
        a.z += v[u].z;
        a.w += v[u].w;
    }
    *reinterpret_cast<float4*>(&lchain[r / 4][(r % 4) * kCw + 4 * q]) = a;
    __syncthreads();
    {
        const int j = t % kCw, g = t / kCw;
        const float* ch = lchain[g];
        lgrp[g][j] = ((ch[j] + ch[kCw + j]) + ch[2 * kCw + j]) + ch[3 * kCw + j];
    }
    __syncthreads();
    if (t < kCw) {
        float sum = lgrp[0][t];
#pragma unroll
        for (int g = 1; g < 16; ++g) sum += lgrp[g][t];
        const int c = blockIdx.x * kCw + t;
        if (c < C) (blockIdx.y ? ob : og)[c] = sum;
    }
}

__global__ void fill_zero2(float* __restrict__ a, float* __restrict__ b, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        a[i] = 0.0f;
        b[i] = 0.0f;
    }
}

// NV for the fast path, or 0.
int fast_nv(int C, const void* a, const void* b, const void* c, const void* d) {
    if (C % 4 != 0 || C > 1024) return 0;
    if (!aligned16(a) || !aligned16(b) || !aligned16(c) || !aligned16(d)) return 0;
    const int c4 = C / 4;
    return c4 <= 64 ? 1 : (c4 <= 128 ? 2 : 4);
}

int num_chunks(int rows) { return (rows + kRowsPerWg - 1) / kRowsPerWg; }
int num_col_chunks(int C) { return (C + kCw - 1) / kCw; }
// floats of one kind's partials (whole chunks)
size_t part_floats(int P, int C) { return (size_t)P * num_col_chunks(C) * kCw; }

void ln_backward_impl(const char* what, float* dx, float* ggamma, float* gbeta, const float* dy,
    const float* x, const float* gamma, const float* mu, const float* rstd, int rows, int C,
    float* ws, hipStream_t s) {
    NNK_REQUIRE(rows >= 0 && C > 0, what, "%s: bad shape batch=%d C=%d", what, rows, C);
    NNK_REQUIRE(ggamma && gbeta, what, "%s: null pointer", what);
    if (rows == 0) {
        fill_zero2<<<dim3((unsigned)((C + 255) / 256)), dim3(256), 0, s>>>(ggamma, gbeta, C);
        nnk_after_launch(what, s);
        return;
    }
    NNK_REQUIRE(dx && dy && x && gamma && mu && rstd, what, "%s: null pointer", what);
    NNK_REQUIRE(ws == nullptr || aligned16(ws), what, "%s: workspace must be 16-byte aligned", what);
    const int P = num_chunks(rows);
    const size_t pc = part_floats(P, C);
    float* scratch = ws;
    if (!scratch) {
        scratch = nnk_scratch_acquire(2 * pc, s, what);
        if (!scratch) return;
    }
    float* part_g = scratch;
    float* part_b = scratch + pc;
    const int nv = fast_nv(C, dx, dy, x, gamma);
    int Pw = P;  // partial rows written
    if (nv) {
        const bool nt = use_nt(12LL * rows * C);
        // One 1024-thread workgroup (kWideWaves waves) per CU when the rows
        // fill every CU with one, for C <= 256: a quarter of the partial rows
        // of the 4-wave workgroups, each wave's next two rows in flight while
        // it works on the current two, and rows dealt out cyclically over the
        // grid's waves.  With each workgroup on a contiguous 256-row block
        // instead (256 streams 256 KB apart), the two launches took 46.3 us
        // on some boxes.  Same-box A/B at [65536, 256] on such a box: 36.5 us
        // against 38.9 us for the 4-wave grid; on other boxes the contiguous
        // 16-wave form took 35.8-36.3 us against 38.1-39.2 us.  Fewer rows
        // would leave CUs idle that 4-wave workgroups still fill.
        constexpr int kWideRows = kWideWaves * kRowsPerWave;
        const int cus = nnk_device_cus(s);
        const bool wide = nv == 1 && cus > 0 && (rows + kWideRows - 1) / kWideRows >= cus;
        if (wide) {
            Pw = (rows + kWideRows - 1) / kWideRows;
            constexpr int T = kWideWaves * kWave;
            if (nt) ln_bwd_wave<1, 2, kWideWaves, true, true, true><<<Pw, T, 0, s>>>(dx, part_g, part_b, dy, x, gamma, mu, rstd, rows, C);
            else ln_bwd_wave<1, 2, kWideWaves, true, true, false><<<Pw, T, 0, s>>>(dx, part_g, part_b, dy, x, gamma, mu, rstd, rows, C);
        } else {
#define NNK_LN_BWD(NV_, RB_)                                                                                                 \
    (nt ? ln_bwd_wave<NV_, RB_, 4, false, false, true><<<P, kTpb, 0, s>>>(dx, part_g, part_b, dy, x, gamma, mu, rstd, rows, C) \
        : ln_bwd_wave<NV_, RB_, 4, false, false, false><<<P, kTpb, 0, s>>>(dx, part_g, part_b, dy, x, gamma, mu, rstd, rows, C))
            switch (nv) {
            case 1: NNK_LN_BWD(1, 4); break;
            case 2: NNK_LN_BWD(2, 2); break;
            default: NNK_LN_BWD(4, 1); break;
            }
#undef NNK_LN_BWD
        }
    } else {
        ln_bwd_dx_generic<<<rows, kTpb, 0, s>>>(dx, dy, x, gamma, mu, rstd, C);
        ln_param_partial_generic<<<dim3((unsigned)((C + kWave - 1) / kWave), (unsigned)P), kTpb, 0, s>>>(
            part_g, part_b, dy, x, mu, rstd, rows, C);
    }
    const dim3 cgrid((unsigned)num_col_chunks(C), 2u);
    if (Pw <= kSmallP) ln_colsum_small<<<cgrid, kTpb, 0, s>>>(ggamma, gbeta, part_g, part_b, Pw, C);
    else ln_colsum_chunk<<<cgrid, kTpb, 0, s>>>(ggamma, gbeta, part_g, part_b, Pw, C);
    if (!ws) nnk_scratch_release(scratch, s);
    nnk_after_launch(what, s);
}

}  // namespace

extern "C" {

void launch_layernorm_forward(float* y, float* mu, float* rstd, const float* x, const float* gamma,
    const float* beta, int batch, int C, float eps, hipStream_t s) {
    const char* what = "launch_layernorm_forward";
    NNK_REQUIRE(batch >= 0 && C > 0, what, "%s: bad shape batch=%d C=%d", what, batch, C);
    if (batch == 0) return;
    NNK_REQUIRE(y && mu && rstd && x && gamma && beta, what, "%s: null pointer", what);
    const int nv = fast_nv(C, y, x, gamma, beta);
    if (nv == 1) {
        constexpr int RB = 4;  // four 1 KB rows in flight per wave: 24.3 -> 23.6 us at [65536, 256]
        if (use_nt(8LL * batch * C))
            ln_fwd_wave<1, RB, true><<<(unsigned)((batch + kNw * RB - 1) / (kNw * RB)), kTpb, 0, s>>>(y, mu, rstd, x, gamma, beta, batch, C, eps);
        else
            ln_fwd_wave<1, RB, false><<<(unsigned)((batch + kNw * RB - 1) / (kNw * RB)), kTpb, 0, s>>>(y, mu, rstd, x, gamma, beta, batch, C, eps);
    } else if (nv == 2) {
        constexpr int RB = 2;
        if (use_nt(8LL * batch * C))
            ln_fwd_wave<2, RB, true><<<(unsigned)((batch + kNw * RB - 1) / (kNw * RB)), kTpb, 0, s>>>(y, mu, rstd, x, gamma, beta, batch, C, eps);
        else
            ln_fwd_wave<2, RB, false><<<(unsigned)((batch + kNw * RB - 1) / (kNw * RB)), kTpb, 0, s>>>(y, mu, rstd, x, gamma, beta, batch, C, eps);
    } else if (nv == 4) {
        constexpr int RB = 1;
        if (use_nt(8LL * batch * C))
            ln_fwd_wave<4, RB, true><<<(unsigned)((batch + kNw * RB - 1) / (kNw * RB)), kTpb, 0, s>>>(y, mu, rstd, x, gamma, beta, batch, C, eps);
        else
            ln_fwd_wave<4, RB, false><<<(unsigned)((batch + kNw * RB - 1) / (kNw * RB)), kTpb, 0, s>>>(y, mu, rstd, x, gamma, beta, batch, C, eps);
    } else {
        ln_fwd_generic<<<(unsigned)batch, kTpb, 0, s>>>(y, mu, rstd, x, gamma, beta, C, eps);
    }
    nnk_after_launch(what, s);
}

void launch_layernorm_backward(float* grad_in, float* ggamma, float* gbeta, const float* grad_out,
    const float* x, const float* gamma, const float* mu, const float* rstd, int batch, int C,
    hipStream_t s) {
    ln_backward_impl("launch_layernorm_backward", grad_in, ggamma, gbeta, grad_out, x, gamma, mu,
        rstd, batch, C, nullptr, s);
}

void launch_layernorm_backward_ws(float* grad_in, float* ggamma, float* gbeta,
    const float* grad_out, const float* x, const float* gamma, const float* mu,
    const float* rstd, int batch, int C, float* workspace, hipStream_t s) {
    if (!workspace) {
        nnk_set_error(hipErrorInvalidValue, "launch_layernorm_backward_ws: null workspace");
        return;
    }
    ln_backward_impl("launch_layernorm_backward_ws", grad_in, ggamma, gbeta, grad_out, x, gamma,
        mu, rstd, batch, C, workspace, s);
}

size_t nnhip_layernorm_backward_workspace(int batch, int C) {
    if (batch <= 0 || C <= 0) return 0;
    // dgamma and dbeta partials, P rows of whole 16-channel chunks each
    return 2 * part_floats(num_chunks(batch), C);
}

}  // extern "C"
