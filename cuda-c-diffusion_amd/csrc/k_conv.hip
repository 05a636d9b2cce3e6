// k_conv.hip -- NHWC im2col and the gather form of col2im.
// Reference maths: src/kernels.cu:750-838.
//
// im2col: col[(b,oh,ow), (kh,kw,ci)] = im[b, oh*s+kh-p, ow*s+kw-p, ci] or 0.
//   Threads walk col in memory order (float4 when C % 4 == 0), so stores are
//   fully coalesced and each K*K segment of a row reads C contiguous floats
//   of one pixel.  Bit-exact: a copy.
// col2im: each im element gathers its contributions instead of the
//   reference's scatter with atomicAdd.  The additions are done in the order
//   of the reference kernel's sequential index (ascending oh, then ow), which
//   is kh descending then kw descending, as plain fp32 adds starting from the
//   value already in grad_im (launch_col2im) or from +0.0f (launch_col2im_set).
//   Every col element is read once; no memset and no atomics.
// In large launches (use_nt) col and grad_im stream with nontemporal stores
// and loads; the image side of im2col, read up to K*K times, always uses
// ordinary loads.
#include "nnk_common.h"

namespace {

using namespace nnk;

constexpr int kTpb = 256;
// One unit per thread on a one-shot grid for the generic im2col and for
// col2im (col2im_set at cfg3: 113 -> 105 us against four units per thread).
constexpr int kUnroll = 1;
// Passes in flight per thread in im2col_rows_kernel for K != 3.  The rows
// kernel keeps all passes of a tile in one workgroup: one pass per workgroup
// (one float4 per thread) measured 142 us against 113 us at cfg3, its nine
// taps of an image row then being read on different XCDs.
constexpr int kRowsBatch = 4;
constexpr long long kPerBlock = (long long)kTpb * kUnroll;

struct ConvGeom {
    int H, W, C, K, stride, pad, Ho, Wo;
};

// VW = 4 (float4, C % 4 == 0) or 1.  Unit index u walks col in memory order.
template <int VW, bool NT>
__global__ __launch_bounds__(kTpb) void im2col_kernel(float* __restrict__ col,
    const float* __restrict__ im, ConvGeom g, long long units, FastDiv div_row,
    FastDiv div_cv, FastDiv div_k, FastDiv div_wo, FastDiv div_ho) {
    const int CV = g.C / VW;  // vectors per pixel
    const long long base = (long long)blockIdx.x * kPerBlock + threadIdx.x;
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const long long q = base + (long long)u * kTpb;
        if (q >= units) continue;
        uint32_t row, j, seg, cv, kh, kw, pix, ow, b, oh;
        div_row.divmod((uint32_t)q, row, j);   // j in [0, K*K*CV)
        div_cv.divmod(j, seg, cv);             // seg = kh*K + kw
        div_k.divmod(seg, kh, kw);
        div_wo.divmod(row, pix, ow);
        div_ho.divmod(pix, b, oh);
        const int ih = (int)oh * g.stride + (int)kh - g.pad;
        const int iw = (int)ow * g.stride + (int)kw - g.pad;
        const bool in = ih >= 0 && ih < g.H && iw >= 0 && iw < g.W;
        const size_t src = (((size_t)b * g.H + (in ? ih : 0)) * g.W + (in ? iw : 0)) * g.C + (size_t)cv * VW;
        if constexpr (VW == 4) {
            const float4 v = in ? ld4(im + src) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            stS<NT>(col + 4 * q, v);
        } else {
            col[q] = in ? im[src] : 0.0f;
            (void)CV;
        }
    }
}

// Fast im2col (C % 4 == 0 and CV = C/4 dividing the workgroup size, CV >= 4).
// A workgroup writes RT = SPI whole col rows (SPI = kTpb / CV kernel-window
// segments per pass), so every thread keeps one float4 column cv and walks
// the segments s = tid / CV, + SPI, ... of the tile: exactly K*K passes, each
// pass storing kTpb consecutive float4 of col.  The per-row image origin
// (b, oh*stride - pad, ow*stride - pad) comes from an LDS table.  Bit-exact.
constexpr int kMaxRowsPerTile = 64;
// NB = passes whose loads are in flight together: K*K for the common 3x3
// kernel (all nine), kRowsBatch otherwise.
template <int NB, bool NT>
__global__ __launch_bounds__(kTpb) void im2col_rows_kernel(float* __restrict__ col,
    const float* __restrict__ im, ConvGeom g, int rows, int CV, FastDiv div_k, FastDiv div_kk,
    FastDiv div_wo, FastDiv div_ho) {
    __shared__ int4 origin[kMaxRowsPerTile];  // (ih0, iw0, b * H, row valid)
    const int SPI = kTpb / CV;
    const int KK = g.K * g.K;
    const int row0 = blockIdx.x * SPI;
    if ((int)threadIdx.x < SPI) {
        const int row = row0 + (int)threadIdx.x;
        int4 o = make_int4(0, 0, 0, 0);
        if (row < rows) {
            uint32_t pix, ow, b, oh;
            div_wo.divmod((uint32_t)row, pix, ow);
            div_ho.divmod(pix, b, oh);
            o = make_int4((int)oh * g.stride - g.pad, (int)ow * g.stride - g.pad, (int)b * g.H, 1);
        }
        origin[threadIdx.x] = o;
    }
    __syncthreads();
    const int cv = (int)threadIdx.x % CV;
    uint32_t r, seg;  // segment index s = tid / CV + pass * SPI = r * KK + seg
    div_kk.divmod((uint32_t)threadIdx.x / (uint32_t)CV, r, seg);
    float* out = col + ((size_t)row0 * KK) * g.C + (size_t)threadIdx.x * 4;
    // passes in batches of NB: all loads of a batch are in flight together
    for (int p0 = 0; p0 < KK; p0 += NB) {
        float4 v[NB];
        bool st[NB];
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            const int4 o = origin[r];
            st[u] = p0 + u < KK && o.w;
            uint32_t kh, kw;
            div_k.divmod(seg, kh, kw);
            const int ih = o.x + (int)kh, iw = o.y + (int)kw;
            const bool in = st[u] && ih >= 0 && ih < g.H && iw >= 0 && iw < g.W;
            v[u] = in ? ld4(im + ((size_t)(o.z + ih) * g.W + iw) * g.C + cv * 4) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            uint32_t q;
            div_kk.divmod(seg + (uint32_t)SPI, q, seg);
            r = r + q < (uint32_t)SPI ? r + q : (uint32_t)SPI - 1;  // stays inside the origin table
        }
#pragma unroll
        for (int u = 0; u < NB; ++u)
            if (st[u]) stS<NT>(out + (size_t)(p0 + u) * kTpb * 4, v[u]);
    }
}

template <int VW, bool UNIT_STRIDE, bool ACCUM, bool NT>
__global__ __launch_bounds__(kTpb) void col2im_kernel(float* __restrict__ grad_im,
    const float* __restrict__ grad_col, ConvGeom g, long long units, FastDiv div_cv,
    FastDiv div_w, FastDiv div_h) {
    const int KKC = g.K * g.K * g.C;
    const long long base = (long long)blockIdx.x * kPerBlock + threadIdx.x;
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const long long q = base + (long long)u * kTpb;
        if (q >= units) continue;
        uint32_t pix, cv, rest, iw, b, ih;
        div_cv.divmod((uint32_t)q, pix, cv);
        div_w.divmod(pix, rest, iw);
        div_h.divmod(rest, b, ih);
        const int ci = (int)cv * VW;
        float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if constexpr (ACCUM) {
            if constexpr (VW == 4) acc = ldS<NT>(grad_im + 4 * q);
            else acc.x = grad_im[q];
        }
        for (int kh = g.K - 1; kh >= 0; --kh) {
            const int hn = (int)ih + g.pad - kh;
            if (hn < 0) continue;
            int oh = hn;
            if constexpr (!UNIT_STRIDE) {
                if (hn % g.stride != 0) continue;
                oh = hn / g.stride;
            }
            if (oh >= g.Ho) continue;
            for (int kw = g.K - 1; kw >= 0; --kw) {
                const int wn = (int)iw + g.pad - kw;
                if (wn < 0) continue;
                int ow = wn;
                if constexpr (!UNIT_STRIDE) {
                    if (wn % g.stride != 0) continue;
                    ow = wn / g.stride;
                }
                if (ow >= g.Wo) continue;
                const size_t src = (((size_t)b * g.Ho + oh) * g.Wo + ow) * KKC + (size_t)(kh * g.K + kw) * g.C + ci;
                if constexpr (VW == 4) {
                    const float4 v = ldS<NT>(grad_col + src);
                    acc.x = acc.x + v.x;
                    acc.y = acc.y + v.y;
                    acc.z = acc.z + v.z;
                    acc.w = acc.w + v.w;
                } else {
                    acc.x = acc.x + grad_col[src];
                }
            }
        }
        if constexpr (VW == 4) stS<NT>(grad_im + 4 * q, acc);
        else grad_im[q] = acc.x;
    }
}

bool geom_ok(const char* what, int batch, int H, int W, int C, int K, int stride, int pad,
    int Ho, int Wo) {
    if (batch < 0 || H <= 0 || W <= 0 || C <= 0 || K <= 0 || stride <= 0 || pad < 0 || Ho < 0 || Wo < 0) {
        nnk_set_error(hipErrorInvalidValue, "%s: bad geometry batch=%d H=%d W=%d C=%d K=%d stride=%d pad=%d Ho=%d Wo=%d",
            what, batch, H, W, C, K, stride, pad, Ho, Wo);
        return false;
    }
    // Any H_out/W_out is memory-safe here (both kernels bounds-check the image
    // side), as in the reference, which trusts the caller's (H+2p-K)/s+1.
    const long long col = (long long)batch * Ho * Wo * K * K * C;
    const long long im = (long long)batch * H * W * C;
    if (col >= (1LL << 31) || im >= (1LL << 31)) {
        nnk_set_error(hipErrorInvalidValue, "%s: tensors exceed 2^31 elements", what);
        return false;
    }
    return true;
}

unsigned blocks_for(long long units) {
    const long long b = (units + kPerBlock - 1) / kPerBlock;
    return (unsigned)(b > 0 ? b : 1);
}

template <bool ACCUM>
void col2im_impl(const char* what, float* grad_im, const float* grad_col, int batch, int H, int W,
    int C, int K, int stride, int pad, int Ho, int Wo, hipStream_t s) {
    if (!geom_ok(what, batch, H, W, C, K, stride, pad, Ho, Wo)) return;
    if (batch == 0) return;
    NNK_REQUIRE(grad_im && grad_col, what, "%s: null pointer", what);
    const ConvGeom g{H, W, C, K, stride, pad, Ho, Wo};
    const bool vec = C % 4 == 0 && aligned16(grad_im) && aligned16(grad_col);
    const int VWr = vec ? 4 : 1;
    const long long units = (long long)batch * H * W * (C / VWr);
    const FastDiv dcv((uint32_t)(C / VWr)), dw((uint32_t)W), dh((uint32_t)H);
    const unsigned blocks = blocks_for(units);
    const bool nt = use_nt(4LL * ((long long)batch * Ho * Wo * K * K * C + (long long)batch * H * W * C));
    if (vec) {
        if (stride == 1 && nt) col2im_kernel<4, true, ACCUM, true><<<blocks, kTpb, 0, s>>>(grad_im, grad_col, g, units, dcv, dw, dh);
        else if (stride == 1) col2im_kernel<4, true, ACCUM, false><<<blocks, kTpb, 0, s>>>(grad_im, grad_col, g, units, dcv, dw, dh);
        else if (nt) col2im_kernel<4, false, ACCUM, true><<<blocks, kTpb, 0, s>>>(grad_im, grad_col, g, units, dcv, dw, dh);
        else col2im_kernel<4, false, ACCUM, false><<<blocks, kTpb, 0, s>>>(grad_im, grad_col, g, units, dcv, dw, dh);
    } else {
        if (stride == 1) col2im_kernel<1, true, ACCUM, false><<<blocks, kTpb, 0, s>>>(grad_im, grad_col, g, units, dcv, dw, dh);
        else col2im_kernel<1, false, ACCUM, false><<<blocks, kTpb, 0, s>>>(grad_im, grad_col, g, units, dcv, dw, dh);
    }
    nnk_after_launch(what, s);
}

}  // namespace

extern "C" {

void launch_im2col(float* col, const float* im, int batch, int H, int W, int C, int K, int stride,
    int pad, int H_out, int W_out, hipStream_t s) {
    const char* what = "launch_im2col";
    if (!geom_ok(what, batch, H, W, C, K, stride, pad, H_out, W_out)) return;
    if (batch == 0 || H_out == 0 || W_out == 0) return;
    NNK_REQUIRE(col && im, what, "%s: null pointer", what);
    const ConvGeom g{H, W, C, K, stride, pad, H_out, W_out};
    const bool vec = C % 4 == 0 && aligned16(col) && aligned16(im);
    const int VWr = vec ? 4 : 1;
    const int CV = C / VWr;
    const long long units = (long long)batch * H_out * W_out * K * K * CV;
    const FastDiv drow((uint32_t)(K * K * CV)), dcv((uint32_t)CV), dk((uint32_t)K),
        dwo((uint32_t)W_out), dho((uint32_t)H_out);
    const bool nt = use_nt(4LL * (units * VWr + (long long)batch * H * W * C));
    if (vec && CV >= kTpb / kMaxRowsPerTile && kTpb % CV == 0) {
        const long long rows = (long long)batch * H_out * W_out;
        const int rows_per_tile = kTpb / CV;
        const unsigned tiles = (unsigned)((rows + rows_per_tile - 1) / rows_per_tile);
        const FastDiv dkk((uint32_t)(K * K));
        if (K == 3 && nt) im2col_rows_kernel<9, true><<<tiles, kTpb, 0, s>>>(col, im, g, (int)rows, CV, dk, dkk, dwo, dho);
        else if (K == 3) im2col_rows_kernel<9, false><<<tiles, kTpb, 0, s>>>(col, im, g, (int)rows, CV, dk, dkk, dwo, dho);
        else if (nt) im2col_rows_kernel<kRowsBatch, true><<<tiles, kTpb, 0, s>>>(col, im, g, (int)rows, CV, dk, dkk, dwo, dho);
        else im2col_rows_kernel<kRowsBatch, false><<<tiles, kTpb, 0, s>>>(col, im, g, (int)rows, CV, dk, dkk, dwo, dho);
    } else if (vec) {
        if (nt) im2col_kernel<4, true><<<blocks_for(units), kTpb, 0, s>>>(col, im, g, units, drow, dcv, dk, dwo, dho);
        else im2col_kernel<4, false><<<blocks_for(units), kTpb, 0, s>>>(col, im, g, units, drow, dcv, dk, dwo, dho);
    } else {
        im2col_kernel<1, false><<<blocks_for(units), kTpb, 0, s>>>(col, im, g, units, drow, dcv, dk, dwo, dho);
    }
    nnk_after_launch(what, s);
}

void launch_col2im(float* grad_im, const float* grad_col, int batch, int H, int W, int C, int K,
    int stride, int pad, int H_out, int W_out, hipStream_t s) {
    col2im_impl<true>("launch_col2im", grad_im, grad_col, batch, H, W, C, K, stride, pad, H_out,
        W_out, s);
}

void launch_col2im_set(float* grad_im, const float* grad_col, int batch, int H, int W, int C,
    int K, int stride, int pad, int H_out, int W_out, hipStream_t s) {
    col2im_impl<false>("launch_col2im_set", grad_im, grad_col, batch, H, W, C, K, stride, pad,
        H_out, W_out, s);
}

}  // extern "C"
