/* oracle.c -- CPU restatement of the reference's fused-layer maths.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h): the checker of the HIP launch layer
 * and, in its *_f32 form, the reported CPU baseline.  Built with
 * -ffp-contract=off so every a*b+c is a rounded multiply and a rounded add,
 * as the device code of the launch layer is built.
 *
 * Pinning (tests/test_oracle.py): Pade coefficients re-derived from the
 * continued fraction; activations and norms against torch on CPU where the
 * maths coincide; GroupNorm(G=1) == LayerNorm; closed forms (zero mean / unit
 * variance, tangential weight-norm gradient, mp weight identities, Adam step
 * 1, EMA geometric decay); im2col/col2im against brute force and F.unfold /
 * F.fold; finite-difference gradchecks of every backward with the reference's
 * gradcheck tolerances (tests/gradcheck.c:15-21, 51-56).
 *
 * The maths restated here is vyeoms/cuda-c-diffusion's (MIT License; the
 * notice is in THIRD_PARTY_NOTICES.md at the repository root).
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------
 * Activation family: kernels.cu:6-68
 * ------------------------------------------------------------------------ */

float orc_pade_tanh(float x) /* kernels.cu:6-12 */
{
    float x2 = x * x;
    float p = x * (135135.0f + x2 * (17325.0f + x2 * (378.0f + x2)));
    float q = 135135.0f + x2 * (62370.0f + x2 * (3150.0f + x2 * 28.0f));
    return fmaxf(-1.0f, fminf(1.0f, p / q));
}

float orc_pade_sigmoid(float x) /* kernels.cu:14-17 */
{
    return fmaxf(0.0f, fminf(1.0f, (orc_pade_tanh(x * 0.5f) + 1.0f) * 0.5f));
}

static const float kGeluC = 0.7978845608f;
static const float kGeluA = 0.044715f;
#define MP_SILU_SCALE (1.0f / 0.596f)

float orc_act(float v, int act) /* kernels.cu:21-38 */
{
    switch (act) {
    case ORC_RELU: return v > 0.0f ? v : 0.0f;
    case ORC_GELU: return 0.5f * v * (1.0f + orc_pade_tanh(kGeluC * (v + kGeluA * v * v * v)));
    case ORC_SILU: return v * orc_pade_sigmoid(v);
    case ORC_MP_SILU: return v * orc_pade_sigmoid(v) * MP_SILU_SCALE;
    case ORC_TANH: return orc_pade_tanh(v);
    default: return v;
    }
}

float orc_act_grad(float z, int act) /* kernels.cu:40-68 */
{
    switch (act) {
    case ORC_RELU: return z > 0.0f ? 1.0f : 0.0f;
    case ORC_TANH: {
        float t = orc_pade_tanh(z);
        return 1.0f - t * t;
    }
    case ORC_SILU: {
        float s = orc_pade_sigmoid(z);
        return s * (1.0f + z * (1.0f - s));
    }
    case ORC_MP_SILU: {
        float s = orc_pade_sigmoid(z);
        return s * (1.0f + z * (1.0f - s)) * MP_SILU_SCALE;
    }
    case ORC_GELU: {
        float u = kGeluC * (z + kGeluA * z * z * z);
        float t = orc_pade_tanh(u);
        float du = kGeluC * (1.0f + 3.0f * kGeluA * z * z);
        return 0.5f * (1.0f + t) + 0.5f * z * (1.0f - t * t) * du;
    }
    default: return 1.0f;
    }
}

/* ------------------------------------------------------------------------
 * Elementwise
 * ------------------------------------------------------------------------ */

void orc_activation_forward(float* out, const float* in, long long n, int act) /* kernels.cu:103-109 */
{
    for (long long i = 0; i < n; ++i) out[i] = orc_act(in[i], act);
}

void orc_activation_backward(float* gin, const float* gout, const float* in, long long n, int act) /* kernels.cu:111-117 */
{
    for (long long i = 0; i < n; ++i) gin[i] = gout[i] * orc_act_grad(in[i], act);
}

void orc_weighted_sum(float* out, const float* a, const float* b, float wa, float wb, long long n) /* kernels.cu:308-314 */
{
    for (long long i = 0; i < n; ++i) out[i] = wa * a[i] + wb * b[i];
}

void orc_mp_sum_weights(float t, float* wa, float* wb) /* kernels.cu:363-364 */
{
    float d = sqrtf((1.0f - t) * (1.0f - t) + t * t);
    *wa = (1.0f - t) / d;
    *wb = t / d;
}

void orc_mp_cat_weights(float t, int Na, int Nb, float* wa, float* wb) /* kernels.cu:1251-1257 */
{
    float denom = (1.0f - t) * (1.0f - t) + t * t;
    float Cs = sqrtf((float)(Na + Nb) / denom);
    *wa = Cs / sqrtf((float)Na) * (1.0f - t);
    *wb = Cs / sqrtf((float)Nb) * t;
}

void orc_mp_cat(float* out, const float* a, const float* b, float wa, float wb, long long rows,
    int Na, int Nb) /* kernels.cu:318-328 */
{
    int N = Na + Nb;
    for (long long r = 0; r < rows; ++r)
        for (int c = 0; c < N; ++c)
            out[r * N + c] = c < Na ? wa * a[r * Na + c] : wb * b[r * Nb + (c - Na)];
}

void orc_mp_split(float* ga, float* gb, const float* g, float wa, float wb, long long rows,
    int Ca, int Cb) /* kernels.cu:1215-1232 */
{
    int N = Ca + Cb;
    for (long long r = 0; r < rows; ++r)
        for (int c = 0; c < N; ++c) {
            if (c < Ca) ga[r * Ca + c] = wa * g[r * N + c];
            else gb[r * Cb + (c - Ca)] = wb * g[r * N + c];
        }
}

void orc_scale_by_scalar(float* x, float s, long long n) /* kernels.cu:300-306 */
{
    for (long long i = 0; i < n; ++i) x[i] *= s;
}

void orc_add_bias(float* Y, const float* b, long long M, int N) /* kernels.cu:95-101 */
{
    for (long long m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n) Y[m * N + n] += b[n];
}

void orc_bias_grad(float* gb, const float* g, long long rows, int N) /* kernels.cu:148-161 */
{
    for (int n = 0; n < N; ++n) {
        double s = 0.0;
        for (long long r = 0; r < rows; ++r) s += g[r * N + n];
        gb[n] = (float)s;
    }
}

void orc_sgd_step(float* p, const float* g, float lr, long long n) /* kernels.cu:163-168 */
{
    for (long long i = 0; i < n; ++i) p[i] -= lr * g[i];
}

void orc_adam_step(float* p, float* m, float* v, const float* g, float lr, float b1, float b2,
    float eps, float bc1, float bc2, long long n) /* kernels.cu:170-183 */
{
    for (long long i = 0; i < n; ++i) {
        float gi = g[i];
        float mi = b1 * m[i] + (1.0f - b1) * gi;
        float vi = b2 * v[i] + (1.0f - b2) * gi * gi;
        m[i] = mi;
        v[i] = vi;
        p[i] -= lr * (mi / bc1) / (sqrtf(vi / bc2) + eps);
    }
}

void orc_adam_bias_corrections(float b1, float b2, int t, float* bc1, float* bc2) /* optimizer.c:62-64 */
{
    *bc1 = 1.0f - powf(b1, (float)t);
    *bc2 = 1.0f - powf(b2, (float)t);
}

/* ------------------------------------------------------------------------
 * GroupNorm (kernels.cu:622-717), NHWC, double accumulation
 * ------------------------------------------------------------------------ */

void orc_groupnorm_forward(float* y, float* mu, float* rstd, const float* x, const float* gamma,
    const float* beta, int B, int HW, int C, int G, float eps, int act)
{
    int cpg = C / G;
    long long n = (long long)HW * cpg;
#pragma omp parallel for schedule(static)
    for (int idx = 0; idx < B * G; ++idx) {
        int b = idx / G, g = idx % G, c0 = g * cpg;
        const float* xb = x + (size_t)b * HW * C;
        double s = 0.0, sq = 0.0;
        for (int hw = 0; hw < HW; ++hw)
            for (int cl = 0; cl < cpg; ++cl) {
                double v = xb[(size_t)hw * C + c0 + cl];
                s += v;
                sq += v * v;
            }
        double mean_d = s / (double)n;
        double var_d = sq / (double)n - mean_d * mean_d; /* kernels.cu:644-645 */
        float mean = (float)mean_d;
        float rs = (float)(1.0 / sqrt(var_d + (double)eps));
        mu[idx] = mean;
        rstd[idx] = rs;
        float* yb = y + (size_t)b * HW * C;
        for (int hw = 0; hw < HW; ++hw)
            for (int cl = 0; cl < cpg; ++cl) {
                size_t o = (size_t)hw * C + c0 + cl;
                yb[o] = orc_act(gamma[c0 + cl] * ((xb[o] - mean) * rs) + beta[c0 + cl], act);
            }
    }
}

void orc_groupnorm_backward(float* dx, float* ggamma, float* gbeta, const float* dy,
    const float* x, const float* gamma, const float* beta, const float* mu, const float* rstd,
    int B, int HW, int C, int G, int act)
{
    int cpg = C / G;
    long long n = (long long)HW * cpg;
    double* cg = (double*)calloc((size_t)B * C, sizeof(double));
    double* cb = (double*)calloc((size_t)B * C, sizeof(double));
#pragma omp parallel for schedule(static)
    for (int idx = 0; idx < B * G; ++idx) {
        int b = idx / G, g = idx % G, c0 = g * cpg;
        float mean = mu[idx], rs = rstd[idx];
        size_t base = (size_t)b * HW * C;
        double S1 = 0.0, S2 = 0.0;
        for (int hw = 0; hw < HW; ++hw)
            for (int cl = 0; cl < cpg; ++cl) {
                size_t o = base + (size_t)hw * C + c0 + cl;
                int c = c0 + cl;
                float xh = (x[o] - mean) * rs;
                float d = dy[o];
                if (act != ORC_IDENTITY) d = d * orc_act_grad(gamma[c] * xh + beta[c], act);
                float gv = d * gamma[c];
                S1 += gv;
                S2 += (double)gv * xh;
                cg[(size_t)b * C + c] += (double)d * xh;
                cb[(size_t)b * C + c] += d;
            }
        float m1 = (float)(S1 / (double)n);
        float m2 = (float)(S2 / (double)n);
        for (int hw = 0; hw < HW; ++hw)
            for (int cl = 0; cl < cpg; ++cl) {
                size_t o = base + (size_t)hw * C + c0 + cl;
                int c = c0 + cl;
                float xh = (x[o] - mean) * rs;
                float d = dy[o];
                if (act != ORC_IDENTITY) d = d * orc_act_grad(gamma[c] * xh + beta[c], act);
                float gv = d * gamma[c];
                dx[o] = rs * ((gv - m1) - xh * m2);
            }
    }
    for (int c = 0; c < C; ++c) {
        double sg = 0.0, sb = 0.0;
        for (int b = 0; b < B; ++b) {
            sg += cg[(size_t)b * C + c];
            sb += cb[(size_t)b * C + c];
        }
        ggamma[c] = (float)sg;
        gbeta[c] = (float)sb;
    }
    free(cg);
    free(cb);
}

/* ------------------------------------------------------------------------
 * LayerNorm (kernels.cu:491-567): two-pass statistics per row
 * ------------------------------------------------------------------------ */

void orc_layernorm_forward(float* y, float* mu, float* rstd, const float* x, const float* gamma,
    const float* beta, long long rows, int C, float eps)
{
#pragma omp parallel for schedule(static)
    for (long long r = 0; r < rows; ++r) {
        const float* xr = x + r * C;
        double s = 0.0;
        for (int c = 0; c < C; ++c) s += xr[c];
        double m_d = s / (double)C;
        double q = 0.0;
        for (int c = 0; c < C; ++c) {
            double d = (double)xr[c] - m_d;
            q += d * d;
        }
        float m = (float)m_d;
        float rs = (float)(1.0 / sqrt(q / (double)C + (double)eps));
        mu[r] = m;
        rstd[r] = rs;
        for (int c = 0; c < C; ++c) y[r * C + c] = gamma[c] * ((xr[c] - m) * rs) + beta[c];
    }
}

void orc_layernorm_backward(float* dx, float* ggamma, float* gbeta, const float* dy,
    const float* x, const float* gamma, const float* mu, const float* rstd, long long rows, int C)
{
#pragma omp parallel for schedule(static)
    for (long long r = 0; r < rows; ++r) {
        float m = mu[r], rs = rstd[r];
        double S1 = 0.0, S2 = 0.0;
        for (int c = 0; c < C; ++c) {
            float xh = (x[r * C + c] - m) * rs;
            float gv = dy[r * C + c] * gamma[c];
            S1 += gv;
            S2 += (double)gv * xh;
        }
        float m1 = (float)(S1 / (double)C), m2 = (float)(S2 / (double)C);
        for (int c = 0; c < C; ++c) {
            float xh = (x[r * C + c] - m) * rs;
            float gv = dy[r * C + c] * gamma[c];
            dx[r * C + c] = rs * ((gv - m1) - xh * m2);
        }
    }
    for (int c = 0; c < C; ++c) {
        double sg = 0.0, sb = 0.0;
        for (long long r = 0; r < rows; ++r) {
            float xh = (x[r * C + c] - mu[r]) * rstd[r];
            float d = dy[r * C + c];
            sg += (double)d * xh;
            sb += d;
        }
        ggamma[c] = (float)sg;
        gbeta[c] = (float)sb;
    }
}

/* ------------------------------------------------------------------------
 * Weight normalisation (kernels.cu:255-297)
 * ------------------------------------------------------------------------ */

void orc_weight_normalize(float* W, int in, int out, float eps)
{
    for (int j = 0; j < out; ++j) {
        double ss = 0.0;
        for (int i = 0; i < in; ++i) {
            double w = W[(size_t)i * out + j];
            ss += w * w;
        }
        float inv = (float)(1.0 / sqrt(ss + (double)eps));
        for (int i = 0; i < in; ++i) W[(size_t)i * out + j] *= inv;
    }
}

void orc_weight_normalize_backward(float* gW, const float* Wn, float gain, float* g_gain,
    int in, int out)
{
    double total = 0.0;
    for (int j = 0; j < out; ++j) {
        double dot = 0.0;
        for (int i = 0; i < in; ++i) dot += (double)Wn[(size_t)i * out + j] * gW[(size_t)i * out + j];
        total += dot;
        float d = (float)dot;
        for (int i = 0; i < in; ++i) {
            size_t o = (size_t)i * out + j;
            gW[o] = gain * (gW[o] - d * Wn[o]);
        }
    }
    g_gain[0] = (float)((double)g_gain[0] + total);
}

/* ------------------------------------------------------------------------
 * Embeddings: the float argument as the reference forms it, the
 * transcendental in double rounded once (the correctly rounded float value).
 * ------------------------------------------------------------------------ */

void orc_mp_fourier(float* out, const float* x, const float* freqs, const float* phases,
    int batch, int C) /* kernels.cu:385-394 */
{
    for (int b = 0; b < batch; ++b)
        for (int k = 0; k < C; ++k) {
            float arg = 6.28318530718f * (x[b] * freqs[k] + phases[k]);
            out[(size_t)b * C + k] = 1.41421356237f * (float)cos((double)arg);
        }
}

void orc_sinusoidal(float* out, const float* t, int batch, int C, float log_max_period) /* kernels.cu:444-456 */
{
    int half = C / 2;
    for (int b = 0; b < batch; ++b)
        for (int c = 0; c < C; ++c) {
            int j = c < half ? c : c - half;
            float e = -log_max_period * (float)j / (float)half;
            float freq = (float)exp((double)e);
            float arg = t[b] * freq;
            out[(size_t)b * C + c] = c < half ? (float)sin((double)arg) : (float)cos((double)arg);
        }
}

/* ------------------------------------------------------------------------
 * im2col / col2im (kernels.cu:750-816)
 * ------------------------------------------------------------------------ */

void orc_im2col(float* col, const float* im, int B, int H, int W, int C, int K, int stride,
    int pad, int Ho, int Wo)
{
    size_t KKC = (size_t)K * K * C;
    for (int b = 0; b < B; ++b)
        for (int oh = 0; oh < Ho; ++oh)
            for (int ow = 0; ow < Wo; ++ow)
                for (int kh = 0; kh < K; ++kh)
                    for (int kw = 0; kw < K; ++kw)
                        for (int ci = 0; ci < C; ++ci) {
                            int ih = oh * stride + kh - pad, iw = ow * stride + kw - pad;
                            float v = 0.0f;
                            if (ih >= 0 && ih < H && iw >= 0 && iw < W)
                                v = im[(((size_t)b * H + ih) * W + iw) * C + ci];
                            size_t row = ((size_t)b * Ho + oh) * Wo + ow;
                            col[row * KKC + (size_t)(kh * K + kw) * C + ci] = v;
                        }
}

void orc_col2im(float* grad_im, const float* grad_col, int B, int H, int W, int C, int K,
    int stride, int pad, int Ho, int Wo)
{
    size_t KKC = (size_t)K * K * C;
    /* ascending sequential index (b, oh, ow, kh, kw, ci) */
    for (int b = 0; b < B; ++b)
        for (int oh = 0; oh < Ho; ++oh)
            for (int ow = 0; ow < Wo; ++ow)
                for (int kh = 0; kh < K; ++kh)
                    for (int kw = 0; kw < K; ++kw)
                        for (int ci = 0; ci < C; ++ci) {
                            int ih = oh * stride + kh - pad, iw = ow * stride + kw - pad;
                            if (ih >= 0 && ih < H && iw >= 0 && iw < W) {
                                size_t row = ((size_t)b * Ho + oh) * Wo + ow;
                                size_t dst = (((size_t)b * H + ih) * W + iw) * C + ci;
                                grad_im[dst] = grad_im[dst] + grad_col[row * KKC + (size_t)(kh * K + kw) * C + ci];
                            }
                        }
}

/* ------------------------------------------------------------------------
 * Spatial (per sample and channel) broadcasts and reductions over NHWC
 * tensors: kernels.cu:1052-1178.  x is [B, HW, C]; v is [B, C].
 * ------------------------------------------------------------------------ */

void orc_spatial_add(float* x, const float* v, int B, int HW, int C) /* kernels.cu:1132-1142 */
{
    for (long long b = 0; b < B; ++b)
        for (long long i = 0; i < (long long)HW * C; ++i) {
            float* p = x + b * HW * C + i;
            *p = *p + v[b * C + i % C];
        }
}

void orc_spatial_reduce_sum(float* out, const float* x, int B, int HW, int C) /* kernels.cu:1145-1158 */
{
    /* accumulated in double: the truth the parallel sums are checked against */
    for (long long b = 0; b < B; ++b)
        for (int c = 0; c < C; ++c) {
            double s = 0.0;
            for (long long r = 0; r < HW; ++r) s += (double)x[(b * HW + r) * C + c];
            out[b * C + c] = (float)s;
        }
}

void orc_spatial_modulate(float* out, const float* x, const float* cond, int B, int HW, int C)
/* kernels.cu:1055-1067: out = in * (cond + 1) */
{
    for (long long b = 0; b < B; ++b)
        for (long long i = 0; i < (long long)HW * C; ++i)
            out[b * HW * C + i] = x[b * HW * C + i] * (cond[b * C + i % C] + 1.0f);
}

void orc_spatial_modulate_backward(float* gin, float* gcond, const float* gout, const float* x,
    const float* cond, int B, int HW, int C) /* kernels.cu:1070-1101 */
{
    for (long long b = 0; b < B; ++b) {
        for (long long i = 0; i < (long long)HW * C; ++i)
            gin[b * HW * C + i] = gout[b * HW * C + i] * (cond[b * C + i % C] + 1.0f);
        for (int c = 0; c < C; ++c) {
            double s = 0.0;
            for (long long r = 0; r < HW; ++r) {
                const long long k = (b * HW + r) * C + c;
                s += (double)(gout[k] * x[k]);
            }
            gcond[b * C + c] = (float)s;
        }
    }
}

void orc_spatial_modulate_act_forward(float* out, const float* x, const float* cond, int B, int HW,
    int C, int act)
/* the reference's pair spatial_modulate + activation_forward (cond_conv_residual.c:30-33) */
{
    for (long long b = 0; b < B; ++b)
        for (long long i = 0; i < (long long)HW * C; ++i)
            out[b * HW * C + i] = orc_act(x[b * HW * C + i] * (cond[b * C + i % C] + 1.0f), act);
}

void orc_spatial_modulate_act_backward(float* gin, float* gcond, const float* gout, const float* x,
    const float* cond, int B, int HW, int C, int act)
/* the reference's pair activation_backward + spatial_modulate_backward
   (cond_conv_residual.c:46-49): g2 = gout * act'(x (cond + 1)),
   gin = g2 (cond + 1), gcond = sum_hw g2 x */
{
    for (long long b = 0; b < B; ++b) {
        for (int c = 0; c < C; ++c) {
            const float m = cond[b * C + c] + 1.0f;
            double s = 0.0;
            for (long long r = 0; r < HW; ++r) {
                const long long k = (b * HW + r) * C + c;
                const float g2 = gout[k] * orc_act_grad(x[k] * m, act);
                gin[k] = g2 * m;
                s += (double)(g2 * x[k]);
            }
            gcond[b * C + c] = (float)s;
        }
    }
}

/* ------------------------------------------------------------------------
 * fp32-faithful OpenMP transcription (CPU baseline): the reference kernels'
 * per-unit maths with fp32 serial accumulation (kernels.cu:622-717).
 * ------------------------------------------------------------------------ */

void orc_set_threads(int n)
{
#ifdef _OPENMP
    omp_set_num_threads(n > 0 ? n : 1);
#else
    (void)n;
#endif
}

int orc_get_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void orc_groupnorm_forward_f32(float* y, float* mu, float* rstd, const float* x,
    const float* gamma, const float* beta, int B, int HW, int C, int G, float eps, int act)
{
    int cpg = C / G;
    int n = HW * cpg;
#pragma omp parallel for schedule(static)
    for (int idx = 0; idx < B * G; ++idx) {
        int b = idx / G, g = idx % G, c0 = g * cpg;
        const float* xb = x + (size_t)b * HW * C;
        float s = 0.0f, sq = 0.0f;
        for (int hw = 0; hw < HW; ++hw)
            for (int cl = 0; cl < cpg; ++cl) {
                float v = xb[(size_t)hw * C + c0 + cl];
                s += v;
                sq += v * v;
            }
        float mean = s / (float)n;
        float var = sq / (float)n - mean * mean;
        float rs = 1.0f / sqrtf(var + eps);
        mu[idx] = mean;
        rstd[idx] = rs;
        float* yb = y + (size_t)b * HW * C;
        for (int hw = 0; hw < HW; ++hw)
            for (int cl = 0; cl < cpg; ++cl) {
                size_t o = (size_t)hw * C + c0 + cl;
                yb[o] = orc_act(gamma[c0 + cl] * ((xb[o] - mean) * rs) + beta[c0 + cl], act);
            }
    }
}

void orc_groupnorm_backward_f32(float* dx, float* ggamma, float* gbeta, const float* dy,
    const float* x, const float* gamma, const float* beta, const float* mu, const float* rstd,
    int B, int HW, int C, int G, int act)
{
    int cpg = C / G;
    int n = HW * cpg;
#pragma omp parallel for schedule(static)
    for (int idx = 0; idx < B * G; ++idx) {
        int b = idx / G, g = idx % G, c0 = g * cpg;
        float mean = mu[idx], rs = rstd[idx];
        size_t base = (size_t)b * HW * C;
        float pg = 0.0f, pgx = 0.0f;
        for (int hw = 0; hw < HW; ++hw)
            for (int cl = 0; cl < cpg; ++cl) {
                size_t o = base + (size_t)hw * C + c0 + cl;
                int c = c0 + cl;
                float xh = (x[o] - mean) * rs;
                float d = dy[o];
                if (act != ORC_IDENTITY) d = d * orc_act_grad(gamma[c] * xh + beta[c], act);
                float gv = d * gamma[c];
                pg += gv;
                pgx += gv * xh;
            }
        float inv_n = 1.0f / (float)n;
        for (int hw = 0; hw < HW; ++hw)
            for (int cl = 0; cl < cpg; ++cl) {
                size_t o = base + (size_t)hw * C + c0 + cl;
                int c = c0 + cl;
                float xh = (x[o] - mean) * rs;
                float d = dy[o];
                if (act != ORC_IDENTITY) d = d * orc_act_grad(gamma[c] * xh + beta[c], act);
                float gv = d * gamma[c];
                dx[o] = rs * (gv - pg * inv_n - xh * pgx * inv_n);
            }
    }
    /* kernels.cu:696-717: one serial loop per channel */
#pragma omp parallel for schedule(static)
    for (int c = 0; c < C; ++c) {
        int g = c / cpg;
        float gg = 0.0f, gb = 0.0f;
        for (int b = 0; b < B; ++b) {
            float mean = mu[b * G + g], rs = rstd[b * G + g];
            for (int hw = 0; hw < HW; ++hw) {
                size_t o = ((size_t)b * HW + hw) * C + c;
                float xh = (x[o] - mean) * rs;
                float d = dy[o];
                if (act != ORC_IDENTITY) d = d * orc_act_grad(gamma[c] * xh + beta[c], act);
                gg += d * xh;
                gb += d;
            }
        }
        ggamma[c] = gg;
        gbeta[c] = gb;
    }
}
