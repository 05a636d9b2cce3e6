/* refcalls.c -- compile-only check of the drop-in boundary (never linked or
 * run).  The reference's launcher block (src/nn.h:348-466) re-typed for HIP:
 * every prototype keeps the reference's parameter types and order with the
 * CUDA stream replaced by hipStream_t, and each launcher of include/nn_hip.h
 * must be assignable to a pointer of that exact type (gcc -Werror rejects any
 * difference in a parameter's type or const-ness).  Below them, call sites
 * written the way the reference's host modules call the launchers, with
 * arguments of the types those modules pass (struct fields of int / float /
 * float*, a Context-like stream member).  tests/test_abi.py compiles this
 * file with gcc -std=c11 -Wall -Wextra -Werror. */
#include <stdio.h>
#include <stdlib.h>

#include "nn_hip.h"
#include "nn_hip_rt.h"

/* ---- the reference's prototypes, stream re-typed (src/nn.h:354-456) ---- */
typedef void add_bias_t(float* Y, const float* b, int M, int N, hipStream_t s);
typedef void act_fwd_t(float* out, const float* in, int n, Activation act, hipStream_t s);
typedef void act_bwd_t(float* grad_in, const float* grad_out, const float* in, int n, Activation act,
    hipStream_t s);
typedef void bias_grad_t(float* gb, const float* grad_out, int batch, int N, hipStream_t s);
typedef void sgd_t(float* p, const float* g, float lr, int n, hipStream_t s);
typedef void adam_t(float* p, float* m, float* v, const float* g, float lr, float beta1, float beta2, float eps,
    float bc1, float bc2, int n, hipStream_t s);
typedef void wn_t(float* W, int in, int out, float eps, hipStream_t s);
typedef void wn_bwd_t(float* gW, const float* Wn, const float* gain, float* g_gain, int in, int out, hipStream_t s);
typedef void scale_t(float* x, const float* s, int n, hipStream_t st);
typedef void mp_sum_t(float* out, const float* a, const float* b, float t, int n, hipStream_t s);
typedef void wsum_t(float* out, const float* a, const float* b, float wa, float wb, int n, hipStream_t s);
typedef void fourier_t(float* out, const float* x, const float* freqs, const float* phases, int batch, int C,
    hipStream_t s);
typedef void sinus_t(float* out, const float* t, int batch, int C, float log_max_period, hipStream_t s);
typedef void ln_fwd_t(float* y, float* mu, float* rstd, const float* x, const float* gamma, const float* beta,
    int batch, int C, float eps, hipStream_t s);
typedef void ln_bwd_t(float* grad_in, float* ggamma, float* gbeta, const float* grad_out, const float* x,
    const float* gamma, const float* mu, const float* rstd, int batch, int C, hipStream_t s);
typedef void gn_fwd_t(float* y, float* mu, float* rstd, const float* x, const float* gamma, const float* beta,
    int batch, int HW, int C, int G, float eps, hipStream_t s);
typedef void gn_bwd_t(float* dx, float* ggamma, float* gbeta, const float* dy, const float* x, const float* gamma,
    const float* mu, const float* rstd, int batch, int HW, int C, int G, hipStream_t s);
typedef void mp_cat_t(float* out, const float* a, const float* b, float t, int batch, int Na, int Nb,
    hipStream_t s);
typedef void im2col_t(float* col, const float* im, int batch, int H, int W, int C, int K, int stride, int pad,
    int H_out, int W_out, hipStream_t s);
typedef void col2im_t(float* grad_im, const float* grad_col, int batch, int H, int W, int C, int K, int stride,
    int pad, int H_out, int W_out, hipStream_t s);
typedef void smod_t(float* out, const float* in, const float* cond, int batch, int H, int W, int C, hipStream_t s);
typedef void smod_bwd_t(float* grad_in, float* grad_cond, const float* grad_out, const float* in, const float* cond,
    int batch, int H, int W, int C, hipStream_t s);
typedef void sadd_t(float* inout, const float* bias, int batch, int H, int W, int C, hipStream_t s);
typedef void sred_t(float* out, const float* in, int batch, int HW, int C, hipStream_t s);
typedef void mp_ccat_t(float* out, const float* a, const float* b, float t, int spatial, int Ca, int Cb,
    hipStream_t s);
typedef void mp_csplit_t(float* grad_a, float* grad_b, const float* grad_out, float t, int spatial, int Ca, int Cb,
    hipStream_t s);

add_bias_t* const ref_add_bias = launch_add_bias;
act_fwd_t* const ref_activation_forward = launch_activation_forward;
act_bwd_t* const ref_activation_backward = launch_activation_backward;
bias_grad_t* const ref_bias_grad = launch_bias_grad;
sgd_t* const ref_sgd_step = launch_sgd_step;
adam_t* const ref_adam_step = launch_adam_step;
wn_t* const ref_weight_normalize = launch_weight_normalize;
wn_bwd_t* const ref_weight_normalize_backward = launch_weight_normalize_backward;
scale_t* const ref_scale_by_scalar = launch_scale_by_scalar;
mp_sum_t* const ref_mp_sum = launch_mp_sum;
wsum_t* const ref_weighted_sum = launch_weighted_sum;
fourier_t* const ref_mp_fourier = launch_mp_fourier;
sinus_t* const ref_sinusoidal = launch_sinusoidal;
ln_fwd_t* const ref_layernorm_forward = launch_layernorm_forward;
ln_bwd_t* const ref_layernorm_backward = launch_layernorm_backward;
gn_fwd_t* const ref_groupnorm_forward = launch_groupnorm_forward;
gn_bwd_t* const ref_groupnorm_backward = launch_groupnorm_backward;
mp_cat_t* const ref_mp_cat = launch_mp_cat;
im2col_t* const ref_im2col = launch_im2col;
col2im_t* const ref_col2im = launch_col2im;
smod_t* const ref_spatial_modulate = launch_spatial_modulate;
smod_bwd_t* const ref_spatial_modulate_backward = launch_spatial_modulate_backward;
sadd_t* const ref_spatial_add = launch_spatial_add;
sred_t* const ref_spatial_reduce_sum = launch_spatial_reduce_sum;
mp_ccat_t* const ref_mp_channel_cat = launch_mp_channel_cat;
mp_csplit_t* const ref_mp_channel_split = launch_mp_channel_split;

/* ---- call sites as the reference's host modules write them ---- */
typedef struct {                                              /* src/nn.h:71-77, re-typed for HIP */
    NnHostRng rng;                                            /* was curandGenerator_t curand */
    hipStream_t stream;
} RefContext;
typedef struct {                                              /* fields of the modules' state structs */
    int C, G, HW, dim, in, out, C_in, C_out, K, stride, pad, Hi, Wi, Ho, Wo, H, W;
    float eps, log_max_period, wa, wb, t;
    Activation act;
    float *gamma, *beta, *ggamma, *gbeta, *mu, *rstd, *W_, *gW, *gain, *g_gain, *col, *b, *gb;
    float *freqs, *phases, *h0, *h1, *h2, *c, *gc, *m, *v, *shadow, *param, *grad;
} RefState;

void nn_reference_call_sites(RefState* st, RefContext* ctx, float* out, const float* in, float* grad_in,
    const float* grad_out, int batch, int n);
void nn_reference_call_sites(RefState* st, RefContext* ctx, float* out, const float* in, float* grad_in,
    const float* grad_out, int batch, int n)
{
    const int M = batch * st->Ho * st->Wo, Kg = st->K * st->K * st->C_in;
    /* src/groupnorm.c:16, 27 */
    launch_groupnorm_forward(out, st->mu, st->rstd, in, st->gamma, st->beta, batch, st->HW, st->C, st->G, st->eps,
        ctx->stream);
    launch_groupnorm_backward(grad_in, st->ggamma, st->gbeta, grad_out, in, st->gamma, st->mu, st->rstd, batch,
        st->HW, st->C, st->G, ctx->stream);
    /* src/layernorm.c:16, 26 */
    launch_layernorm_forward(out, st->mu, st->rstd, in, st->gamma, st->beta, batch, st->C, st->eps, ctx->stream);
    launch_layernorm_backward(grad_in, st->ggamma, st->gbeta, grad_out, in, st->gamma, st->mu, st->rstd, batch,
        st->C, ctx->stream);
    /* src/activation.c:12, 21 */
    launch_activation_forward(out, in, batch * st->dim, st->act, ctx->stream);
    launch_activation_backward(grad_in, grad_out, in, batch * st->dim, st->act, ctx->stream);
    /* src/mp_linear.c:16-18, 32, 38 */
    launch_weight_normalize(st->W_, st->in, st->out, st->eps, ctx->stream);
    launch_scale_by_scalar(out, st->gain, batch * st->out, ctx->stream);
    launch_weight_normalize_backward(st->gW, st->W_, st->gain, st->g_gain, st->in, st->out, ctx->stream);
    /* src/conv2d.c:24, 33, 57, 64 */
    launch_im2col(st->col, in, batch, st->Hi, st->Wi, st->C_in, st->K, st->stride, st->pad, st->Ho, st->Wo,
        ctx->stream);
    launch_add_bias(out, st->b, M, st->C_out, ctx->stream);
    launch_scale_by_scalar(st->col, st->gain, M * Kg, ctx->stream);
    launch_bias_grad(st->gb, grad_out, M, st->C_out, ctx->stream);
    launch_col2im(grad_in, st->col, batch, st->Hi, st->Wi, st->C_in, st->K, st->stride, st->pad, st->Ho, st->Wo,
        ctx->stream);
    /* src/mp_fourier.c:13, src/sinusoidal.c:14 */
    launch_mp_fourier(out, in, st->freqs, st->phases, batch, st->C, ctx->stream);
    launch_sinusoidal(out, in, batch, st->C, st->log_max_period, ctx->stream);
    /* src/optimizer.c:58, 66 and src/ema.c:32 */
    launch_sgd_step(st->param, st->grad, st->eps, n, ctx->stream);
    launch_adam_step(st->param, st->m, st->v, st->grad, st->eps, 0.9f, 0.999f, 1e-8f, st->wa, st->wb, n,
        ctx->stream);
    launch_weighted_sum(st->shadow, st->shadow, st->param, st->wa, 1.0f - st->wa, n, ctx->stream);
    /* src/conv_residual.c:33, 54 */
    launch_spatial_add(st->h2, st->c, batch, st->H, st->W, st->C, ctx->stream);
    launch_spatial_reduce_sum(st->gc, st->h2, batch, st->H * st->W, st->C, ctx->stream);
    /* src/cond_conv_residual.c:31, 35, 50 */
    launch_spatial_modulate(st->h2, st->h1, st->c, batch, st->H, st->W, st->C, ctx->stream);
    launch_weighted_sum(out, in, st->h1, st->wa, st->wb, n, ctx->stream);
    launch_spatial_modulate_backward(st->h1, st->gc, st->h2, st->h1, st->c, batch, st->H, st->W, st->C,
        ctx->stream);
    /* src/unet.c:176, 215 and the mp ops of src/nn.h:378-379, 408-409 */
    launch_mp_channel_cat(out, in, st->h0, st->t, batch * st->H * st->W, st->C_in, st->C_out, ctx->stream);
    launch_mp_channel_split(grad_in, st->h0, grad_out, st->t, batch * st->H * st->W, st->C_in, st->C_out,
        ctx->stream);
    launch_mp_sum(out, in, st->h1, st->t, n, ctx->stream);
    launch_mp_cat(out, in, st->h1, st->t, batch, st->C_in, st->C_out, ctx->stream);
}

/* ---- weight initialisation, re-typed: NN_HIP_CHECK and the fill of
   src/nn.h:13-21, 117-135 over the library's host generator, then the call
   sites of the path's modules with ctx->curand replaced by &ctx->rng
   (src/conv2d.c:124, 132, src/mp_linear.c:73, src/linear.c:62,
   src/mp_fourier.c:49-50) and the generator's creation
   (ddpm/main_ddpm.c:143-145) ---- */
#define NN_HIP_CHECK(call)                                                                       \
    do {                                                                                         \
        hipError_t e_ = (call);                                                                  \
        if (e_ != hipSuccess) {                                                                  \
            fprintf(stderr, "HIP %s:%d: %s\n", __FILE__, __LINE__, hipGetErrorString(e_));      \
            exit(1);                                                                             \
        }                                                                                        \
    } while (0)

static inline void nn_fill_normal(NnHostRng* g, float* dst, size_t n, float mean, float std)
{
    NN_HIP_CHECK((hipError_t)nnhip_fill_normal(g, dst, n, mean, std));
}

void nn_reference_init_sites(RefState* st, RefContext* ctx, unsigned long long seed, int Kg, int in_dim,
    int out_dim, int num_channels, float bandwidth);
void nn_reference_init_sites(RefState* st, RefContext* ctx, unsigned long long seed, int Kg, int in_dim,
    int out_dim, int num_channels, float bandwidth)
{
    nnhip_rng_seed(&ctx->rng, (uint64_t)seed);                                   /* main_ddpm.c:143-145 */
    nn_fill_normal(&ctx->rng, st->W_, (size_t)Kg * st->C_out, 0.0f, 1.0f);        /* conv2d.c:124 */
    nn_fill_normal(&ctx->rng, st->W_, (size_t)Kg * st->C_out, 0.0f, st->eps);     /* conv2d.c:132 */
    nn_fill_normal(&ctx->rng, st->W_, (size_t)in_dim * out_dim, 0.0f, 1.0f);      /* mp_linear.c:73 */
    nn_fill_normal(&ctx->rng, st->W_, (size_t)in_dim * out_dim, 0.0f, st->eps);   /* linear.c:62 */
    nn_fill_normal(&ctx->rng, st->freqs, num_channels, 0.0f, bandwidth);         /* mp_fourier.c:49 */
    NN_HIP_CHECK((hipError_t)nnhip_fill_uniform(&ctx->rng, st->phases, num_channels)); /* mp_fourier.c:50 */
}
