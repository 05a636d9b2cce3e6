/* conv2d.c -- NHWC conv2d, plain (bias) or magnitude-preserving (forced
 * weight norm + gain).  Reference: src/conv2d.c:6-145.  Weights are
 * [K*K*C_in, C_out] row-major (conv2d.c:114-115).
 * Forward: the implicit-GEMM kernel on the matrix cores when the channel counts
 * allow it (C_in % 32 == 0, C_out % 64 == 0), with the bias or gain in its
 * epilogue; otherwise im2col + rocBLAS GEMM + bias/gain pass, as the reference.
 * NNHIP_CONV_PATH=gemm forces the latter.  Backward: the weight gradient as
 * an implicit GEMM too (C_in % 4 == 0, C_out % 64 == 0), the stride-1 input
 * gradient as the implicit forward of grad_out with the flipped kernel
 * (C_out % 32 == 0, C_in % 64 == 0); otherwise im2col + rocBLAS GEMMs and the
 * gather col2im, which needs no memset of grad_in. */
#include <math.h>
#include <string.h>

#include "nn_gemm.h"

typedef struct {
    int C_in, C_out, K, stride, pad;
    int Hi, Wi, Ho, Wo;
    int max_batch, mp_mode;
    float eps;
    float *Wt, *gW;
    float *b, *gb;
    float *gain, *g_gain;
    float* wn_ws;  /* weight-norm backward workspace (mp mode; zero-filled at create) */
    float* col;
    float* WT;     /* [C_out, K*K*C_in] weight for the implicit GEMM (NULL when unsupported) */
    float* WF;     /* [C_in, K*K*C_out] flipped weight for the implicit input gradient (or NULL) */
    float* wg_ws;  /* implicit weight-gradient workspace (or NULL) */
    int wgrad_implicit;
} Conv2DState;

static int gemm_forced(void)
{
    const char* e = getenv("NNHIP_CONV_PATH");
    return e && strcmp(e, "gemm") == 0;
}

static int use_implicit(const Conv2DState* st) { return st->WT && !gemm_forced(); }

static void conv2d_forward(Module* self, const float* in, float* out, int batch, Context* ctx)
{
    Conv2DState* st = (Conv2DState*)self->state;
    NN_ASSERT(batch <= st->max_batch, "conv2d: batch exceeds max_batch");
    int M = batch * st->Ho * st->Wo;
    int Kg = st->K * st->K * st->C_in;
    if (use_implicit(st)) {
        if (st->mp_mode) launch_weight_normalize(st->Wt, Kg, st->C_out, st->eps, ctx->stream);
        launch_transpose(st->WT, st->Wt, Kg, st->C_out, ctx->stream);
        launch_conv2d_forward_implicit(out, in, st->WT, st->mp_mode ? NULL : st->b, st->mp_mode ? st->gain : NULL,
            batch, st->Hi, st->Wi, st->C_in, st->C_out, st->K, st->stride, st->pad, st->Ho, st->Wo, ctx->stream);
        return;
    }
    launch_im2col(st->col, in, batch, st->Hi, st->Wi, st->C_in, st->K, st->stride, st->pad,
        st->Ho, st->Wo, ctx->stream);
    if (st->mp_mode) {
        launch_weight_normalize(st->Wt, Kg, st->C_out, st->eps, ctx->stream);
        nn_gemm_forward(ctx->blas, 1.0f, st->col, st->Wt, out, M, Kg, st->C_out);
        launch_scale_by_scalar(out, st->gain, M * st->C_out, ctx->stream);
    } else {
        nn_gemm_forward(ctx->blas, 1.0f, st->col, st->Wt, out, M, Kg, st->C_out);
        launch_add_bias(out, st->b, M, st->C_out, ctx->stream);
    }
}

static void conv2d_backward(Module* self, const float* in, const float* out,
    const float* grad_out, float* grad_in, int batch, Context* ctx)
{
    (void)out;
    Conv2DState* st = (Conv2DState*)self->state;
    NN_ASSERT(batch <= st->max_batch, "conv2d: batch exceeds max_batch");
    int M = batch * st->Ho * st->Wo;
    int Kg = st->K * st->K * st->C_in;
    const int forced = gemm_forced();
    if (st->wgrad_implicit && !forced) {
        launch_conv2d_weight_grad_implicit(st->gW, in, grad_out, batch, st->Hi, st->Wi, st->C_in, st->C_out, st->K,
            st->stride, st->pad, st->Ho, st->Wo, st->wg_ws, ctx->stream);
    } else {
        launch_im2col(st->col, in, batch, st->Hi, st->Wi, st->C_in, st->K, st->stride, st->pad,
            st->Ho, st->Wo, ctx->stream);
        nn_gemm_dW(ctx->blas, 1.0f, st->col, grad_out, st->gW, M, Kg, st->C_out);
    }
    if (st->mp_mode) {
        nnhip_fill_f32(st->g_gain, 0.0f, 1, ctx->stream);
        launch_weight_normalize_backward_ws(st->gW, st->Wt, st->gain, st->g_gain, Kg, st->C_out,
            st->wn_ws, ctx->stream);
    } else {
        launch_bias_grad(st->gb, grad_out, M, st->C_out, ctx->stream);
    }
    if (!grad_in) return;
    if (st->WF && !forced) {
        /* stride 1: dx = conv(dy, flipped kernel, pad K-1-pad), times the gain in mp mode */
        launch_conv2d_flip_weights(st->WF, st->Wt, st->K, st->C_in, st->C_out, ctx->stream);
        launch_conv2d_forward_implicit(grad_in, grad_out, st->WF, NULL, st->mp_mode ? st->gain : NULL, batch,
            st->Ho, st->Wo, st->C_out, st->C_in, st->K, 1, st->K - 1 - st->pad, st->Hi, st->Wi, ctx->stream);
        return;
    }
    nn_gemm_dX(ctx->blas, 1.0f, st->Wt, grad_out, st->col, M, Kg, st->C_out);
    if (st->mp_mode) launch_scale_by_scalar(st->col, st->gain, M * Kg, ctx->stream);
    launch_col2im_set(grad_in, st->col, batch, st->Hi, st->Wi, st->C_in, st->K, st->stride,
        st->pad, st->Ho, st->Wo, ctx->stream);
}

static void conv2d_parameters(Module* self, ParamList* pl)
{
    Conv2DState* st = (Conv2DState*)self->state;
    param_list_add(pl, st->Wt, st->gW, st->K * st->K * st->C_in * st->C_out);
    if (st->mp_mode) param_list_add(pl, st->gain, st->g_gain, 1);
    else param_list_add(pl, st->b, st->gb, st->C_out);
}

static void conv2d_free(Module* self)
{
    Conv2DState* st = (Conv2DState*)self->state;
    (void)hipFree(st->Wt);
    (void)hipFree(st->gW);
    (void)hipFree(st->col);
    if (st->WT) (void)hipFree(st->WT);
    if (st->WF) (void)hipFree(st->WF);
    if (st->wg_ws) (void)hipFree(st->wg_ws);
    if (st->mp_mode) {
        (void)hipFree(st->gain);
        (void)hipFree(st->g_gain);
        (void)hipFree(st->wn_ws);
    } else {
        (void)hipFree(st->b);
        (void)hipFree(st->gb);
    }
    free(st);
    free(self);
}

Module* conv2d_create(Context* ctx, int C_in, int C_out, int K, int stride, int pad, int H, int W,
    int max_batch, int mp_mode, float gain)
{
    Module* m = (Module*)malloc(sizeof(Module));
    Conv2DState* st = (Conv2DState*)malloc(sizeof(Conv2DState));
    st->C_in = C_in;
    st->C_out = C_out;
    st->K = K;
    st->stride = stride;
    st->pad = pad;
    st->Hi = H;
    st->Wi = W;
    st->Ho = (H + 2 * pad - K) / stride + 1;
    st->Wo = (W + 2 * pad - K) / stride + 1;
    st->max_batch = max_batch;
    st->mp_mode = mp_mode;
    st->eps = 1e-4f;
    int Kg = K * K * C_in;
    st->Wt = nn_device_alloc((size_t)Kg * C_out);
    st->gW = nn_device_alloc((size_t)Kg * C_out);
    st->col = nn_device_alloc((size_t)max_batch * st->Ho * st->Wo * Kg);
    st->WT = nnhip_conv2d_implicit_supported(C_in, C_out) ? nn_device_alloc((size_t)Kg * C_out) : NULL;
    /* the input gradient of a stride-1 convolution is a forward convolution of
       grad_out (C_out channels in, C_in out) with padding K-1-pad >= 0 */
    st->WF = (stride == 1 && pad <= K - 1 && nnhip_conv2d_implicit_supported(C_out, C_in))
        ? nn_device_alloc((size_t)Kg * C_out) : NULL;
    st->wgrad_implicit = nnhip_conv2d_wgrad_implicit_supported(C_in, C_out);
    {
        const size_t n = st->wgrad_implicit
            ? nnhip_conv2d_wgrad_workspace(max_batch, C_in, C_out, K, st->Ho, st->Wo) : 0;
        st->wg_ws = n ? nn_device_alloc(n) : NULL;
    }
    if (mp_mode) {
        st->b = NULL;
        st->gb = NULL;
        st->gain = nn_device_alloc(1);
        st->g_gain = nn_device_alloc(1);
        const size_t n = nnhip_weight_normalize_backward_workspace(C_out);
        st->wn_ws = nn_device_alloc(n);
        NN_HIP_CHECK(hipMemset(st->wn_ws, 0, (n ? n : 1) * sizeof(float)));
        nn_fill_normal(ctx, st->Wt, (size_t)Kg * C_out, 0.0f, 1.0f);
        NN_HIP_CHECK(hipMemcpy(st->gain, &gain, sizeof(float), hipMemcpyHostToDevice));
    } else {
        st->gain = NULL;
        st->g_gain = NULL;
        st->wn_ws = NULL;
        st->b = nn_device_alloc((size_t)C_out);
        st->gb = nn_device_alloc((size_t)C_out);
        nn_fill_normal(ctx, st->Wt, (size_t)Kg * C_out, 0.0f, sqrtf(2.0f / (float)Kg));
        NN_HIP_CHECK(hipMemset(st->b, 0, (size_t)C_out * sizeof(float)));
    }
    m->name = "conv2d";
    m->in_dim = H * W * C_in;
    m->out_dim = st->Ho * st->Wo * C_out;
    m->state = st;
    m->forward = conv2d_forward;
    m->backward = conv2d_backward;
    m->parameters = conv2d_parameters;
    m->free = conv2d_free;
    return m;
}
