/* mp_linear.c -- magnitude-preserving linear layer: forced weight
 * normalisation, GEMM, device-scalar gain.  Reference: src/mp_linear.c:5-86
 * (eps 1e-4, N(0,1) init, gain gradient zeroed then accumulated). */
#include "nn_gemm.h"

typedef struct {
    int in, out;
    float eps;
    float *W, *gW;
    float *gain, *g_gain;
    float* wn_ws;  /* weight-norm backward workspace (zero-filled at create) */
} MPLinearState;

static void mp_linear_forward(Module* self, const float* in, float* out, int batch, Context* ctx)
{
    MPLinearState* st = (MPLinearState*)self->state;
    launch_weight_normalize(st->W, st->in, st->out, st->eps, ctx->stream);
    nn_gemm_forward(ctx->blas, 1.0f, in, st->W, out, batch, st->in, st->out);
    launch_scale_by_scalar(out, st->gain, batch * st->out, ctx->stream);
}

static void mp_linear_backward(Module* self, const float* in, const float* out,
    const float* grad_out, float* grad_in, int batch, Context* ctx)
{
    (void)out;
    MPLinearState* st = (MPLinearState*)self->state;
    nn_gemm_dW(ctx->blas, 1.0f, in, grad_out, st->gW, batch, st->in, st->out);
    nnhip_fill_f32(st->g_gain, 0.0f, 1, ctx->stream);
    launch_weight_normalize_backward_ws(st->gW, st->W, st->gain, st->g_gain, st->in, st->out,
        st->wn_ws, ctx->stream);
    if (grad_in) {
        nn_gemm_dX(ctx->blas, 1.0f, st->W, grad_out, grad_in, batch, st->in, st->out);
        launch_scale_by_scalar(grad_in, st->gain, batch * st->in, ctx->stream);
    }
}

static void mp_linear_parameters(Module* self, ParamList* pl)
{
    MPLinearState* st = (MPLinearState*)self->state;
    param_list_add(pl, st->W, st->gW, st->in * st->out);
    param_list_add(pl, st->gain, st->g_gain, 1);
}

static void mp_linear_free(Module* self)
{
    MPLinearState* st = (MPLinearState*)self->state;
    (void)hipFree(st->W);
    (void)hipFree(st->gW);
    (void)hipFree(st->gain);
    (void)hipFree(st->g_gain);
    (void)hipFree(st->wn_ws);
    free(st);
    free(self);
}

Module* mp_linear_create(Context* ctx, int in_dim, int out_dim, float gain_init)
{
    Module* m = (Module*)malloc(sizeof(Module));
    MPLinearState* st = (MPLinearState*)malloc(sizeof(MPLinearState));
    st->in = in_dim;
    st->out = out_dim;
    st->eps = 1e-4f;
    st->W = nn_device_alloc((size_t)in_dim * out_dim);
    st->gW = nn_device_alloc((size_t)in_dim * out_dim);
    st->gain = nn_device_alloc(1);
    st->g_gain = nn_device_alloc(1);
    {
        const size_t n = nnhip_weight_normalize_backward_workspace(out_dim);
        st->wn_ws = nn_device_alloc(n);
        NN_HIP_CHECK(hipMemset(st->wn_ws, 0, (n ? n : 1) * sizeof(float)));
    }
    nn_fill_normal(ctx, st->W, (size_t)in_dim * out_dim, 0.0f, 1.0f);
    NN_HIP_CHECK(hipMemcpy(st->gain, &gain_init, sizeof(float), hipMemcpyHostToDevice));
    m->name = "mp_linear";
    m->in_dim = in_dim;
    m->out_dim = out_dim;
    m->state = st;
    m->forward = mp_linear_forward;
    m->backward = mp_linear_backward;
    m->parameters = mp_linear_parameters;
    m->free = mp_linear_free;
    return m;
}
