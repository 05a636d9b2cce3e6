/* linear.c -- dense layer with bias: GEMM + bias add, backward GEMMs + bias
 * gradient.  Reference: src/linear.c:1-76 (He normal init with std
 * sqrt(2 / fan_in), zero bias; gradients overwritten by every backward).
 * The time-embedding projection of the DDPM residual block. */
#include <math.h>

#include "nn_gemm.h"

typedef struct {
    int in, out;
    float *W, *b;
    float *gW, *gb;
} LinearState;

static void linear_forward(Module* self, const float* in, float* out, int batch, Context* ctx)
{
    LinearState* st = (LinearState*)self->state;
    nn_gemm_forward(ctx->blas, 1.0f, in, st->W, out, batch, st->in, st->out);
    launch_add_bias(out, st->b, batch, st->out, ctx->stream);
}

static void linear_backward(Module* self, const float* in, const float* out,
    const float* grad_out, float* grad_in, int batch, Context* ctx)
{
    (void)out;
    LinearState* st = (LinearState*)self->state;
    nn_gemm_dW(ctx->blas, 1.0f, in, grad_out, st->gW, batch, st->in, st->out);
    launch_bias_grad(st->gb, grad_out, batch, st->out, ctx->stream);
    if (grad_in) nn_gemm_dX(ctx->blas, 1.0f, st->W, grad_out, grad_in, batch, st->in, st->out);
}

static void linear_parameters(Module* self, ParamList* pl)
{
    LinearState* st = (LinearState*)self->state;
    param_list_add(pl, st->W, st->gW, st->in * st->out);
    param_list_add(pl, st->b, st->gb, st->out);
}

static void linear_free(Module* self)
{
    LinearState* st = (LinearState*)self->state;
    (void)hipFree(st->W);
    (void)hipFree(st->b);
    (void)hipFree(st->gW);
    (void)hipFree(st->gb);
    free(st);
    free(self);
}

Module* linear_create(Context* ctx, int in_dim, int out_dim)
{
    Module* m = (Module*)malloc(sizeof(Module));
    LinearState* st = (LinearState*)malloc(sizeof(LinearState));
    st->in = in_dim;
    st->out = out_dim;
    st->W = nn_device_alloc((size_t)in_dim * out_dim);
    st->b = nn_device_alloc((size_t)out_dim);
    st->gW = nn_device_alloc((size_t)in_dim * out_dim);
    st->gb = nn_device_alloc((size_t)out_dim);
    nn_fill_normal(ctx, st->W, (size_t)in_dim * out_dim, 0.0f, sqrtf(2.0f / (float)in_dim));
    NN_HIP_CHECK(hipMemset(st->b, 0, (size_t)out_dim * sizeof(float)));
    m->name = "linear";
    m->in_dim = in_dim;
    m->out_dim = out_dim;
    m->state = st;
    m->forward = linear_forward;
    m->backward = linear_backward;
    m->parameters = linear_parameters;
    m->free = linear_free;
    return m;
}
