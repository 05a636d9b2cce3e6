/* layernorm.c -- per-row LayerNorm module.  Reference: src/layernorm.c:4-80
 * (eps 1e-5, gamma=1, beta=0, cached per-row mu/rstd). */
#include "nn_modules.h"

typedef struct {
    int C, max_batch;
    float eps;
    float *gamma, *beta;
    float *ggamma, *gbeta;
    float *mu, *rstd;
    float* work;
} LayerNormState;

static void layernorm_forward(Module* self, const float* in, float* out, int batch, Context* ctx)
{
    LayerNormState* st = (LayerNormState*)self->state;
    NN_ASSERT(batch <= st->max_batch, "layernorm: batch exceeds max_batch");
    launch_layernorm_forward(out, st->mu, st->rstd, in, st->gamma, st->beta, batch, st->C,
        st->eps, ctx->stream);
}

static void layernorm_backward(Module* self, const float* in, const float* out,
    const float* grad_out, float* grad_in, int batch, Context* ctx)
{
    (void)out;
    LayerNormState* st = (LayerNormState*)self->state;
    NN_ASSERT(batch <= st->max_batch, "layernorm: batch exceeds max_batch");
    launch_layernorm_backward_ws(grad_in, st->ggamma, st->gbeta, grad_out, in, st->gamma,
        st->mu, st->rstd, batch, st->C, st->work, ctx->stream);
}

static void layernorm_parameters(Module* self, ParamList* pl)
{
    LayerNormState* st = (LayerNormState*)self->state;
    param_list_add(pl, st->gamma, st->ggamma, st->C);
    param_list_add(pl, st->beta, st->gbeta, st->C);
}

static void layernorm_free(Module* self)
{
    LayerNormState* st = (LayerNormState*)self->state;
    (void)hipFree(st->gamma);
    (void)hipFree(st->beta);
    (void)hipFree(st->ggamma);
    (void)hipFree(st->gbeta);
    (void)hipFree(st->mu);
    (void)hipFree(st->rstd);
    (void)hipFree(st->work);
    free(st);
    free(self);
}

Module* layernorm_create(int dim, int max_batch)
{
    Module* m = (Module*)malloc(sizeof(Module));
    LayerNormState* st = (LayerNormState*)malloc(sizeof(LayerNormState));
    st->C = dim;
    st->max_batch = max_batch;
    st->eps = 1e-5f;
    st->gamma = nn_device_alloc((size_t)dim);
    st->beta = nn_device_alloc((size_t)dim);
    st->ggamma = nn_device_alloc((size_t)dim);
    st->gbeta = nn_device_alloc((size_t)dim);
    st->mu = nn_device_alloc((size_t)max_batch);
    st->rstd = nn_device_alloc((size_t)max_batch);
    st->work = nn_device_alloc(nnhip_layernorm_backward_workspace(max_batch, dim));

    float* ones = (float*)malloc((size_t)dim * sizeof(float));
    for (int i = 0; i < dim; ++i) ones[i] = 1.0f;
    NN_HIP_CHECK(hipMemcpy(st->gamma, ones, (size_t)dim * sizeof(float), hipMemcpyHostToDevice));
    NN_HIP_CHECK(hipMemset(st->beta, 0, (size_t)dim * sizeof(float)));
    free(ones);

    m->name = "layernorm";
    m->in_dim = dim;
    m->out_dim = dim;
    m->state = st;
    m->forward = layernorm_forward;
    m->backward = layernorm_backward;
    m->parameters = layernorm_parameters;
    m->free = layernorm_free;
    return m;
}
