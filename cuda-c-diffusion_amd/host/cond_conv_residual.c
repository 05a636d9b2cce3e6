/* cond_conv_residual.c -- the EDM2 block (spatial convolution variant) on the
 * fused kernels.  Reference: src/cond_conv_residual.c:1-144:
 *   h0 = mp_silu(x); h1 = conv0(h0); c = emb_lin(emb) (mp_linear, gain 0);
 *   h2 = h1 * (c + 1); h3 = mp_silu(h2); h4 = conv1(h3); out = mp_sum(x, h4, t).
 * Same maths, parameters and ParamList order (conv0, emb_lin, conv1).  The
 * modulation and the activation after it run as one fused launch each way
 * (launch_spatial_modulate_act_forward / _backward): h2 and gh2 are never
 * stored, and grad_cond is a parallel fixed-order reduction.
 */
#include <math.h>

#include "nn_modules.h"

typedef struct {
    int C, emb_dim, max_batch, H, W, cond_slot;
    float wa, wb;
    Module *conv0, *emb_lin, *conv1;
    float *h0, *h1, *c, *h3, *h4;
    float *gh4, *gh3, *gh1, *gh0, *gc, *gxb, *grad_emb_local;
    float* red_ws;
} CondConvResState;

static void ccr_forward(Module* self, const float* in, float* out, int batch, Context* ctx)
{
    CondConvResState* st = (CondConvResState*)self->state;
    NN_ASSERT(batch <= st->max_batch, "cond_conv_residual: batch exceeds max_batch");
    const int n = batch * st->H * st->W * st->C;
    launch_activation_forward(st->h0, in, n, ACT_MP_SILU, ctx->stream);
    st->conv0->forward(st->conv0, st->h0, st->h1, batch, ctx);
    st->emb_lin->forward(st->emb_lin, ctx->cond[st->cond_slot].fwd, st->c, batch, ctx);
    launch_spatial_modulate_act_forward(st->h3, st->h1, st->c, batch, st->H, st->W, st->C, ACT_MP_SILU,
        ctx->stream);
    st->conv1->forward(st->conv1, st->h3, st->h4, batch, ctx);
    launch_weighted_sum(out, in, st->h4, st->wa, st->wb, n, ctx->stream);
}

static void ccr_backward(Module* self, const float* in, const float* out,
    const float* grad_out, float* grad_in, int batch, Context* ctx)
{
    (void)out;
    CondConvResState* st = (CondConvResState*)self->state;
    const int n = batch * st->H * st->W * st->C;
    launch_weighted_sum(st->gh4, grad_out, grad_out, st->wb, 0.0f, n, ctx->stream);
    st->conv1->backward(st->conv1, st->h3, st->h4, st->gh4, st->gh3, batch, ctx);
    launch_spatial_modulate_act_backward(st->gh1, st->gc, st->gh3, st->h1, st->c, batch, st->H, st->W, st->C,
        ACT_MP_SILU, st->red_ws, ctx->stream);
    st->conv0->backward(st->conv0, st->h0, st->h1, st->gh1, st->gh0, batch, ctx);
    launch_activation_backward(st->gxb, st->gh0, in, n, ACT_MP_SILU, ctx->stream);
    st->emb_lin->backward(st->emb_lin, ctx->cond[st->cond_slot].fwd, st->c, st->gc, st->grad_emb_local,
        batch, ctx);
    launch_weighted_sum(ctx->cond[st->cond_slot].grad, ctx->cond[st->cond_slot].grad, st->grad_emb_local,
        1.0f, 1.0f, batch * st->emb_dim, ctx->stream);
    launch_weighted_sum(grad_in, grad_out, st->gxb, st->wa, 1.0f, n, ctx->stream);
}

static void ccr_parameters(Module* self, ParamList* pl)
{
    CondConvResState* st = (CondConvResState*)self->state;
    st->conv0->parameters(st->conv0, pl);
    st->emb_lin->parameters(st->emb_lin, pl);
    st->conv1->parameters(st->conv1, pl);
}

static void ccr_free(Module* self)
{
    CondConvResState* st = (CondConvResState*)self->state;
    st->conv0->free(st->conv0);
    st->emb_lin->free(st->emb_lin);
    st->conv1->free(st->conv1);
    float* bufs[] = {st->h0, st->h1, st->c, st->h3, st->h4, st->gh4, st->gh3, st->gh1, st->gh0, st->gc,
        st->gxb, st->grad_emb_local, st->red_ws};
    for (size_t i = 0; i < sizeof bufs / sizeof bufs[0]; ++i) (void)hipFree(bufs[i]);
    free(st);
    free(self);
}

Module* cond_conv_residual_create(Context* ctx, int C, int emb_dim, int H, int W, int max_batch, float t,
    int cond_slot)
{
    Module* m = (Module*)malloc(sizeof(Module));
    CondConvResState* st = (CondConvResState*)malloc(sizeof(CondConvResState));
    st->C = C;
    st->emb_dim = emb_dim;
    st->max_batch = max_batch;
    st->H = H;
    st->W = W;
    st->cond_slot = cond_slot;
    /* mp_sum weights in host float (src/cond_conv_residual.c:108-110) */
    const float d = sqrtf((1.0f - t) * (1.0f - t) + t * t);
    st->wa = (1.0f - t) / d;
    st->wb = t / d;
    st->conv0 = conv2d_create(ctx, C, C, 3, 1, 1, H, W, max_batch, 1, 1.0f);
    st->emb_lin = mp_linear_create(ctx, emb_dim, C, 0.0f);
    st->conv1 = conv2d_create(ctx, C, C, 3, 1, 1, H, W, max_batch, 1, 1.0f);
    const size_t ns = (size_t)max_batch * H * W * C;
    st->h0 = nn_device_alloc(ns);
    st->h1 = nn_device_alloc(ns);
    st->c = nn_device_alloc((size_t)max_batch * C);
    st->h3 = nn_device_alloc(ns);
    st->h4 = nn_device_alloc(ns);
    st->gh4 = nn_device_alloc(ns);
    st->gh3 = nn_device_alloc(ns);
    st->gh1 = nn_device_alloc(ns);
    st->gh0 = nn_device_alloc(ns);
    st->gc = nn_device_alloc((size_t)max_batch * C);
    st->gxb = nn_device_alloc(ns);
    st->grad_emb_local = nn_device_alloc((size_t)max_batch * emb_dim);
    st->red_ws = nn_device_alloc(nnhip_spatial_reduce_workspace(max_batch, H * W, C));
    m->name = "cond_conv_residual";
    m->in_dim = H * W * C;
    m->out_dim = H * W * C;
    m->state = st;
    m->forward = ccr_forward;
    m->backward = ccr_backward;
    m->parameters = ccr_parameters;
    m->free = ccr_free;
    return m;
}
