/* conv_residual.c -- the classic DDPM residual block on the fused kernels.
 * Reference: src/conv_residual.c:1-150:
 *   h = GroupNorm(x) -> SiLU -> conv3x3;  h += Linear(emb) (broadcast over H,W);
 *   h = GroupNorm(h) -> SiLU -> conv3x3;  out = x + h.
 * Same maths, parameters and ParamList order (gn1, conv1, time_proj, gn2,
 * conv2: src/conv_residual.c:68-76).  Executed differently:
 *   * each GroupNorm -> SiLU pair is one fused module (forward writes only the
 *     activated output; backward recomputes the pre-activation), so the
 *     reference's h0/h3 and gh0/gh3 tensors and their HBM round trips are gone;
 *   * the embedding broadcast and its gradient (spatial_add / spatial_reduce_sum)
 *     are the parallel kernels, the reduction into a lent workspace.
 */
#include "nn_modules.h"

typedef struct {
    int C, emb_dim, max_batch, H, W, G, cond_slot;
    Module *gn1, *gn2;   /* GroupNorm + SiLU */
    Module *conv1, *conv2;
    Module* time_proj;
    float *h1, *h2, *h4; /* act(gn1(x)), conv1(h1) + emb, act(gn2(h2)) */
    float* c;
    float *gh4, *gh2, *gh1, *gxb;
    float* gc;
    float* grad_emb_local;
    float* red_ws;
} ConvResState;

static void cr_forward(Module* self, const float* in, float* out, int batch, Context* ctx)
{
    ConvResState* st = (ConvResState*)self->state;
    NN_ASSERT(batch <= st->max_batch, "conv_residual: batch exceeds max_batch");
    const int n = batch * st->H * st->W * st->C;
    st->gn1->forward(st->gn1, in, st->h1, batch, ctx);
    st->conv1->forward(st->conv1, st->h1, st->h2, batch, ctx);
    st->time_proj->forward(st->time_proj, ctx->cond[st->cond_slot].fwd, st->c, batch, ctx);
    launch_spatial_add(st->h2, st->c, batch, st->H, st->W, st->C, ctx->stream);
    st->gn2->forward(st->gn2, st->h2, st->h4, batch, ctx);
    st->conv2->forward(st->conv2, st->h4, out, batch, ctx);
    launch_weighted_sum(out, in, out, 1.0f, 1.0f, n, ctx->stream);
}

static void cr_backward(Module* self, const float* in, const float* out,
    const float* grad_out, float* grad_in, int batch, Context* ctx)
{
    (void)out;
    ConvResState* st = (ConvResState*)self->state;
    const int n = batch * st->H * st->W * st->C;
    st->conv2->backward(st->conv2, st->h4, NULL, grad_out, st->gh4, batch, ctx);
    st->gn2->backward(st->gn2, st->h2, NULL, st->gh4, st->gh2, batch, ctx);
    launch_spatial_reduce_sum_ws(st->gc, st->gh2, batch, st->H * st->W, st->C, st->red_ws, ctx->stream);
    st->time_proj->backward(st->time_proj, ctx->cond[st->cond_slot].fwd, st->c, st->gc,
        st->grad_emb_local, batch, ctx);
    launch_weighted_sum(ctx->cond[st->cond_slot].grad, ctx->cond[st->cond_slot].grad,
        st->grad_emb_local, 1.0f, 1.0f, batch * st->emb_dim, ctx->stream);
    st->conv1->backward(st->conv1, st->h1, NULL, st->gh2, st->gh1, batch, ctx);
    st->gn1->backward(st->gn1, in, NULL, st->gh1, st->gxb, batch, ctx);
    launch_weighted_sum(grad_in, grad_out, st->gxb, 1.0f, 1.0f, n, ctx->stream);
}

static void cr_parameters(Module* self, ParamList* pl)
{
    ConvResState* st = (ConvResState*)self->state;
    st->gn1->parameters(st->gn1, pl);
    st->conv1->parameters(st->conv1, pl);
    st->time_proj->parameters(st->time_proj, pl);
    st->gn2->parameters(st->gn2, pl);
    st->conv2->parameters(st->conv2, pl);
}

static void cr_free(Module* self)
{
    ConvResState* st = (ConvResState*)self->state;
    st->gn1->free(st->gn1);
    st->gn2->free(st->gn2);
    st->conv1->free(st->conv1);
    st->conv2->free(st->conv2);
    st->time_proj->free(st->time_proj);
    float* bufs[] = {st->h1, st->h2, st->h4, st->c, st->gh4, st->gh2, st->gh1, st->gxb, st->gc,
        st->grad_emb_local, st->red_ws};
    for (size_t i = 0; i < sizeof bufs / sizeof bufs[0]; ++i) (void)hipFree(bufs[i]);
    free(st);
    free(self);
}

Module* conv_residual_create(Context* ctx, int C, int emb_dim, int H, int W, int max_batch, int num_groups,
    int cond_slot)
{
    Module* m = (Module*)malloc(sizeof(Module));
    ConvResState* st = (ConvResState*)malloc(sizeof(ConvResState));
    st->C = C;
    st->emb_dim = emb_dim;
    st->max_batch = max_batch;
    st->H = H;
    st->W = W;
    st->G = num_groups;
    st->cond_slot = cond_slot;
    /* created in the reference's order, so the generator draws the same
       sequence of initial weights (src/conv_residual.c:117-121) */
    st->gn1 = spatial_groupnorm_act_create(C, num_groups, H, W, max_batch, ACT_SILU);
    st->conv1 = conv2d_create(ctx, C, C, 3, 1, 1, H, W, max_batch, 0, 1.0f);
    st->time_proj = linear_create(ctx, emb_dim, C);
    st->gn2 = spatial_groupnorm_act_create(C, num_groups, H, W, max_batch, ACT_SILU);
    st->conv2 = conv2d_create(ctx, C, C, 3, 1, 1, H, W, max_batch, 0, 1.0f);
    const size_t ns = (size_t)max_batch * H * W * C;
    st->h1 = nn_device_alloc(ns);
    st->h2 = nn_device_alloc(ns);
    st->h4 = nn_device_alloc(ns);
    st->c = nn_device_alloc((size_t)max_batch * C);
    st->gh4 = nn_device_alloc(ns);
    st->gh2 = nn_device_alloc(ns);
    st->gh1 = nn_device_alloc(ns);
    st->gxb = nn_device_alloc(ns);
    st->gc = nn_device_alloc((size_t)max_batch * C);
    st->grad_emb_local = nn_device_alloc((size_t)max_batch * emb_dim);
    st->red_ws = nn_device_alloc(nnhip_spatial_reduce_workspace(max_batch, H * W, C));
    m->name = "conv_residual";
    m->in_dim = H * W * C;
    m->out_dim = H * W * C;
    m->state = st;
    m->forward = cr_forward;
    m->backward = cr_backward;
    m->parameters = cr_parameters;
    m->free = cr_free;
    return m;
}
