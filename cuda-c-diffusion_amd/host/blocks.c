/* blocks.c -- the two diffusion residual blocks that call the fused path most,
 * as Layers with child modules and an arena of intermediate tensors.
 *
 * The maths, the parameters, their ParamList order and the construction
 * (weight-draw) order are the reference's:
 *   DDPM  (src/conv_residual.c:1-150)      out = x + conv2(act(GN2(conv1(act(GN1(x))) + proj(emb))))
 *         children gn1, conv1, proj, gn2, conv2 (src/conv_residual.c:68-76, 117-121)
 *   EDM2  (src/cond_conv_residual.c:1-144) out = mp_sum(x, conv1(mp_silu(conv0(mp_silu(x)) * (lin(emb) + 1))), t)
 *         children conv0, emb_lin (gain 0), conv1 (src/cond_conv_residual.c:64-70, 115-119)
 * Both read the embedding from ctx->cond[slot].fwd and add its gradient into
 * ctx->cond[slot].grad.
 *
 * The schedule is this library's:
 *   * every GroupNorm -> SiLU pair is one fused module, the modulation and the
 *     MP-SiLU after it one fused launch each way; the pre-activation tensors
 *     and their gradients never exist;
 *   * the DDPM block's embedding broadcast add is folded into GN2 (its input
 *     h + c is formed inside the GroupNorm kernels, never stored) and the
 *     embedding gradient's pixel sum into GN2's backward, wherever the fused
 *     shift kernels take the shape; elsewhere GN2 adds c into h in place and
 *     sums the gradient's pixels itself, as the reference does;
 *   * the EDM block's modulation gradient is a parallel reduction into a lent
 *     workspace;
 *   * the passes next to the convolutions are folded into the implicit-GEMM
 *     kernels (where those take the convolution): the residual add / mp_sum
 *     into the last convolution's epilogue, the EDM modulation + MP-SiLU into
 *     conv0's, and the MP-SiLU gradient with the wa residual into conv0's
 *     input-gradient epilogue;
 *   * the arena holds only what the backward reads (the inputs of the
 *     children) plus two gradient tensors that the backward reuses as each
 *     one's last reader has run.
 */
#include <math.h>

#include "layer.h"

/* ------------------------------------------------------------------------
 * DDPM residual block
 * ------------------------------------------------------------------------ */

enum { DS_GN1, DS_CONV1, DS_PROJ, DS_GN2, DS_CONV2 };
enum { DT_A1, DT_H, DT_C, DT_A2, DT_G0, DT_G1, DT_GC, DT_GEMB };
enum { DD_C, DD_EMB, DD_HW, DD_SLOT };

static void ddpm_fwd(Layer* L, const float* x, float* out, int batch, Context* ctx)
{
    Module** s = L->sub;
    float** t = L->buf;
    s[DS_GN1]->forward(s[DS_GN1], x, t[DT_A1], batch, ctx);                         /* a1 = silu(gn1(x)) */
    s[DS_CONV1]->forward(s[DS_CONV1], t[DT_A1], t[DT_H], batch, ctx);               /* h = conv1(a1) */
    s[DS_PROJ]->forward(s[DS_PROJ], ctx->cond[L->dim[DD_SLOT]].fwd, t[DT_C], batch, ctx); /* c = proj(emb) */
    groupnorm_shift_forward(s[DS_GN2], t[DT_H], t[DT_C], t[DT_A2], batch, ctx);      /* a2 = silu(gn2(h + c)) */
    conv2d_forward_residual(s[DS_CONV2], t[DT_A2], out, x, 1.0f, 1.0f, batch, ctx);  /* out = x + conv2(a2) */
}

static void ddpm_bwd(Layer* L, const float* x, const float* out, const float* g_out, float* g_x, int batch,
    Context* ctx)
{
    (void)out;
    Module** s = L->sub;
    float** t = L->buf;
    const int n = batch * L->dim[DD_HW] * L->dim[DD_C];
    CondSlot* slot = &ctx->cond[L->dim[DD_SLOT]];
    s[DS_CONV2]->backward(s[DS_CONV2], t[DT_A2], NULL, g_out, t[DT_G0], batch, ctx);   /* G0 = d a2 */
    groupnorm_shift_backward(s[DS_GN2], t[DT_H], t[DT_C], t[DT_G0], t[DT_G1], t[DT_GC], batch,
        ctx);                                                                          /* G1 = d h, dc */
    s[DS_PROJ]->backward(s[DS_PROJ], slot->fwd, t[DT_C], t[DT_GC], t[DT_GEMB], batch, ctx);
    launch_weighted_sum(slot->grad, slot->grad, t[DT_GEMB], 1.0f, 1.0f, batch * L->dim[DD_EMB], ctx->stream);
    s[DS_CONV1]->backward(s[DS_CONV1], t[DT_A1], NULL, t[DT_G1], t[DT_G0], batch, ctx); /* G0 = d a1 */
    s[DS_GN1]->backward(s[DS_GN1], x, NULL, t[DT_G0], t[DT_G1], batch, ctx);            /* G1 = d x (block) */
    launch_weighted_sum(g_x, g_out, t[DT_G1], 1.0f, 1.0f, n, ctx->stream);              /* + residual */
}

static const LayerKind kDdpmBlock = {"conv_residual", ddpm_fwd, ddpm_bwd};

Module* conv_residual_create(Context* ctx, int C, int emb_dim, int H, int W, int max_batch, int num_groups,
    int cond_slot)
{
    const int HW = H * W;
    Layer* L = layer_begin(&kDdpmBlock, HW * C, HW * C, max_batch);
    L->dim[DD_C] = C;
    L->dim[DD_EMB] = emb_dim;
    L->dim[DD_HW] = HW;
    L->dim[DD_SLOT] = cond_slot;
    /* children in the reference's creation order (its weight draws) */
    layer_sub(L, spatial_groupnorm_act_create(C, num_groups, H, W, max_batch, ACT_SILU));
    layer_sub(L, conv2d_create(ctx, C, C, 3, 1, 1, H, W, max_batch, 0, 1.0f));
    layer_sub(L, linear_create(ctx, emb_dim, C));
    layer_sub(L, spatial_groupnorm_act_shift_create(C, num_groups, H, W, max_batch, ACT_SILU));
    layer_sub(L, conv2d_create(ctx, C, C, 3, 1, 1, H, W, max_batch, 0, 1.0f));
    const size_t ns = (size_t)max_batch * HW * C;
    layer_buf(L, ns, 0);                                   /* a1 */
    layer_buf(L, ns, 0);                                   /* h */
    layer_buf(L, (size_t)max_batch * C, 0);                /* c */
    layer_buf(L, ns, 0);                                   /* a2 */
    layer_buf(L, ns, 0);                                   /* gradient tensor 0 */
    layer_buf(L, ns, 0);                                   /* gradient tensor 1 */
    layer_buf(L, (size_t)max_batch * C, 0);                /* dc */
    layer_buf(L, (size_t)max_batch * emb_dim, 0);          /* d emb of this block */
    return layer_end(L);
}

/* ------------------------------------------------------------------------
 * EDM2 residual block (spatial convolution variant)
 * ------------------------------------------------------------------------ */

enum { ES_CONV0, ES_LIN, ES_CONV1 };
enum { ET_H0, ET_H1, ET_C, ET_H3, ET_G0, ET_G1, ET_GC, ET_GEMB, ET_RED };
enum { ED_C, ED_EMB, ED_HW, ED_SLOT };

static void edm_fwd(Layer* L, const float* x, float* out, int batch, Context* ctx)
{
    Module** s = L->sub;
    float** t = L->buf;
    const int n = batch * L->dim[ED_HW] * L->dim[ED_C];
    launch_activation_forward(t[ET_H0], x, n, ACT_MP_SILU, ctx->stream);              /* h0 = mp_silu(x) */
    s[ES_LIN]->forward(s[ES_LIN], ctx->cond[L->dim[ED_SLOT]].fwd, t[ET_C], batch, ctx); /* c = lin(emb) */
    conv2d_forward_modulate_act(s[ES_CONV0], t[ET_H0], t[ET_H1], t[ET_H3], t[ET_C], ACT_MP_SILU, batch,
        ctx);                                                                         /* h1 = conv0(h0), h3 = mp_silu(h1 (c+1)) */
    conv2d_forward_residual(s[ES_CONV1], t[ET_H3], out, x, L->k[0], L->k[1], batch, ctx); /* mp_sum(x, conv1(h3), t) */
}

static void edm_bwd(Layer* L, const float* x, const float* out, const float* g_out, float* g_x, int batch,
    Context* ctx)
{
    (void)out;
    Module** s = L->sub;
    float** t = L->buf;
    const int n = batch * L->dim[ED_HW] * L->dim[ED_C];
    CondSlot* slot = &ctx->cond[L->dim[ED_SLOT]];
    launch_weighted_sum(t[ET_G0], g_out, g_out, L->k[1], 0.0f, n, ctx->stream);       /* G0 = wb d out */
    s[ES_CONV1]->backward(s[ES_CONV1], t[ET_H3], NULL, t[ET_G0], t[ET_G1], batch, ctx); /* G1 = d h3 */
    launch_spatial_modulate_act_backward(t[ET_G0], t[ET_GC], t[ET_G1], t[ET_H1], t[ET_C], batch, L->dim[ED_HW], 1,
        L->dim[ED_C], ACT_MP_SILU, t[ET_RED], ctx->stream);                           /* G0 = d h1, dc */
    conv2d_backward_act_residual(s[ES_CONV0], t[ET_H0], t[ET_G0], g_x, x, ACT_MP_SILU, g_out, L->k[0], t[ET_G1],
        batch, ctx);                                                                  /* d x = wa d out + d h0 mp_silu'(x) */
    s[ES_LIN]->backward(s[ES_LIN], slot->fwd, t[ET_C], t[ET_GC], t[ET_GEMB], batch, ctx);
    launch_weighted_sum(slot->grad, slot->grad, t[ET_GEMB], 1.0f, 1.0f, batch * L->dim[ED_EMB], ctx->stream);
}

static const LayerKind kEdmBlock = {"cond_conv_residual", edm_fwd, edm_bwd};

Module* cond_conv_residual_create(Context* ctx, int C, int emb_dim, int H, int W, int max_batch, float t,
    int cond_slot)
{
    const int HW = H * W;
    Layer* L = layer_begin(&kEdmBlock, HW * C, HW * C, max_batch);
    L->dim[ED_C] = C;
    L->dim[ED_EMB] = emb_dim;
    L->dim[ED_HW] = HW;
    L->dim[ED_SLOT] = cond_slot;
    /* mp_sum weights in host float (src/cond_conv_residual.c:108-110) */
    const float d = sqrtf((1.0f - t) * (1.0f - t) + t * t);
    L->k[0] = (1.0f - t) / d;
    L->k[1] = t / d;
    layer_sub(L, conv2d_create(ctx, C, C, 3, 1, 1, H, W, max_batch, 1, 1.0f));
    layer_sub(L, mp_linear_create(ctx, emb_dim, C, 0.0f));
    layer_sub(L, conv2d_create(ctx, C, C, 3, 1, 1, H, W, max_batch, 1, 1.0f));
    const size_t ns = (size_t)max_batch * HW * C;
    layer_buf(L, ns, 0);                                   /* h0 */
    layer_buf(L, ns, 0);                                   /* h1 */
    layer_buf(L, (size_t)max_batch * C, 0);                /* c */
    layer_buf(L, ns, 0);                                   /* h3 */
    layer_buf(L, ns, 0);                                   /* gradient tensor 0 */
    layer_buf(L, ns, 0);                                   /* gradient tensor 1 */
    layer_buf(L, (size_t)max_batch * C, 0);                /* dc */
    layer_buf(L, (size_t)max_batch * emb_dim, 0);          /* d emb of this block */
    layer_buf(L, nnhip_spatial_reduce_workspace(max_batch, HW, C), 1);
    return layer_end(L);
}
