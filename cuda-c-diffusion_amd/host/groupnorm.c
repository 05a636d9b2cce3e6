/* groupnorm.c -- NHWC GroupNorm module and the fused GroupNorm+activation
 * module.  Reference: src/groupnorm.c:4-87 (state, eps 1e-5, gamma=1,
 * beta=0, C % G assertion, cached mu/rstd of the last forward).
 * The backward lends the launch layer a workspace sized for max_batch so a
 * call allocates nothing.
 */
#include "nn_modules.h"

typedef struct {
    int C, G, H, W, max_batch;
    Activation act; /* ACT_IDENTITY for the plain GroupNorm */
    float eps;
    float *gamma, *beta;
    float *ggamma, *gbeta;
    float *mu, *rstd;
    float* work;     /* backward workspace, sized for max_batch */
    float* fwork;    /* forward workspace, sized for max_batch (NULL when none is needed) */
} GroupNormState;

static void groupnorm_forward(Module* self, const float* in, float* out, int batch, Context* ctx)
{
    GroupNormState* st = (GroupNormState*)self->state;
    NN_ASSERT(batch <= st->max_batch, "groupnorm: batch exceeds max_batch");
    launch_groupnorm_act_forward_ws(out, st->mu, st->rstd, in, st->gamma, st->beta, batch,
        st->H * st->W, st->C, st->G, st->eps, st->act, st->fwork, ctx->stream);
}

static void groupnorm_backward(Module* self, const float* in, const float* out,
    const float* grad_out, float* grad_in, int batch, Context* ctx)
{
    (void)out;
    GroupNormState* st = (GroupNormState*)self->state;
    NN_ASSERT(batch <= st->max_batch, "groupnorm: batch exceeds max_batch");
    launch_groupnorm_act_backward_ws(grad_in, st->ggamma, st->gbeta, grad_out, in, st->gamma,
        st->beta, st->mu, st->rstd, batch, st->H * st->W, st->C, st->G, st->act, st->work,
        ctx->stream);
}

static void groupnorm_parameters(Module* self, ParamList* pl)
{
    GroupNormState* st = (GroupNormState*)self->state;
    param_list_add(pl, st->gamma, st->ggamma, st->C);
    param_list_add(pl, st->beta, st->gbeta, st->C);
}

static void groupnorm_free(Module* self)
{
    GroupNormState* st = (GroupNormState*)self->state;
    (void)hipFree(st->gamma);
    (void)hipFree(st->beta);
    (void)hipFree(st->ggamma);
    (void)hipFree(st->gbeta);
    (void)hipFree(st->mu);
    (void)hipFree(st->rstd);
    (void)hipFree(st->work);
    if (st->fwork) (void)hipFree(st->fwork);
    free(st);
    free(self);
}

static Module* groupnorm_make(int C, int num_groups, int H, int W, int max_batch, Activation act,
    const char* name)
{
    NN_ASSERT(num_groups > 0 && C % num_groups == 0, "groupnorm: C must be divisible by num_groups");
    Module* m = (Module*)malloc(sizeof(Module));
    GroupNormState* st = (GroupNormState*)malloc(sizeof(GroupNormState));
    st->C = C;
    st->G = num_groups;
    st->H = H;
    st->W = W;
    st->max_batch = max_batch;
    st->act = act;
    st->eps = 1e-5f;
    st->gamma = nn_device_alloc((size_t)C);
    st->beta = nn_device_alloc((size_t)C);
    st->ggamma = nn_device_alloc((size_t)C);
    st->gbeta = nn_device_alloc((size_t)C);
    st->mu = nn_device_alloc((size_t)max_batch * num_groups);
    st->rstd = nn_device_alloc((size_t)max_batch * num_groups);
    {
        const size_t bw = nnhip_groupnorm_backward_workspace(max_batch, H * W, C, num_groups);
        st->work = nn_device_alloc(bw);
        NN_HIP_CHECK(hipMemset(st->work, 0, (bw ? bw : 1) * sizeof(float)));  /* status word starts clear */
    }
    {
        /* The forward need grows with the batch, so the max_batch size covers
         * every smaller batch; 0 means no workspace (the launcher then draws
         * one from the stream-ordered pool if a smaller batch wants one). */
        const size_t fw = nnhip_groupnorm_forward_workspace(max_batch, H * W, C, num_groups);
        st->fwork = fw ? nn_device_alloc(fw) : NULL;
        if (st->fwork) NN_HIP_CHECK(hipMemset(st->fwork, 0, fw * sizeof(float)));
    }

    float* ones = (float*)malloc((size_t)C * sizeof(float));
    for (int i = 0; i < C; ++i) ones[i] = 1.0f;
    NN_HIP_CHECK(hipMemcpy(st->gamma, ones, (size_t)C * sizeof(float), hipMemcpyHostToDevice));
    NN_HIP_CHECK(hipMemset(st->beta, 0, (size_t)C * sizeof(float)));
    free(ones);

    m->name = name;
    m->in_dim = H * W * C;
    m->out_dim = H * W * C;
    m->state = st;
    m->forward = groupnorm_forward;
    m->backward = groupnorm_backward;
    m->parameters = groupnorm_parameters;
    m->free = groupnorm_free;
    return m;
}

Module* spatial_groupnorm_create(int C, int num_groups, int H, int W, int max_batch)
{
    return groupnorm_make(C, num_groups, H, W, max_batch, ACT_IDENTITY, "groupnorm");
}

Module* spatial_groupnorm_act_create(int C, int num_groups, int H, int W, int max_batch,
    Activation act)
{
    return groupnorm_make(C, num_groups, H, W, max_batch, act, "groupnorm_act");
}
