/* optimizer.c -- SGD and Adam over a ParamList.  Reference:
 * src/optimizer.c:7-97 (per-tensor zeroed moments, step counter, host-float
 * bias corrections 1-powf(beta, t)).  Adam steps are one multi-tensor launch
 * over the whole list (the plan is built on first use and rebuilt when the
 * list changes); optimizer_step_ema folds the EMA update into the same launch.
 */
#include <math.h>
#include <string.h>

#include "nn_hip_rt.h"
#include "nn_internal.h"

typedef enum { OPT_SGD = 0, OPT_ADAM } OptKind;

struct Optimizer {
    OptKind kind;
    float lr, beta1, beta2, eps;
    int t;
    int n;
    int* sizes;
    float **m, **v;
    /* multi-tensor plan and the list (and EMA) it was built for */
    NnMultiTensorPlan* plan;
    const EMA* plan_ema;
    Param* plan_items;
    int plan_count;
};

Optimizer* optimizer_sgd(const ParamList* pl, float lr)
{
    Optimizer* o = (Optimizer*)calloc(1, sizeof(Optimizer));
    o->kind = OPT_SGD;
    o->lr = lr;
    o->n = pl->count;
    return o;
}

Optimizer* optimizer_adam(const ParamList* pl, float lr, float beta1, float beta2, float eps)
{
    Optimizer* o = (Optimizer*)calloc(1, sizeof(Optimizer));
    o->kind = OPT_ADAM;
    o->lr = lr;
    o->beta1 = beta1;
    o->beta2 = beta2;
    o->eps = eps;
    o->n = pl->count;
    o->sizes = (int*)malloc((size_t)(o->n > 0 ? o->n : 1) * sizeof(int));
    o->m = (float**)malloc((size_t)(o->n > 0 ? o->n : 1) * sizeof(float*));
    o->v = (float**)malloc((size_t)(o->n > 0 ? o->n : 1) * sizeof(float*));
    for (int i = 0; i < o->n; ++i) {
        size_t sz = (size_t)pl->items[i].size;
        o->sizes[i] = pl->items[i].size;
        o->m[i] = nn_device_alloc(sz);
        o->v[i] = nn_device_alloc(sz);
        NN_HIP_CHECK(hipMemset(o->m[i], 0, sz * sizeof(float)));
        NN_HIP_CHECK(hipMemset(o->v[i], 0, sz * sizeof(float)));
    }
    return o;
}

static int plan_matches(const Optimizer* o, const ParamList* pl, const EMA* ema)
{
    if (!o->plan || o->plan_ema != ema || o->plan_count != pl->count) return 0;
    return memcmp(o->plan_items, pl->items, (size_t)pl->count * sizeof(Param)) == 0;
}

static void ensure_plan(Optimizer* o, const ParamList* pl, const EMA* ema)
{
    if (plan_matches(o, pl, ema)) return;
    NN_ASSERT(pl->count == o->n, "optimizer: parameter list does not match the optimizer");
    NN_ASSERT(!ema || nn_ema_count(ema) == pl->count, "optimizer: EMA does not match the list");
    nnhip_multi_tensor_plan_destroy(o->plan);
    free(o->plan_items);
    NnTensorSlot* slots = (NnTensorSlot*)malloc((size_t)(pl->count > 0 ? pl->count : 1) * sizeof(NnTensorSlot));
    for (int i = 0; i < pl->count; ++i) {
        NN_ASSERT(pl->items[i].size == o->sizes[i], "optimizer: tensor size changed");
        slots[i].p = pl->items[i].param;
        slots[i].m = o->m[i];
        slots[i].v = o->v[i];
        slots[i].g = pl->items[i].grad;
        slots[i].shadow = ema ? nn_ema_shadow(ema, i) : NULL;
        slots[i].n = pl->items[i].size;
    }
    o->plan = nnhip_multi_tensor_plan_create(slots, pl->count);
    free(slots);
    if (!o->plan) {
        char msg[256];
        nnhip_get_last_error(msg, sizeof msg);
        fprintf(stderr, "optimizer: %s\n", msg);
        exit(1);
    }
    o->plan_ema = ema;
    o->plan_count = pl->count;
    o->plan_items = (Param*)malloc((size_t)(pl->count > 0 ? pl->count : 1) * sizeof(Param));
    memcpy(o->plan_items, pl->items, (size_t)pl->count * sizeof(Param));
}

static void adam_launch(Optimizer* o, const ParamList* pl, const EMA* ema, Context* ctx)
{
    ensure_plan(o, pl, ema);
    o->t++;
    float bc1 = 1.0f - powf(o->beta1, (float)o->t);
    float bc2 = 1.0f - powf(o->beta2, (float)o->t);
    float w0 = 1.0f, w1 = 0.0f;
    if (ema) {
        w0 = nn_ema_decay(ema);
        w1 = 1.0f - nn_ema_decay(ema);
    }
    launch_adam_ema_step(o->plan, o->lr, o->beta1, o->beta2, o->eps, bc1, bc2, w0, w1, ctx->stream);
}

void optimizer_step(Optimizer* o, const ParamList* pl, Context* ctx)
{
    if (o->kind == OPT_SGD) {
        for (int i = 0; i < pl->count; ++i)
            launch_sgd_step(pl->items[i].param, pl->items[i].grad, o->lr, pl->items[i].size, ctx->stream);
        return;
    }
    adam_launch(o, pl, NULL, ctx);
}

void optimizer_step_ema(Optimizer* o, EMA* ema, const ParamList* pl, Context* ctx)
{
    NN_ASSERT(o->kind == OPT_ADAM, "optimizer_step_ema: Adam only");
    adam_launch(o, pl, ema, ctx);
}

void optimizer_set_lr(Optimizer* o, float lr) { o->lr = lr; }
int optimizer_timestep(const Optimizer* o) { return o->t; }
void optimizer_set_timestep(Optimizer* o, int t) { o->t = t; }

void optimizer_moment_lists(const Optimizer* o, ParamList* m, ParamList* v)
{
    NN_ASSERT(o->kind == OPT_ADAM, "optimizer_moment_lists: Adam only");
    for (int i = 0; i < o->n; ++i) {
        param_list_add(m, o->m[i], NULL, o->sizes[i]);
        param_list_add(v, o->v[i], NULL, o->sizes[i]);
    }
}

void optimizer_free(Optimizer* o)
{
    if (o->m) {
        for (int i = 0; i < o->n; ++i) {
            (void)hipFree(o->m[i]);
            (void)hipFree(o->v[i]);
        }
    }
    free(o->m);
    free(o->v);
    free(o->sizes);
    nnhip_multi_tensor_plan_destroy(o->plan);
    free(o->plan_items);
    free(o);
}
