/* ema.c -- exponential moving average of a parameter list (src/nn.h:
 * 240-246).
 *
 * Contract kept from the reference (src/ema.c:12-69): the shadow starts as a
 * copy of the parameters; an update is shadow = decay * shadow + (1 - decay)
 * * param, with 1 - decay formed in host float (src/ema.c:33), after the
 * optimizer step; ema_swap exchanges parameters and shadow (to sample with
 * the averaged weights and back) and returns with the exchange done.
 *
 * Here the shadow is one device allocation holding every tensor (plus a
 * spare the size of the largest, for ema_swap), and an update is one launch
 * of the multi-tensor kernel over a plan of (param, shadow) pairs, rebuilt
 * only when the parameter list changes.
 */
#include <string.h>

#include "nn_internal.h"

struct EMA {
    float decay;
    int count;
    int* n;          /* tensor sizes, ParamList order */
    float** shadow;  /* views into the arena */
    float* spare;    /* swap buffer (view into the arena) */
    float* arena;
    NnMultiTensorPlan* plan;
    float** plan_param; /* the parameter pointers the plan was built for */
};

EMA* ema_create(const ParamList* pl, float decay)
{
    EMA* e = (EMA*)calloc(1, sizeof(EMA));
    e->decay = decay;
    e->count = pl->count;
    const int slots = pl->count > 0 ? pl->count : 1;
    e->n = (int*)calloc((size_t)slots, sizeof(int));
    e->shadow = (float**)calloc((size_t)slots, sizeof(float*));
    e->plan_param = (float**)calloc((size_t)slots, sizeof(float*));
    size_t total = 0, largest = 0;
    for (int i = 0; i < pl->count; ++i) {
        const size_t n = (size_t)pl->items[i].size;
        total += (n + 63) / 64 * 64; /* 256-byte aligned views */
        if (n > largest) largest = n;
    }
    e->arena = nn_device_alloc(total + largest);
    float* at = e->arena;
    for (int i = 0; i < pl->count; ++i) {
        e->n[i] = pl->items[i].size;
        e->shadow[i] = at;
        at += ((size_t)e->n[i] + 63) / 64 * 64;
        NN_HIP_CHECK(hipMemcpy(e->shadow[i], pl->items[i].param, (size_t)e->n[i] * sizeof(float),
            hipMemcpyDeviceToDevice));
    }
    e->spare = at;
    return e;
}

int nn_ema_count(const EMA* ema) { return ema->count; }
float nn_ema_decay(const EMA* ema) { return ema->decay; }
float* nn_ema_shadow(const EMA* ema, int i) { return ema->shadow[i]; }

/* The (param, shadow) plan for this list, rebuilt when its pointers change. */
static const NnMultiTensorPlan* ema_plan(EMA* e, const ParamList* pl)
{
    NN_ASSERT(pl->count == e->count, "ema_update: list does not match the EMA");
    int same = e->plan != NULL;
    for (int i = 0; same && i < pl->count; ++i) same = e->plan_param[i] == pl->items[i].param;
    if (same) return e->plan;
    nnhip_multi_tensor_plan_destroy(e->plan);
    NnTensorSlot* t = (NnTensorSlot*)calloc((size_t)(pl->count > 0 ? pl->count : 1), sizeof(NnTensorSlot));
    for (int i = 0; i < pl->count; ++i) {
        NN_ASSERT(pl->items[i].size == e->n[i], "ema_update: tensor size changed");
        t[i].p = pl->items[i].param;
        t[i].shadow = e->shadow[i];
        t[i].n = e->n[i];
        e->plan_param[i] = pl->items[i].param;
    }
    e->plan = nnhip_multi_tensor_plan_create(t, pl->count);
    free(t);
    NN_ASSERT(e->plan != NULL, "ema_update: plan creation failed");
    return e->plan;
}

void ema_update(EMA* ema, const ParamList* pl, Context* ctx)
{
    launch_ema_update(ema_plan(ema, pl), ema->decay, 1.0f - ema->decay, ctx->stream);
}

void ema_swap(EMA* ema, ParamList* pl, Context* ctx)
{
    NN_ASSERT(pl->count == ema->count, "ema_swap: list does not match the EMA");
    for (int i = 0; i < ema->count; ++i) {
        const size_t bytes = (size_t)ema->n[i] * sizeof(float);
        NN_HIP_CHECK(hipMemcpyAsync(ema->spare, pl->items[i].param, bytes, hipMemcpyDeviceToDevice, ctx->stream));
        NN_HIP_CHECK(hipMemcpyAsync(pl->items[i].param, ema->shadow[i], bytes, hipMemcpyDeviceToDevice, ctx->stream));
        NN_HIP_CHECK(hipMemcpyAsync(ema->shadow[i], ema->spare, bytes, hipMemcpyDeviceToDevice, ctx->stream));
    }
    NN_HIP_CHECK(hipStreamSynchronize(ctx->stream));
}

void ema_shadow_list(const EMA* ema, ParamList* shadow)
{
    for (int i = 0; i < ema->count; ++i) param_list_add(shadow, ema->shadow[i], NULL, ema->n[i]);
}

void ema_free(EMA* ema)
{
    nnhip_multi_tensor_plan_destroy(ema->plan);
    (void)hipFree(ema->arena);
    free(ema->plan_param);
    free(ema->shadow);
    free(ema->n);
    free(ema);
}
