/* ema.c -- exponential moving average of the parameters.  Reference:
 * src/ema.c:5-69 (shadow copies at creation, shadow = decay*shadow +
 * (1-decay)*param with 1-decay in host float, swap via a temporary).
 * An update is one multi-tensor launch over the list. */
#include <string.h>

#include "nn_internal.h"

struct EMA {
    float decay;
    int count;
    int* sizes;
    float** shadow;
    NnMultiTensorPlan* plan;
    Param* plan_items;
};

EMA* ema_create(const ParamList* pl, float decay)
{
    EMA* ema = (EMA*)calloc(1, sizeof(EMA));
    ema->decay = decay;
    ema->count = pl->count;
    ema->sizes = (int*)malloc((size_t)(pl->count > 0 ? pl->count : 1) * sizeof(int));
    ema->shadow = (float**)malloc((size_t)(pl->count > 0 ? pl->count : 1) * sizeof(float*));
    for (int i = 0; i < pl->count; ++i) {
        ema->sizes[i] = pl->items[i].size;
        ema->shadow[i] = nn_device_alloc((size_t)pl->items[i].size);
        NN_HIP_CHECK(hipMemcpy(ema->shadow[i], pl->items[i].param,
            (size_t)pl->items[i].size * sizeof(float), hipMemcpyDeviceToDevice));
    }
    return ema;
}

int nn_ema_count(const EMA* ema) { return ema->count; }
float nn_ema_decay(const EMA* ema) { return ema->decay; }
float* nn_ema_shadow(const EMA* ema, int i) { return ema->shadow[i]; }

void ema_update(EMA* ema, const ParamList* pl, Context* ctx)
{
    NN_ASSERT(pl->count == ema->count, "ema_update: list does not match the EMA");
    if (!ema->plan || memcmp(ema->plan_items, pl->items, (size_t)pl->count * sizeof(Param)) != 0) {
        nnhip_multi_tensor_plan_destroy(ema->plan);
        free(ema->plan_items);
        NnTensorSlot* slots = (NnTensorSlot*)calloc((size_t)(pl->count > 0 ? pl->count : 1), sizeof(NnTensorSlot));
        for (int i = 0; i < pl->count; ++i) {
            NN_ASSERT(pl->items[i].size == ema->sizes[i], "ema_update: tensor size changed");
            slots[i].p = pl->items[i].param;
            slots[i].shadow = ema->shadow[i];
            slots[i].n = pl->items[i].size;
        }
        ema->plan = nnhip_multi_tensor_plan_create(slots, pl->count);
        free(slots);
        NN_ASSERT(ema->plan != NULL, "ema_update: plan creation failed");
        ema->plan_items = (Param*)malloc((size_t)(pl->count > 0 ? pl->count : 1) * sizeof(Param));
        memcpy(ema->plan_items, pl->items, (size_t)pl->count * sizeof(Param));
    }
    launch_ema_update(ema->plan, ema->decay, 1.0f - ema->decay, ctx->stream);
}

void ema_swap(EMA* ema, ParamList* pl, Context* ctx)
{
    int max_size = 0;
    for (int i = 0; i < ema->count; ++i)
        if (ema->sizes[i] > max_size) max_size = ema->sizes[i];
    float* tmp = nn_device_alloc((size_t)max_size);
    for (int i = 0; i < ema->count; ++i) {
        size_t bytes = (size_t)ema->sizes[i] * sizeof(float);
        NN_HIP_CHECK(hipMemcpyAsync(tmp, pl->items[i].param, bytes, hipMemcpyDeviceToDevice, ctx->stream));
        NN_HIP_CHECK(hipMemcpyAsync(pl->items[i].param, ema->shadow[i], bytes, hipMemcpyDeviceToDevice, ctx->stream));
        NN_HIP_CHECK(hipMemcpyAsync(ema->shadow[i], tmp, bytes, hipMemcpyDeviceToDevice, ctx->stream));
    }
    NN_HIP_CHECK(hipStreamSynchronize(ctx->stream));
    (void)hipFree(tmp);
}

void ema_shadow_list(const EMA* ema, ParamList* shadow)
{
    for (int i = 0; i < ema->count; ++i) param_list_add(shadow, ema->shadow[i], NULL, ema->sizes[i]);
}

void ema_free(EMA* ema)
{
    for (int i = 0; i < ema->count; ++i) (void)hipFree(ema->shadow[i]);
    free(ema->shadow);
    free(ema->sizes);
    nnhip_multi_tensor_plan_destroy(ema->plan);
    free(ema->plan_items);
    free(ema);
}
