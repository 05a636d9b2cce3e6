/* layer.c -- construction, the shared vtable and the device arena of the
 * host modules (see layer.h). */
#include <string.h>

#include "layer.h"

/* Each buffer starts on a 256-byte boundary: the kernels' vector accesses
   and workspace headers want at least 16. */
#define LAYER_ALIGN_FLOATS 64

static void layer_forward_vt(Module* self, const float* in, float* out, int batch, Context* ctx)
{
    Layer* L = as_layer(self);
    NN_ASSERT(L->max_batch <= 0 || batch <= L->max_batch, L->kind->name);
    L->kind->fwd(L, in, out, batch, ctx);
}

static void layer_backward_vt(Module* self, const float* in, const float* out, const float* grad_out,
    float* grad_in, int batch, Context* ctx)
{
    Layer* L = as_layer(self);
    NN_ASSERT(L->max_batch <= 0 || batch <= L->max_batch, L->kind->name);
    if (L->kind->bwd) L->kind->bwd(L, in, out, grad_out, grad_in, batch, ctx);
}

static void layer_parameters_vt(Module* self, ParamList* pl)
{
    Layer* L = as_layer(self);
    for (int i = 0; i < L->nparam; ++i) param_list_add(pl, L->buf[L->pval[i]], L->buf[L->pgrad[i]], L->pn[i]);
    for (int i = 0; i < L->nsub; ++i)
        if (L->sub[i]->parameters) L->sub[i]->parameters(L->sub[i], pl);
}

static void layer_free_vt(Module* self)
{
    Layer* L = as_layer(self);
    for (int i = 0; i < L->nsub; ++i) L->sub[i]->free(L->sub[i]);
    if (L->arena) (void)hipFree(L->arena);
    free(L);
}

Layer* layer_begin(const LayerKind* kind, int in_dim, int out_dim, int max_batch)
{
    Layer* L = (Layer*)calloc(1, sizeof(Layer));
    NN_ASSERT(L != NULL, "layer_begin: out of host memory");
    L->kind = kind;
    L->max_batch = max_batch;
    L->act = ACT_IDENTITY;
    L->mod.name = kind->name;
    L->mod.in_dim = in_dim;
    L->mod.out_dim = out_dim;
    L->mod.state = L;
    return L;
}

int layer_buf(Layer* L, size_t floats, int zero)
{
    NN_ASSERT(L->nbuf < LAYER_MAX_BUFS, "layer_buf: too many buffers");
    L->want[L->nbuf] = floats;
    L->zero[L->nbuf] = (unsigned char)(zero != 0);
    return L->nbuf++;
}

void layer_param(Layer* L, int value_buf, int grad_buf, int n)
{
    NN_ASSERT(L->nparam < LAYER_MAX_PARAMS, "layer_param: too many parameter tensors");
    L->pval[L->nparam] = value_buf;
    L->pgrad[L->nparam] = grad_buf;
    L->pn[L->nparam] = n;
    L->nparam++;
}

void layer_sub(Layer* L, Module* child)
{
    NN_ASSERT(L->nsub < LAYER_MAX_SUBS, "layer_sub: too many child modules");
    L->sub[L->nsub++] = child;
}

Module* layer_end(Layer* L)
{
    size_t total = 0, at[LAYER_MAX_BUFS];
    for (int i = 0; i < L->nbuf; ++i) {
        at[i] = total;
        total += (L->want[i] + LAYER_ALIGN_FLOATS - 1) / LAYER_ALIGN_FLOATS * LAYER_ALIGN_FLOATS;
    }
    if (total) {
        L->arena = nn_device_alloc(total);
        for (int i = 0; i < L->nbuf; ++i) {
            if (!L->want[i]) continue;
            L->buf[i] = L->arena + at[i];
            if (L->zero[i]) NN_HIP_CHECK(hipMemset(L->buf[i], 0, L->want[i] * sizeof(float)));
        }
    }
    L->mod.forward = layer_forward_vt;
    L->mod.backward = layer_backward_vt;
    L->mod.parameters = layer_parameters_vt;
    L->mod.free = layer_free_vt;
    return &L->mod;
}

void layer_fill_value(Layer* L, int b, size_t n, float value)
{
    if (!n) return;
    float* h = (float*)malloc(n * sizeof(float));
    NN_ASSERT(h != NULL, "layer_fill_value: out of host memory");
    for (size_t i = 0; i < n; ++i) h[i] = value;
    NN_HIP_CHECK(hipMemcpy(L->buf[b], h, n * sizeof(float), hipMemcpyHostToDevice));
    free(h);
}
