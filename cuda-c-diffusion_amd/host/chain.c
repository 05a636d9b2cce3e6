/* chain.c -- the Sequential container (src/nn.h:295-301): modules run in a
 * chain, the container owning the tensors between them.
 *
 * Contract kept from the reference (src/sequential.c:31-118): the forward
 * input is copied into the container first (so the backward sees it even if
 * the caller reuses its buffer), module i reads the previous output and
 * writes its own, the backward walks the chain in reverse with each module
 * given the same in/out pointers it saw forward, sequential_output is the
 * last output and sequential_input_grad the gradient w.r.t. the input.
 *
 * Here every tensor of the chain lives in one device allocation: link i
 * holds module i and views of its input activation and of the gradient
 * w.r.t. that input; the chain's output follows the links' inputs.  Every
 * view starts on a 256-byte boundary whatever the widths and max_batch, so
 * the kernels' 128-bit accesses and alignment requirements hold for each.
 */
#include "nn_modules.h"

#define CHAIN_ALIGN_FLOATS 64

static size_t chain_round(size_t floats)
{
    return (floats + CHAIN_ALIGN_FLOATS - 1) / CHAIN_ALIGN_FLOATS * CHAIN_ALIGN_FLOATS;
}

typedef struct {
    Module* m;
    float* x;  /* the module's input (the chain input copy for link 0) */
    float* gx; /* gradient w.r.t. x */
} Link;

struct Sequential {
    int n, max_batch;
    Link* link;
    float* y; /* output of the last module */
    float* arena;
};

Sequential* sequential_create(Module** modules, int n, int max_batch)
{
    NN_ASSERT(n > 0, "sequential_create: empty chain");
    for (int i = 1; i < n; ++i) {
        if (modules[i]->in_dim != modules[i - 1]->out_dim) {
            fprintf(stderr, "sequential_create: %s produces %d values per sample but %s takes %d\n",
                modules[i - 1]->name, modules[i - 1]->out_dim, modules[i]->name, modules[i]->in_dim);
            exit(1);
        }
    }
    Sequential* s = (Sequential*)calloc(1, sizeof(Sequential));
    s->n = n;
    s->max_batch = max_batch;
    s->link = (Link*)calloc((size_t)n, sizeof(Link));
    /* n inputs + 1 output + n input gradients, each max_batch rows */
    const size_t mb = (size_t)max_batch;
    size_t total = chain_round(mb * (size_t)modules[n - 1]->out_dim);
    for (int i = 0; i < n; ++i) total += 2 * chain_round(mb * (size_t)modules[i]->in_dim);
    s->arena = nn_device_alloc(total);
    float* at = s->arena;
    for (int i = 0; i < n; ++i) {
        s->link[i].m = modules[i];
        s->link[i].x = at;
        at += chain_round(mb * (size_t)modules[i]->in_dim);
        s->link[i].gx = at;
        at += chain_round(mb * (size_t)modules[i]->in_dim);
    }
    s->y = at;
    return s;
}

void sequential_forward(Sequential* s, const float* input, int batch, Context* ctx)
{
    NN_ASSERT(batch <= s->max_batch, "sequential_forward: batch exceeds max_batch");
    NN_HIP_CHECK(hipMemcpyAsync(s->link[0].x, input, (size_t)batch * s->link[0].m->in_dim * sizeof(float),
        hipMemcpyDeviceToDevice, ctx->stream));
    for (int i = 0; i < s->n; ++i) {
        float* out = i + 1 < s->n ? s->link[i + 1].x : s->y;
        s->link[i].m->forward(s->link[i].m, s->link[i].x, out, batch, ctx);
    }
}

void sequential_backward(Sequential* s, const float* grad_output, int batch, Context* ctx)
{
    NN_ASSERT(batch <= s->max_batch, "sequential_backward: batch exceeds max_batch");
    const float* g = grad_output;
    for (int i = s->n - 1; i >= 0; --i) {
        Link* k = &s->link[i];
        const float* out = i + 1 < s->n ? s->link[i + 1].x : s->y;
        k->m->backward(k->m, k->x, out, g, k->gx, batch, ctx);
        g = k->gx;
    }
}

float* sequential_output(Sequential* s) { return s->y; }
float* sequential_input_grad(Sequential* s) { return s->link[0].gx; }

void sequential_parameters(Sequential* s, ParamList* pl)
{
    for (int i = 0; i < s->n; ++i)
        if (s->link[i].m->parameters) s->link[i].m->parameters(s->link[i].m, pl);
}

void sequential_free(Sequential* s)
{
    for (int i = 0; i < s->n; ++i) s->link[i].m->free(s->link[i].m);
    (void)hipFree(s->arena);
    free(s->link);
    free(s);
}
