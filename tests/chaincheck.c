/* chaincheck.c -- the Sequential container against the same modules called
 * one by one (src/sequential.c:31-118 semantics): bit-identical output,
 * input gradient and parameter gradients, the ParamList in module order, and
 * the forward input copied into the chain (the caller may reuse its buffer
 * before the backward).  Built into tests/_build/libgradcheck.so;
 * nn_chaincheck_run() returns the number of mismatches (0 = pass);
 * nn_chaincheck_odd_run() does the same for a chain whose first link has an
 * odd width and an odd batch ahead of an implicit-GEMM convolution, which
 * needs its input view 16-byte aligned.  Needs a GPU. */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "nn_modules.h"

static float* upload_random(Context* ctx, int n)
{
    float* d = nn_device_alloc((size_t)n);
    nn_fill_normal(ctx, d, (size_t)n, 0.0f, 1.0f);
    return d;
}

static float* fetch(const float* d, int n)
{
    float* h = (float*)malloc((size_t)n * sizeof(float));
    NN_HIP_CHECK(hipMemcpy(h, d, (size_t)n * sizeof(float), hipMemcpyDeviceToHost));
    return h;
}

static int differs(const char* what, const float* a, const float* b, int n)
{
    if (memcmp(a, b, (size_t)n * sizeof(float)) == 0) return 0;
    fprintf(stderr, "chaincheck: %s differs\n", what);
    return 1;
}

int nn_chaincheck_run(void)
{
    const int batch = 6, D = 64, O = 32;
    Context ctx;
    nn_context_init(&ctx, 99, 0);
    Module* mods[3] = {layernorm_create(D, batch), activation_create(D, ACT_SILU), linear_create(&ctx, D, O)};
    Sequential* s = sequential_create(mods, 3, batch);
    int bad = 0;

    ParamList pl;
    param_list_init(&pl);
    sequential_parameters(s, &pl);
    const int want[4] = {D, D, D * O, O};
    bad += pl.count != 4;
    for (int i = 0; i < pl.count && i < 4; ++i) bad += pl.items[i].size != want[i];

    float* x = upload_random(&ctx, batch * D);
    float* g = upload_random(&ctx, batch * O);
    float* x_saved = fetch(x, batch * D);
    sequential_forward(s, x, batch, &ctx);
    nn_fill_normal(&ctx, x, (size_t)batch * D, 0.0f, 1.0f); /* the caller reuses its input buffer */
    sequential_backward(s, g, batch, &ctx);
    NN_HIP_CHECK(hipDeviceSynchronize());
    float* y_chain = fetch(sequential_output(s), batch * O);
    float* gx_chain = fetch(sequential_input_grad(s), batch * D);
    float* pg_chain[4];
    for (int i = 0; i < 4 && i < pl.count; ++i) pg_chain[i] = fetch(pl.items[i].grad, pl.items[i].size);

    /* the same modules by hand, on the original input */
    float *xin = nn_device_alloc((size_t)batch * D), *t1 = nn_device_alloc((size_t)batch * D),
          *t2 = nn_device_alloc((size_t)batch * D), *y = nn_device_alloc((size_t)batch * O),
          *g2 = nn_device_alloc((size_t)batch * D), *g1 = nn_device_alloc((size_t)batch * D),
          *g0 = nn_device_alloc((size_t)batch * D);
    NN_HIP_CHECK(hipMemcpy(xin, x_saved, (size_t)batch * D * sizeof(float), hipMemcpyHostToDevice));
    mods[0]->forward(mods[0], xin, t1, batch, &ctx);
    mods[1]->forward(mods[1], t1, t2, batch, &ctx);
    mods[2]->forward(mods[2], t2, y, batch, &ctx);
    mods[2]->backward(mods[2], t2, y, g, g2, batch, &ctx);
    mods[1]->backward(mods[1], t1, t2, g2, g1, batch, &ctx);
    mods[0]->backward(mods[0], xin, t1, g1, g0, batch, &ctx);
    NN_HIP_CHECK(hipDeviceSynchronize());
    float* y_hand = fetch(y, batch * O);
    float* gx_hand = fetch(g0, batch * D);
    bad += differs("output", y_chain, y_hand, batch * O);
    bad += differs("input gradient", gx_chain, gx_hand, batch * D);
    for (int i = 0; i < 4 && i < pl.count; ++i) {
        float* h = fetch(pl.items[i].grad, pl.items[i].size);
        char what[32];
        snprintf(what, sizeof what, "parameter gradient %d", i);
        bad += differs(what, pg_chain[i], h, pl.items[i].size);
        free(h);
        free(pg_chain[i]);
    }

    float* bufs[] = {x, g, xin, t1, t2, y, g2, g1, g0};
    for (size_t i = 0; i < sizeof bufs / sizeof bufs[0]; ++i) (void)hipFree(bufs[i]);
    free(x_saved);
    free(y_chain);
    free(gx_chain);
    free(y_hand);
    free(gx_hand);
    param_list_free(&pl);
    sequential_free(s);
    nn_context_destroy(&ctx);
    return bad;
}

/* The chain against its modules run by hand on separately allocated tensors:
   output, input gradient and every parameter gradient bit for bit. */
static int chain_vs_hand(Context* ctx, Module** mods, int n, int batch)
{
    Sequential* s = sequential_create(mods, n, batch);
    const int in0 = mods[0]->in_dim, outn = mods[n - 1]->out_dim;
    float* x = upload_random(ctx, batch * in0);
    float* g = upload_random(ctx, batch * outn);
    sequential_forward(s, x, batch, ctx);
    sequential_backward(s, g, batch, ctx);
    NN_HIP_CHECK(hipDeviceSynchronize());
    int bad = nnhip_get_last_error(NULL, 0) != 0;
    float* y_chain = fetch(sequential_output(s), batch * outn);
    float* gx_chain = fetch(sequential_input_grad(s), batch * in0);
    ParamList pl;
    param_list_init(&pl);
    sequential_parameters(s, &pl);
    float** pg = (float**)calloc((size_t)pl.count, sizeof(float*));
    for (int i = 0; i < pl.count; ++i) pg[i] = fetch(pl.items[i].grad, pl.items[i].size);

    float** act = (float**)calloc((size_t)n + 1, sizeof(float*));
    float** grd = (float**)calloc((size_t)n + 1, sizeof(float*));
    for (int i = 0; i <= n; ++i) {
        const int w = i < n ? mods[i]->in_dim : outn;
        act[i] = nn_device_alloc((size_t)batch * w);
        grd[i] = nn_device_alloc((size_t)batch * w);
    }
    NN_HIP_CHECK(hipMemcpy(act[0], x, (size_t)batch * in0 * sizeof(float), hipMemcpyDeviceToDevice));
    NN_HIP_CHECK(hipMemcpy(grd[n], g, (size_t)batch * outn * sizeof(float), hipMemcpyDeviceToDevice));
    for (int i = 0; i < n; ++i) mods[i]->forward(mods[i], act[i], act[i + 1], batch, ctx);
    for (int i = n - 1; i >= 0; --i) mods[i]->backward(mods[i], act[i], act[i + 1], grd[i + 1], grd[i], batch, ctx);
    NN_HIP_CHECK(hipDeviceSynchronize());
    bad += nnhip_get_last_error(NULL, 0) != 0;
    float* y_hand = fetch(act[n], batch * outn);
    float* gx_hand = fetch(grd[0], batch * in0);
    bad += differs("output", y_chain, y_hand, batch * outn);
    bad += differs("input gradient", gx_chain, gx_hand, batch * in0);
    for (int i = 0; i < pl.count; ++i) {
        float* h = fetch(pl.items[i].grad, pl.items[i].size);
        char what[32];
        snprintf(what, sizeof what, "parameter gradient %d", i);
        bad += differs(what, pg[i], h, pl.items[i].size);
        free(h);
        free(pg[i]);
    }
    for (int i = 0; i <= n; ++i) {
        (void)hipFree(act[i]);
        (void)hipFree(grd[i]);
    }
    free(act);
    free(grd);
    free(pg);
    free(y_chain);
    free(gx_chain);
    free(y_hand);
    free(gx_hand);
    param_list_free(&pl);
    (void)hipFree(x);
    (void)hipFree(g);
    sequential_free(s);
    return bad;
}

int nn_chaincheck_odd_run(void)
{
    /* linear 3 -> 8*8*32 at batch 3: the first link's views hold 9 floats
       each, so the convolution's input view would start 72 bytes into the
       arena without the chain's 256-byte rounding */
    const int batch = 3, H = 8, W = 8, C = 32;
    Context ctx;
    nn_context_init(&ctx, 101, 0);
    Module* mods[2] = {linear_create(&ctx, 3, H * W * C), conv2d_create(&ctx, C, 64, 3, 1, 1, H, W, batch, 0, 1.0f)};
    const int bad = chain_vs_hand(&ctx, mods, 2, batch);
    nn_context_destroy(&ctx);
    return bad;
}
