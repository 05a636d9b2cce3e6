/* blockcheck.c -- the fused diffusion blocks against the reference's own
 * composition of the same launchers (built into _build/libgradcheck.so).
 *
 * The reference DDPM block (src/conv_residual.c:21-66) runs GroupNorm, then a
 * separate SiLU launch, keeps h0/h3, and adds / reduces the embedding with
 * spatial_add / spatial_reduce_sum; the EDM block (src/cond_conv_residual.c:
 * 22-62) runs spatial_modulate and the MP-SiLU as two launches each way.
 * Here those sequences are rebuilt from separate modules and launchers, given
 * the fused block's parameters (same ParamList order and sizes), and both are
 * run forward and backward on the same input and embedding.  Reported: the
 * largest relative difference (max |a - b| / max(|b|, rms(b), floor)) over
 * out, grad_in, every parameter gradient and the embedding gradient, where
 * `floor` is 0 except for the DDPM embedding path's reduced outputs, whose
 * floor is the scale sqrt(sum terms^2) of the terms they add (per tensor, the
 * largest over its entries).  Each tensor's difference is printed on stderr.
 * Needs a GPU.
 */
#define _POSIX_C_SOURCE 200809L
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "nn_modules.h"

static Context g;

static float* dev_normal(size_t n, float std)
{
    float* p = nn_device_alloc(n);
    nn_fill_normal(&g, p, n, 0.0f, std);
    return p;
}

/* max |a - b| / max(|b|, rms(b), floor): `floor` is the scale of the terms a
   reduced output sums (0 for none), so that a sum which cancels to rounding
   noise is measured against the size of what it adds up. */
static double rel_diff_floor(const float* da, const float* db, size_t n, double extra)
{
    float* a = (float*)malloc(n * sizeof(float));
    float* b = (float*)malloc(n * sizeof(float));
    NN_HIP_CHECK(hipMemcpy(a, da, n * sizeof(float), hipMemcpyDeviceToHost));
    NN_HIP_CHECK(hipMemcpy(b, db, n * sizeof(float), hipMemcpyDeviceToHost));
    double ss = 0.0;
    for (size_t i = 0; i < n; ++i) ss += (double)b[i] * b[i];
    const double floor = fmax(n ? sqrt(ss / (double)n) : 0.0, extra);
    double worst = 0.0;
    for (size_t i = 0; i < n; ++i) {
        const double d = fabs((double)a[i] - b[i]) / fmax(fmax(fabs((double)b[i]), floor), 1e-30);
        if (d > worst) worst = d;
    }
    free(a);
    free(b);
    return worst;
}

static double rel_diff(const float* da, const float* db, size_t n) { return rel_diff_floor(da, db, n, 0.0); }

static float* to_host(const float* d, size_t n)
{
    float* h = (float*)malloc(n * sizeof(float));
    NN_HIP_CHECK(hipMemcpy(h, d, n * sizeof(float), hipMemcpyDeviceToHost));
    return h;
}

/* Reference-structure DDPM block state. */
typedef struct {
    Module *gn1, *conv1, *time_proj, *gn2, *conv2;
    float *h0, *h1, *h2, *h3, *h4, *c, *gh4, *gh3, *gh2, *gh1, *gh0, *gxb, *gc, *gemb;
} RefDDPM;

static void copy_params(Module* dst, Module* src)
{
    ParamList a, b;
    param_list_init(&a);
    param_list_init(&b);
    dst->parameters(dst, &a);
    src->parameters(src, &b);
    NN_ASSERT(a.count == b.count, "blockcheck: parameter count");
    for (int k = 0; k < a.count; ++k) {
        NN_ASSERT(a.items[k].size == b.items[k].size, "blockcheck: parameter size");
        NN_HIP_CHECK(hipMemcpy(a.items[k].param, b.items[k].param, (size_t)a.items[k].size * sizeof(float),
            hipMemcpyDeviceToDevice));
    }
    param_list_free(&a);
    param_list_free(&b);
}

/* Largest difference over the parameter gradients; floors[k] (or 0 when
   floors is NULL or k is past nfloors) is parameter k's term scale. */
static double grads_diff(Module* a, Module* b, const double* floors, int nfloors)
{
    ParamList pa, pb;
    param_list_init(&pa);
    param_list_init(&pb);
    a->parameters(a, &pa);
    b->parameters(b, &pb);
    double worst = 0.0;
    for (int k = 0; k < pa.count; ++k) {
        const double f = floors && k < nfloors ? floors[k] : 0.0;
        const double d = rel_diff_floor(pa.items[k].grad, pb.items[k].grad, (size_t)pa.items[k].size, f);
        fprintf(stderr, "  parameter %d (%d floats) gradient: %.3e (term floor %.3e)\n", k, pa.items[k].size, d, f);
        if (d > worst) worst = d;
    }
    param_list_free(&pa);
    param_list_free(&pb);
    return worst;
}

/* Prints one compared tensor's difference (stderr, which the test runner shows
   on failure) and returns the larger of it and `worst`. */
static double report(const char* what, double d, double worst)
{
    fprintf(stderr, "  %s: %.3e\n", what, d);
    return d > worst ? d : worst;
}

/* Parameters of a composite made of sub-modules, in the given order. */
typedef struct {
    Module** subs;
    int n;
} Composite;

static void composite_params(Module* self, ParamList* pl)
{
    Composite* c = (Composite*)self->state;
    for (int i = 0; i < c->n; ++i) c->subs[i]->parameters(c->subs[i], pl);
}

/* Returns the largest relative difference; out_ms[0..1]: fused / reference
   forward+backward time in ms (median of `reps`). */
double nn_blockcheck_ddpm(int B, int H, int W, int C, int G, int emb, int reps, float* out_ms)
{
    nn_context_init(&g, 11ull, (hipStream_t)0);
    const int n = B * H * W * C;
    const int slot = ctx_add_cond(&g, emb, B);
    float* e = dev_normal((size_t)B * emb, 1.0f);
    ctx_set_cond(&g, slot, e);
    Module* fused = conv_residual_create(&g, C, emb, H, W, B, G, slot);

    RefDDPM r;
    r.gn1 = spatial_groupnorm_create(C, G, H, W, B);
    r.conv1 = conv2d_create(&g, C, C, 3, 1, 1, H, W, B, 0, 1.0f);
    r.time_proj = linear_create(&g, emb, C);
    r.gn2 = spatial_groupnorm_create(C, G, H, W, B);
    r.conv2 = conv2d_create(&g, C, C, 3, 1, 1, H, W, B, 0, 1.0f);
    Module* subs[5] = {r.gn1, r.conv1, r.time_proj, r.gn2, r.conv2};
    Composite comp = {subs, 5};
    Module view = {"ref_ddpm", n / B, n / B, &comp, NULL, NULL, composite_params, NULL};
    float** bufs[] = {&r.h0, &r.h1, &r.h2, &r.h3, &r.h4, &r.gh4, &r.gh3, &r.gh2, &r.gh1, &r.gh0, &r.gxb};
    for (size_t i = 0; i < sizeof bufs / sizeof bufs[0]; ++i) *bufs[i] = nn_device_alloc((size_t)n);
    r.c = nn_device_alloc((size_t)B * C);
    r.gc = nn_device_alloc((size_t)B * C);
    r.gemb = nn_device_alloc((size_t)B * emb);

    /* non-trivial GroupNorm affine parameters and biases for both */
    {
        ParamList pl;
        param_list_init(&pl);
        fused->parameters(fused, &pl);
        for (int k = 0; k < pl.count; ++k)
            if (pl.items[k].size == C) nn_fill_normal(&g, pl.items[k].param, (size_t)C, k == 0 || k == 6 ? 1.0f : 0.0f, 0.1f);
        param_list_free(&pl);
    }
    copy_params(&view, fused);

    float* x = dev_normal((size_t)n, 1.0f);
    float* gout = dev_normal((size_t)n, 1.0f);
    float *y_f = nn_device_alloc((size_t)n), *y_r = nn_device_alloc((size_t)n);
    float *gx_f = nn_device_alloc((size_t)n), *gx_r = nn_device_alloc((size_t)n);
    float *ge_f = nn_device_alloc((size_t)B * emb), *ge_r = nn_device_alloc((size_t)B * emb);
    hipStream_t s = g.stream;
    hipEvent_t t0, t1;
    NN_HIP_CHECK(hipEventCreate(&t0));
    NN_HIP_CHECK(hipEventCreate(&t1));
    float best[2] = {1e30f, 1e30f};
    for (int rep = 0; rep < reps + 1; ++rep) {
        /* fused block */
        NN_HIP_CHECK(hipEventRecord(t0, s));
        fused->forward(fused, x, y_f, B, &g);
        ctx_zero_cond_grad(&g, B);
        fused->backward(fused, x, y_f, gout, gx_f, B, &g);
        NN_HIP_CHECK(hipEventRecord(t1, s));
        NN_HIP_CHECK(hipEventSynchronize(t1));
        float ms;
        NN_HIP_CHECK(hipEventElapsedTime(&ms, t0, t1));
        if (rep && ms < best[0]) best[0] = ms;
        NN_HIP_CHECK(hipMemcpy(ge_f, g.cond[slot].grad, (size_t)B * emb * sizeof(float), hipMemcpyDeviceToDevice));

        /* the reference's sequence (src/conv_residual.c:21-66) */
        NN_HIP_CHECK(hipEventRecord(t0, s));
        r.gn1->forward(r.gn1, x, r.h0, B, &g);
        launch_activation_forward(r.h1, r.h0, n, ACT_SILU, s);
        r.conv1->forward(r.conv1, r.h1, r.h2, B, &g);
        r.time_proj->forward(r.time_proj, e, r.c, B, &g);
        launch_spatial_add(r.h2, r.c, B, H, W, C, s);
        r.gn2->forward(r.gn2, r.h2, r.h3, B, &g);
        launch_activation_forward(r.h4, r.h3, n, ACT_SILU, s);
        r.conv2->forward(r.conv2, r.h4, y_r, B, &g);
        launch_weighted_sum(y_r, x, y_r, 1.0f, 1.0f, n, s);
        ctx_zero_cond_grad(&g, B);
        r.conv2->backward(r.conv2, r.h4, NULL, gout, r.gh4, B, &g);
        launch_activation_backward(r.gh3, r.gh4, r.h3, n, ACT_SILU, s);
        r.gn2->backward(r.gn2, r.h2, NULL, r.gh3, r.gh2, B, &g);
        launch_spatial_reduce_sum(r.gc, r.gh2, B, H * W, C, s);
        r.time_proj->backward(r.time_proj, e, r.c, r.gc, r.gemb, B, &g);
        launch_weighted_sum(g.cond[slot].grad, g.cond[slot].grad, r.gemb, 1.0f, 1.0f, B * emb, s);
        r.conv1->backward(r.conv1, r.h1, NULL, r.gh2, r.gh1, B, &g);
        launch_activation_backward(r.gh0, r.gh1, r.h0, n, ACT_SILU, s);
        r.gn1->backward(r.gn1, x, NULL, r.gh0, r.gxb, B, &g);
        launch_weighted_sum(gx_r, gout, r.gxb, 1.0f, 1.0f, n, s);
        NN_HIP_CHECK(hipEventRecord(t1, s));
        NN_HIP_CHECK(hipEventSynchronize(t1));
        NN_HIP_CHECK(hipEventElapsedTime(&ms, t0, t1));
        if (rep && ms < best[1]) best[1] = ms;
        NN_HIP_CHECK(hipMemcpy(ge_r, g.cond[slot].grad, (size_t)B * emb * sizeof(float), hipMemcpyDeviceToDevice));
    }
    /* Term scales of the embedding path's reduced outputs, from the gradient
       dh of GN2's input (r.gh2, [B, HW, C]): dc[b, c] sums dh over the pixels
       (scale s[b, c] = sqrt(sum dh^2)); conv1's and the projection's bias
       gradients sum dc over the samples, the projection's weight gradient
       sums e[b, i] dc[b, c], the embedding gradient sums dc[b, c] W[i, c].
       With one channel per group GN2 removes every per-(sample, channel)
       shift, so these gradients are exactly zero and both sides return
       rounding noise: only the term scale measures that. */
    double floors[10] = {0};
    double worst;
    {
        const int HWn = H * W;
        float* gh = to_host(r.gh2, (size_t)n);
        float* eh = to_host(e, (size_t)B * emb);
        ParamList pl;
        param_list_init(&pl);
        r.time_proj->parameters(r.time_proj, &pl);
        float* wh = to_host(pl.items[0].param, (size_t)emb * C);
        param_list_free(&pl);
        double* sc = (double*)calloc((size_t)B * C, sizeof(double));
        for (int b = 0; b < B; ++b)
            for (int p = 0; p < HWn; ++p)
                for (int c = 0; c < C; ++c) {
                    const double v = gh[((size_t)b * HWn + p) * C + c];
                    sc[(size_t)b * C + c] += v * v;
                }
        double fb = 0.0, fw = 0.0, fe = 0.0;
        for (int c = 0; c < C; ++c) {
            double t = 0.0;
            for (int b = 0; b < B; ++b) t += sc[(size_t)b * C + c];
            fb = fmax(fb, sqrt(t));
            for (int i = 0; i < emb; ++i) {
                double u = 0.0;
                for (int b = 0; b < B; ++b) u += (double)eh[(size_t)b * emb + i] * eh[(size_t)b * emb + i] * sc[(size_t)b * C + c];
                fw = fmax(fw, sqrt(u));
            }
        }
        for (int b = 0; b < B; ++b)
            for (int i = 0; i < emb; ++i) {
                double u = 0.0;
                for (int c = 0; c < C; ++c) u += sc[(size_t)b * C + c] * (double)wh[(size_t)i * C + c] * wh[(size_t)i * C + c];
                fe = fmax(fe, sqrt(u));
            }
        floors[3] = fb;  /* conv1 bias */
        floors[4] = fw;  /* projection weight */
        floors[5] = fb;  /* projection bias */
        free(sc);
        free(gh);
        free(eh);
        free(wh);
        fprintf(stderr, "DDPM block [%d, %d, %d, %d] G=%d emb=%d, relative differences:\n", B, H, W, C, G, emb);
        worst = report("out", rel_diff(y_f, y_r, (size_t)n), 0.0);
        worst = report("grad_in", rel_diff(gx_f, gx_r, (size_t)n), worst);
        worst = report("parameter gradients", grads_diff(fused, &view, floors, 10), worst);
        worst = report("embedding gradient", rel_diff_floor(ge_f, ge_r, (size_t)B * emb, fe), worst);
    }
    out_ms[0] = best[0];
    out_ms[1] = best[1];

    fused->free(fused);
    for (int i = 0; i < 5; ++i) subs[i]->free(subs[i]);
    for (size_t i = 0; i < sizeof bufs / sizeof bufs[0]; ++i) (void)hipFree(*bufs[i]);
    float* more[] = {r.c, r.gc, r.gemb, x, gout, y_f, y_r, gx_f, gx_r, ge_f, ge_r, e};
    for (size_t i = 0; i < sizeof more / sizeof more[0]; ++i) (void)hipFree(more[i]);
    (void)hipEventDestroy(t0);
    (void)hipEventDestroy(t1);
    nn_context_destroy(&g);
    return worst;
}

/* EDM block against its reference sequence (src/cond_conv_residual.c:22-62). */
double nn_blockcheck_edm(int B, int H, int W, int C, int emb, float t, int reps, float* out_ms)
{
    nn_context_init(&g, 13ull, (hipStream_t)0);
    const int n = B * H * W * C;
    const int slot = ctx_add_cond(&g, emb, B);
    float* e = dev_normal((size_t)B * emb, 1.0f);
    ctx_set_cond(&g, slot, e);
    Module* fused = cond_conv_residual_create(&g, C, emb, H, W, B, t, slot);
    Module* conv0 = conv2d_create(&g, C, C, 3, 1, 1, H, W, B, 1, 1.0f);
    Module* emb_lin = mp_linear_create(&g, emb, C, 0.0f);
    Module* conv1 = conv2d_create(&g, C, C, 3, 1, 1, H, W, B, 1, 1.0f);
    Module* subs[3] = {conv0, emb_lin, conv1};
    Composite comp = {subs, 3};
    Module view = {"ref_edm", n / B, n / B, &comp, NULL, NULL, composite_params, NULL};
    /* a non-zero embedding gain (index 3: conv0 W, gain, emb_lin W, gain) */
    {
        ParamList pl;
        param_list_init(&pl);
        fused->parameters(fused, &pl);
        const float gain = 0.7f;
        NN_HIP_CHECK(hipMemcpy(pl.items[3].param, &gain, sizeof gain, hipMemcpyHostToDevice));
        param_list_free(&pl);
    }
    copy_params(&view, fused);
    const float d0 = sqrtf((1.0f - t) * (1.0f - t) + t * t);
    const float wa = (1.0f - t) / d0, wb = t / d0;
    float *h0 = nn_device_alloc((size_t)n), *h1 = nn_device_alloc((size_t)n), *h2 = nn_device_alloc((size_t)n),
          *h3 = nn_device_alloc((size_t)n), *h4 = nn_device_alloc((size_t)n), *gh4 = nn_device_alloc((size_t)n),
          *gh3 = nn_device_alloc((size_t)n), *gh2 = nn_device_alloc((size_t)n), *gh1 = nn_device_alloc((size_t)n),
          *gh0 = nn_device_alloc((size_t)n), *gxb = nn_device_alloc((size_t)n);
    float *c = nn_device_alloc((size_t)B * C), *gc = nn_device_alloc((size_t)B * C),
          *gemb = nn_device_alloc((size_t)B * emb);
    float* x = dev_normal((size_t)n, 1.0f);
    float* gout = dev_normal((size_t)n, 1.0f);
    float *y_f = nn_device_alloc((size_t)n), *y_r = nn_device_alloc((size_t)n);
    float *gx_f = nn_device_alloc((size_t)n), *gx_r = nn_device_alloc((size_t)n);
    float *ge_f = nn_device_alloc((size_t)B * emb), *ge_r = nn_device_alloc((size_t)B * emb);
    hipStream_t s = g.stream;
    hipEvent_t t0, t1;
    NN_HIP_CHECK(hipEventCreate(&t0));
    NN_HIP_CHECK(hipEventCreate(&t1));
    float best[2] = {1e30f, 1e30f};
    for (int rep = 0; rep < reps + 1; ++rep) {
        NN_HIP_CHECK(hipEventRecord(t0, s));
        fused->forward(fused, x, y_f, B, &g);
        ctx_zero_cond_grad(&g, B);
        fused->backward(fused, x, y_f, gout, gx_f, B, &g);
        NN_HIP_CHECK(hipEventRecord(t1, s));
        NN_HIP_CHECK(hipEventSynchronize(t1));
        float ms;
        NN_HIP_CHECK(hipEventElapsedTime(&ms, t0, t1));
        if (rep && ms < best[0]) best[0] = ms;
        NN_HIP_CHECK(hipMemcpy(ge_f, g.cond[slot].grad, (size_t)B * emb * sizeof(float), hipMemcpyDeviceToDevice));

        NN_HIP_CHECK(hipEventRecord(t0, s));
        launch_activation_forward(h0, x, n, ACT_MP_SILU, s);
        conv0->forward(conv0, h0, h1, B, &g);
        emb_lin->forward(emb_lin, e, c, B, &g);
        launch_spatial_modulate(h2, h1, c, B, H, W, C, s);
        launch_activation_forward(h3, h2, n, ACT_MP_SILU, s);
        conv1->forward(conv1, h3, h4, B, &g);
        launch_weighted_sum(y_r, x, h4, wa, wb, n, s);
        ctx_zero_cond_grad(&g, B);
        launch_weighted_sum(gh4, gout, gout, wb, 0.0f, n, s);
        conv1->backward(conv1, h3, h4, gh4, gh3, B, &g);
        launch_activation_backward(gh2, gh3, h2, n, ACT_MP_SILU, s);
        launch_spatial_modulate_backward(gh1, gc, gh2, h1, c, B, H, W, C, s);
        conv0->backward(conv0, h0, h1, gh1, gh0, B, &g);
        launch_activation_backward(gxb, gh0, x, n, ACT_MP_SILU, s);
        emb_lin->backward(emb_lin, e, c, gc, gemb, B, &g);
        launch_weighted_sum(g.cond[slot].grad, g.cond[slot].grad, gemb, 1.0f, 1.0f, B * emb, s);
        launch_weighted_sum(gx_r, gout, gxb, wa, 1.0f, n, s);
        NN_HIP_CHECK(hipEventRecord(t1, s));
        NN_HIP_CHECK(hipEventSynchronize(t1));
        NN_HIP_CHECK(hipEventElapsedTime(&ms, t0, t1));
        if (rep && ms < best[1]) best[1] = ms;
        NN_HIP_CHECK(hipMemcpy(ge_r, g.cond[slot].grad, (size_t)B * emb * sizeof(float), hipMemcpyDeviceToDevice));
    }
    fprintf(stderr, "EDM block [%d, %d, %d, %d] emb=%d, relative differences:\n", B, H, W, C, emb);
    double worst = report("out", rel_diff(y_f, y_r, (size_t)n), 0.0);
    worst = report("grad_in", rel_diff(gx_f, gx_r, (size_t)n), worst);
    worst = report("parameter gradients", grads_diff(fused, &view, NULL, 0), worst);
    worst = report("embedding gradient", rel_diff(ge_f, ge_r, (size_t)B * emb), worst);
    out_ms[0] = best[0];
    out_ms[1] = best[1];
    fused->free(fused);
    for (int i = 0; i < 3; ++i) subs[i]->free(subs[i]);
    float* all[] = {h0, h1, h2, h3, h4, gh4, gh3, gh2, gh1, gh0, gxb, c, gc, gemb, x, gout, y_f, y_r, gx_f, gx_r,
        ge_f, ge_r, e};
    for (size_t i = 0; i < sizeof all / sizeof all[0]; ++i) (void)hipFree(all[i]);
    (void)hipEventDestroy(t0);
    (void)hipEventDestroy(t1);
    nn_context_destroy(&g);
    return worst;
}

/* conv2d module forward and backward on its two paths (implicit GEMMs vs
   im2col + rocBLAS GEMMs, selected with NNHIP_CONV_PATH): returns the largest
   relative difference over y, grad_in and the parameter gradients; out_ms[0..3]
   = implicit / gemm forward, implicit / gemm backward time in ms (best of
   `reps`). */
double nn_convcheck(int B, int H, int W, int Cin, int Cout, int K, int stride, int pad, int mp, int reps,
    float* out_ms)
{
    nn_context_init(&g, 17ull, (hipStream_t)0);
    /* created with the reference's sequence forced, so that it has the im2col
       buffer both paths below need */
    setenv("NNHIP_CONV_PATH", "gemm", 1);
    Module* conv = conv2d_create(&g, Cin, Cout, K, stride, pad, H, W, B, mp, 1.0f);
    if (!mp) {
        ParamList pl;
        param_list_init(&pl);
        conv->parameters(conv, &pl);
        nn_fill_normal(&g, pl.items[1].param, (size_t)Cout, 0.0f, 0.1f);  /* non-zero bias */
        param_list_free(&pl);
    }
    const size_t n_in = (size_t)B * H * W * Cin, n_out = (size_t)B * conv->out_dim;
    float* x = dev_normal(n_in, 1.0f);
    float *y_i = nn_device_alloc(n_out), *y_g = nn_device_alloc(n_out);
    float* gy = dev_normal(n_out, 1.0f);
    float *gx_i = nn_device_alloc(n_in), *gx_g = nn_device_alloc(n_in);
    ParamList pl;
    param_list_init(&pl);
    conv->parameters(conv, &pl);
    float* gsave[2];
    for (int k = 0; k < 2; ++k) gsave[k] = nn_device_alloc((size_t)pl.items[k].size);
    hipEvent_t t0, t1, t2;
    NN_HIP_CHECK(hipEventCreate(&t0));
    NN_HIP_CHECK(hipEventCreate(&t1));
    NN_HIP_CHECK(hipEventCreate(&t2));
    float best[4] = {1e30f, 1e30f, 1e30f, 1e30f};
    double worst = 0.0;
    for (int rep = 0; rep < reps + 1; ++rep) {
        for (int path = 0; path < 2; ++path) {
            setenv("NNHIP_CONV_PATH", path ? "gemm" : "implicit", 1);
            NN_HIP_CHECK(hipEventRecord(t0, g.stream));
            conv->forward(conv, x, path ? y_g : y_i, B, &g);
            NN_HIP_CHECK(hipEventRecord(t1, g.stream));
            conv->backward(conv, x, path ? y_g : y_i, gy, path ? gx_g : gx_i, B, &g);
            NN_HIP_CHECK(hipEventRecord(t2, g.stream));
            NN_HIP_CHECK(hipEventSynchronize(t2));
            float ms;
            NN_HIP_CHECK(hipEventElapsedTime(&ms, t0, t1));
            if (rep && ms < best[path]) best[path] = ms;
            NN_HIP_CHECK(hipEventElapsedTime(&ms, t1, t2));
            if (rep && ms < best[2 + path]) best[2 + path] = ms;
            if (path == 0) {
                for (int k = 0; k < 2; ++k)
                    NN_HIP_CHECK(hipMemcpy(gsave[k], pl.items[k].grad, (size_t)pl.items[k].size * sizeof(float),
                        hipMemcpyDeviceToDevice));
            } else if (rep == reps) {
                for (int k = 0; k < 2; ++k) {
                    const double d = rel_diff(gsave[k], pl.items[k].grad, (size_t)pl.items[k].size);
                    if (d > worst) worst = d;
                }
            }
        }
    }
    unsetenv("NNHIP_CONV_PATH");
    double d = rel_diff(y_i, y_g, n_out);
    if (d > worst) worst = d;
    d = rel_diff(gx_i, gx_g, n_in);
    if (d > worst) worst = d;
    for (int k = 0; k < 4; ++k) out_ms[k] = best[k];
    param_list_free(&pl);
    conv->free(conv);
    (void)hipFree(x);
    (void)hipFree(y_i);
    (void)hipFree(y_g);
    (void)hipFree(gy);
    (void)hipFree(gx_i);
    (void)hipFree(gx_g);
    for (int k = 0; k < 2; ++k) (void)hipFree(gsave[k]);
    (void)hipEventDestroy(t2);
    (void)hipEventDestroy(t0);
    (void)hipEventDestroy(t1);
    nn_context_destroy(&g);
    return d;
}

/* A block's forward + backward captured into a HIP graph on a created stream
   (nnhip_graph_capture_begin/end) and replayed `reps` times.  Every replay
   must reproduce the eager output, input gradient and embedding gradient bit
   for bit (returned: number of mismatching replays, -1 if the capture
   failed).  out_ms[0]: eager forward+backward, out_ms[1]: one graph replay
   (best of reps, each timed alone). */
static int graph_replays(Context* cg, Module* blk, int slot, int B, int n, int emb, float* x, float* gout, int reps,
    float* out_ms)
{
    hipStream_t s = cg->stream;
    float *y = nn_device_alloc((size_t)n), *gx = nn_device_alloc((size_t)n);
    float *y0 = nn_device_alloc((size_t)n), *gx0 = nn_device_alloc((size_t)n);
    float* ge0 = nn_device_alloc((size_t)B * emb);
    hipEvent_t t0, t1;
    NN_HIP_CHECK(hipEventCreate(&t0));
    NN_HIP_CHECK(hipEventCreate(&t1));
    float ms, best_e = 1e30f, best_g = 1e30f;
    /* eager runs (the first also sizes every cached scratch block) */
    for (int rep = 0; rep < 3; ++rep) {
        NN_HIP_CHECK(hipEventRecord(t0, s));
        blk->forward(blk, x, y, B, cg);
        ctx_zero_cond_grad(cg, B);
        blk->backward(blk, x, y, gout, gx, B, cg);
        NN_HIP_CHECK(hipEventRecord(t1, s));
        NN_HIP_CHECK(hipEventSynchronize(t1));
        NN_HIP_CHECK(hipEventElapsedTime(&ms, t0, t1));
        if (rep && ms < best_e) best_e = ms;
    }
    NN_HIP_CHECK(hipMemcpy(y0, y, (size_t)n * sizeof(float), hipMemcpyDeviceToDevice));
    NN_HIP_CHECK(hipMemcpy(gx0, gx, (size_t)n * sizeof(float), hipMemcpyDeviceToDevice));
    NN_HIP_CHECK(hipMemcpy(ge0, cg->cond[slot].grad, (size_t)B * emb * sizeof(float), hipMemcpyDeviceToDevice));

    int bad = -1;
    hipGraphExec_t graph = NULL;
    if (nnhip_graph_capture_begin(s) == 0) {
        blk->forward(blk, x, y, B, cg);
        ctx_zero_cond_grad(cg, B);
        blk->backward(blk, x, y, gout, gx, B, cg);
        graph = nnhip_graph_capture_end(s);
    }
    if (graph) {
        bad = 0;
        for (int rep = 0; rep < reps; ++rep) {
            nnhip_fill_f32(y, 0.0f, (size_t)n, s);
            nnhip_fill_f32(gx, 0.0f, (size_t)n, s);
            NN_HIP_CHECK(hipStreamSynchronize(s));
            NN_HIP_CHECK(hipEventRecord(t0, s));
            NN_HIP_CHECK((hipError_t)nnhip_graph_launch(graph, s));
            NN_HIP_CHECK(hipEventRecord(t1, s));
            NN_HIP_CHECK(hipEventSynchronize(t1));
            NN_HIP_CHECK(hipEventElapsedTime(&ms, t0, t1));
            if (ms < best_g) best_g = ms;
            if (rel_diff(y, y0, (size_t)n) != 0.0 || rel_diff(gx, gx0, (size_t)n) != 0.0 ||
                rel_diff(cg->cond[slot].grad, ge0, (size_t)B * emb) != 0.0)
                ++bad;
            /* eager work on the same buffers and workspaces between replays */
            blk->forward(blk, x, y, B, cg);
            NN_HIP_CHECK(hipStreamSynchronize(s));
        }
        (void)nnhip_graph_destroy(graph);
    }
    out_ms[0] = best_e;
    out_ms[1] = best_g;
    float* more[] = {y, gx, y0, gx0, ge0};
    for (size_t i = 0; i < sizeof more / sizeof more[0]; ++i) (void)hipFree(more[i]);
    (void)hipEventDestroy(t0);
    (void)hipEventDestroy(t1);
    return bad;
}

/* The fused DDPM block (src/conv_residual.c) as a graph; see graph_replays. */
int nn_blockcheck_ddpm_graph(int B, int H, int W, int C, int G, int emb, int reps, float* out_ms)
{
    hipStream_t s = nnhip_stream_create();
    Context cg;
    nn_context_init(&cg, 13ull, s);
    const int n = B * H * W * C;
    const int slot = ctx_add_cond(&cg, emb, B);
    float* e = dev_normal((size_t)B * emb, 1.0f);
    ctx_set_cond(&cg, slot, e);
    Module* blk = conv_residual_create(&cg, C, emb, H, W, B, G, slot);
    float* x = dev_normal((size_t)n, 1.0f);
    float* gout = dev_normal((size_t)n, 1.0f);
    const int bad = graph_replays(&cg, blk, slot, B, n, emb, x, gout, reps, out_ms);
    blk->free(blk);
    (void)hipFree(x);
    (void)hipFree(gout);
    (void)hipFree(e);
    nn_context_destroy(&cg);
    (void)nnhip_stream_destroy(s);
    return bad;
}

/* The fused EDM block (src/cond_conv_residual.c) as a graph, with a non-zero
   embedding gain so that the conditioning path carries gradient. */
int nn_blockcheck_edm_graph(int B, int H, int W, int C, int emb, float t, int reps, float* out_ms)
{
    hipStream_t s = nnhip_stream_create();
    Context cg;
    nn_context_init(&cg, 17ull, s);
    const int n = B * H * W * C;
    const int slot = ctx_add_cond(&cg, emb, B);
    float* e = dev_normal((size_t)B * emb, 1.0f);
    ctx_set_cond(&cg, slot, e);
    Module* blk = cond_conv_residual_create(&cg, C, emb, H, W, B, t, slot);
    {
        ParamList pl;
        param_list_init(&pl);
        blk->parameters(blk, &pl);
        if (pl.count > 3 && pl.items[3].size == 1) nnhip_fill_f32(pl.items[3].param, 0.7f, 1, s);
        param_list_free(&pl);
    }
    float* x = dev_normal((size_t)n, 1.0f);
    float* gout = dev_normal((size_t)n, 1.0f);
    const int bad = graph_replays(&cg, blk, slot, B, n, emb, x, gout, reps, out_ms);
    blk->free(blk);
    (void)hipFree(x);
    (void)hipFree(gout);
    (void)hipFree(e);
    nn_context_destroy(&cg);
    (void)nnhip_stream_destroy(s);
    return bad;
}
