/* gradcheck.c -- finite-difference check of the host modules' backward passes,
 * the method of the reference's only test (reference tests/gradcheck.c:1-321):
 * L = <forward(in), g> for a fixed random cotangent g; central differences
 * with EPS = 1e-3 on up to 20 sampled elements of the input and of every
 * parameter tensor; pass iff |num - ana| <= ATOL + rtol*(|num| + |ana|) with
 * ATOL = 1e-2 and rtol = 2e-2 (reference gradcheck.c:15-21, 51-56, 290-306).
 * Magnitude-preserving layers normalise their weights in place, so a warm-up
 * forward projects them first and every numeric forward restores the snapshot.
 *
 * Built as tests/_build/libgradcheck.so; nn_gradcheck_run() returns the number
 * of failing modules (0 = all pass).  Needs a GPU.
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "nn_modules.h"

#define K_SAMPLES 20
#define GC_EPS 1.0e-3f
#define GC_ATOL 1.0e-2

static Context g_ctx;
static int g_verbose = 1;

static void d2h(float* h, const float* d, int n)
{
    NN_HIP_CHECK(hipMemcpy(h, d, (size_t)n * sizeof(float), hipMemcpyDeviceToHost));
}

static void h2d(float* d, const float* h, int n)
{
    NN_HIP_CHECK(hipMemcpy(d, h, (size_t)n * sizeof(float), hipMemcpyHostToDevice));
}

static double dot_host(const float* a, const float* b, int n)
{
    double s = 0.0;
    for (int i = 0; i < n; ++i) s += (double)a[i] * (double)b[i];
    return s;
}

static double viol_ratio(double num, double ana, double rtol)
{
    return fabs(num - ana) / (GC_ATOL + rtol * (fabs(num) + fabs(ana)));
}

static int pick_indices(int size, int* idx)
{
    if (size <= K_SAMPLES) {
        for (int i = 0; i < size; ++i) idx[i] = i;
        return size;
    }
    for (int i = 0; i < K_SAMPLES; ++i) idx[i] = (int)(nn_rng_uniform(&g_ctx) * size) % size;
    return K_SAMPLES;
}

static double loss_at(Module* m, const float* d_in, float* d_out, float* h_out, const float* h_g,
    int batch, int n_out)
{
    m->forward(m, d_in, d_out, batch, &g_ctx);
    d2h(h_out, d_out, n_out);
    return dot_host(h_out, h_g, n_out);
}

static void restore(const ParamList* pl, float** snap)
{
    for (int k = 0; k < pl->count; ++k) h2d(pl->items[k].param, snap[k], pl->items[k].size);
}

/* cond_slot >= 0: the module also reads ctx->cond[cond_slot].fwd and adds its
   gradient into ctx->cond[cond_slot].grad (the diffusion blocks); that input
   is checked like the module input. */
static int check_module_cond(const char* tag, Module* m, int batch, double rtol, int cond_slot)
{
    int n_in = batch * m->in_dim, n_out = batch * m->out_dim;
    float* d_in = nn_device_alloc((size_t)n_in);
    float* d_out = nn_device_alloc((size_t)n_out);
    float* d_gout = nn_device_alloc((size_t)n_out);
    float* d_gin = nn_device_alloc((size_t)n_in);
    float* h_in = (float*)malloc((size_t)n_in * sizeof(float));
    float* h_out = (float*)malloc((size_t)n_out * sizeof(float));
    float* h_g = (float*)malloc((size_t)n_out * sizeof(float));
    float* h_gin = (float*)malloc((size_t)n_in * sizeof(float));
    for (int i = 0; i < n_in; ++i) h_in[i] = (float)nn_rng_normal(&g_ctx);
    for (int i = 0; i < n_out; ++i) h_g[i] = (float)nn_rng_normal(&g_ctx);
    h2d(d_in, h_in, n_in);
    h2d(d_gout, h_g, n_out);

    ParamList pl;
    param_list_init(&pl);
    if (m->parameters) m->parameters(m, &pl);

    m->forward(m, d_in, d_out, batch, &g_ctx); /* warm-up: project MP weights */
    NN_HIP_CHECK(hipDeviceSynchronize());
    float** snap = (float**)calloc((size_t)(pl.count > 0 ? pl.count : 1), sizeof(float*));
    for (int k = 0; k < pl.count; ++k) {
        snap[k] = (float*)malloc((size_t)pl.items[k].size * sizeof(float));
        d2h(snap[k], pl.items[k].param, pl.items[k].size);
        NN_HIP_CHECK(hipMemset(pl.items[k].grad, 0, (size_t)pl.items[k].size * sizeof(float)));
    }
    int n_cond = cond_slot >= 0 ? batch * g_ctx.cond[cond_slot].dim : 0;
    float* h_cond = (float*)malloc((size_t)(n_cond ? n_cond : 1) * sizeof(float));
    float* h_gcond = (float*)malloc((size_t)(n_cond ? n_cond : 1) * sizeof(float));
    if (n_cond) d2h(h_cond, g_ctx.cond[cond_slot].fwd, n_cond);
    m->forward(m, d_in, d_out, batch, &g_ctx);
    ctx_zero_cond_grad(&g_ctx, batch);
    m->backward(m, d_in, d_out, d_gout, d_gin, batch, &g_ctx);
    NN_HIP_CHECK(hipDeviceSynchronize());
    d2h(h_gin, d_gin, n_in);
    if (n_cond) d2h(h_gcond, g_ctx.cond[cond_slot].grad, n_cond);
    float** ana = (float**)calloc((size_t)(pl.count > 0 ? pl.count : 1), sizeof(float*));
    for (int k = 0; k < pl.count; ++k) {
        ana[k] = (float*)malloc((size_t)pl.items[k].size * sizeof(float));
        d2h(ana[k], pl.items[k].grad, pl.items[k].size);
    }

    double worst = 0.0, worst_num = 0.0, worst_ana = 0.0;
    const char* where = "input";
    int worst_k = -1, worst_j = -1;
    int idx[K_SAMPLES];

    int n = pick_indices(n_in, idx);
    for (int s = 0; s < n; ++s) {
        int j = idx[s];
        float save = h_in[j];
        restore(&pl, snap);
        h_in[j] = save + GC_EPS;
        h2d(d_in, h_in, n_in);
        double lp = loss_at(m, d_in, d_out, h_out, h_g, batch, n_out);
        restore(&pl, snap);
        h_in[j] = save - GC_EPS;
        h2d(d_in, h_in, n_in);
        double lm = loss_at(m, d_in, d_out, h_out, h_g, batch, n_out);
        h_in[j] = save;
        double num = (lp - lm) / (2.0 * GC_EPS);
        double e = viol_ratio(num, h_gin[j], rtol);
        if (e > worst) {
            worst = e;
            where = "input";
            worst_k = -1;
            worst_j = j;
            worst_num = num;
            worst_ana = h_gin[j];
        }
    }
    h2d(d_in, h_in, n_in);

    n = pick_indices(n_cond, idx);
    for (int s = 0; s < n; ++s) {
        int j = idx[s];
        float* d_cond = (float*)g_ctx.cond[cond_slot].fwd;
        float save = h_cond[j];
        restore(&pl, snap);
        h_cond[j] = save + GC_EPS;
        h2d(d_cond, h_cond, n_cond);
        double lp = loss_at(m, d_in, d_out, h_out, h_g, batch, n_out);
        restore(&pl, snap);
        h_cond[j] = save - GC_EPS;
        h2d(d_cond, h_cond, n_cond);
        double lm = loss_at(m, d_in, d_out, h_out, h_g, batch, n_out);
        h_cond[j] = save;
        h2d(d_cond, h_cond, n_cond);
        double num = (lp - lm) / (2.0 * GC_EPS);
        double e = viol_ratio(num, h_gcond[j], rtol);
        if (e > worst) {
            worst = e;
            where = "cond";
            worst_k = -1;
            worst_j = j;
            worst_num = num;
            worst_ana = h_gcond[j];
        }
    }

    for (int k = 0; k < pl.count; ++k) {
        int sz = pl.items[k].size;
        n = pick_indices(sz, idx);
        for (int s = 0; s < n; ++s) {
            int j = idx[s];
            float base = snap[k][j];
            restore(&pl, snap);
            float vp = base + GC_EPS;
            h2d(pl.items[k].param + j, &vp, 1);
            double lp = loss_at(m, d_in, d_out, h_out, h_g, batch, n_out);
            restore(&pl, snap);
            float vm = base - GC_EPS;
            h2d(pl.items[k].param + j, &vm, 1);
            double lm = loss_at(m, d_in, d_out, h_out, h_g, batch, n_out);
            double num = (lp - lm) / (2.0 * GC_EPS);
            double e = viol_ratio(num, ana[k][j], rtol);
            if (e > worst) {
                worst = e;
                where = "param";
                worst_k = k;
                worst_j = j;
                worst_num = num;
                worst_ana = ana[k][j];
            }
        }
    }
    restore(&pl, snap);

    int pass = worst <= 1.0;
    if (g_verbose || !pass) {
        printf("  [%s] %-24s worst_ratio=%.3f (%s", pass ? "PASS" : "FAIL", tag, worst, where);
        if (worst_k >= 0) printf(" #%d", worst_k);
        printf(")\n");
        if (!pass) printf("         at idx %d: numeric=%+.6e analytic=%+.6e\n", worst_j, worst_num, worst_ana);
        fflush(stdout);
    }
    for (int k = 0; k < pl.count; ++k) {
        free(snap[k]);
        free(ana[k]);
    }
    free(snap);
    free(ana);
    param_list_free(&pl);
    m->free(m);
    free(h_in);
    free(h_out);
    free(h_g);
    free(h_gin);
    free(h_cond);
    free(h_gcond);
    (void)hipFree(d_in);
    (void)hipFree(d_out);
    (void)hipFree(d_gout);
    (void)hipFree(d_gin);
    return pass ? 0 : 1;
}

static int check_module(const char* tag, Module* m, int batch, double rtol)
{
    return check_module_cond(tag, m, batch, rtol, -1);
}

/* Set the k-th single-element parameter of m (e.g. an mp gain) to v. */
static Module* with_scalar_param(Module* m, int k, float v)
{
    ParamList pl;
    param_list_init(&pl);
    m->parameters(m, &pl);
    for (int i = 0, seen = 0; i < pl.count; ++i)
        if (pl.items[i].size == 1 && seen++ == k) h2d(pl.items[i].param, &v, 1);
    param_list_free(&pl);
    return m;
}

/* ------------------------------------------------------------------------
 * Directional check for the diffusion blocks at sizes where the per-element
 * check above drowns in fp32 noise (a sampled element moves L = <out, g> by
 * eps * grad, against rounding noise of sqrt(n) * 6e-8 over n outputs).  Per
 * group of inputs (the block input, the embedding, each parameter tensor) a
 * random direction d over the whole group: the analytic directional
 * derivative <grad, d> (double) against (L(+eps d) - L(-eps d)) / (2 eps)
 * with L in double.  Both sides sum millions of terms, so the rounding noise
 * averages out: relative error ~1e-4 at eps = 1e-2, where a wrong or missing
 * gradient term is off by far more.  Parameter directions are scaled by the
 * tensor's RMS (gamma ~ 1, weights ~ 1/sqrt(fan-in); 1 for the zero-initialised
 * biases and betas, whose steps would otherwise vanish).  Returns the worst
 * |num - ana| / max(|ana|, sqrt(sum (grad_i d_i)^2)) over the groups.
 * kind 0: conv_residual (DDPM; groups = GroupNorm groups); kind 1:
 * cond_conv_residual (EDM, t = 0.3, emb_lin gain set to 0.7).  ana_scale
 * multiplies the analytic gradients (1 for the check; the test's sensitivity
 * case passes 1.005, a 0.5% gradient error, which must fail the bar).
 * ------------------------------------------------------------------------ */
#define DC_EPS 1.0e-2

static double dir_loss(Module* m, const float* d_in, float* d_out, float* h_out, const float* h_g, int batch,
    int n_out)
{
    return loss_at(m, d_in, d_out, h_out, h_g, batch, n_out);
}

static double rms_host(const float* a, int n)
{
    double s = 0.0;
    for (int i = 0; i < n; ++i) s += (double)a[i] * a[i];
    return n ? sqrt(s / n) : 0.0;
}

/* One group: base values h_base (n floats, at device address d_dst), analytic
   gradient h_ana, direction h_dir.  Restores the parameters and the group. */
static double dir_group(const char* tag, Module* m, const ParamList* pl, float** snap, float* d_dst,
    const float* h_base, const float* h_ana, const float* h_dir, int n, const float* d_in, float* d_out,
    float* h_out, const float* h_g, int batch, int n_out, double ana_scale, int verbose)
{
    float* h_p = (float*)malloc((size_t)n * sizeof(float));
    double ana = 0.0, floor2 = 0.0;
    for (int i = 0; i < n; ++i) {
        const double t = ana_scale * h_ana[i] * h_dir[i];
        ana += t;
        floor2 += t * t;
    }
    double l[2];
    for (int sgn = 0; sgn < 2; ++sgn) {
        const float e = (float)(sgn ? -DC_EPS : DC_EPS);
        for (int i = 0; i < n; ++i) h_p[i] = h_base[i] + e * h_dir[i];
        restore(pl, snap);
        h2d(d_dst, h_p, n);
        l[sgn] = dir_loss(m, d_in, d_out, h_out, h_g, batch, n_out);
    }
    restore(pl, snap);
    h2d(d_dst, h_base, n);
    const double num = (l[0] - l[1]) / (2.0 * DC_EPS);
    const double scale = fmax(fabs(ana), sqrt(floor2));
    const double rel = fabs(num - ana) / (scale > 0.0 ? scale : 1.0);
    if (verbose) {
        printf("    %-16s n=%-9d analytic %+.6e numeric %+.6e rel %.2e\n", tag, n, ana, num, rel);
        fflush(stdout);
    }
    free(h_p);
    return rel;
}

double nn_dircheck_block(int kind, int batch, int H, int W, int C, int groups, int emb, double ana_scale,
    int verbose)
{
    nn_context_init(&g_ctx, 7ull, (hipStream_t)0);
    int slot = ctx_add_cond(&g_ctx, emb, batch);
    float* d_emb = nn_device_alloc((size_t)batch * emb);
    nn_fill_normal(&g_ctx, d_emb, (size_t)batch * emb, 0.0f, 1.0f);
    ctx_set_cond(&g_ctx, slot, d_emb);
    Module* m = kind == 0 ? conv_residual_create(&g_ctx, C, emb, H, W, batch, groups, slot)
                          : with_scalar_param(cond_conv_residual_create(&g_ctx, C, emb, H, W, batch, 0.3f, slot), 1,
                                0.7f);
    const int n_in = batch * m->in_dim, n_out = batch * m->out_dim, n_cond = batch * emb;
    float* d_in = nn_device_alloc((size_t)n_in);
    float* d_out = nn_device_alloc((size_t)n_out);
    float* d_gout = nn_device_alloc((size_t)n_out);
    float* d_gin = nn_device_alloc((size_t)n_in);
    float* h_in = (float*)malloc((size_t)n_in * sizeof(float));
    float* h_out = (float*)malloc((size_t)n_out * sizeof(float));
    float* h_g = (float*)malloc((size_t)n_out * sizeof(float));
    float* h_gin = (float*)malloc((size_t)n_in * sizeof(float));
    float* h_dir = (float*)malloc((size_t)n_in * sizeof(float));
    float* h_cond = (float*)malloc((size_t)n_cond * sizeof(float));
    float* h_gcond = (float*)malloc((size_t)n_cond * sizeof(float));
    for (int i = 0; i < n_in; ++i) h_in[i] = (float)nn_rng_normal(&g_ctx);
    for (int i = 0; i < n_out; ++i) h_g[i] = (float)nn_rng_normal(&g_ctx);
    h2d(d_in, h_in, n_in);
    h2d(d_gout, h_g, n_out);
    d2h(h_cond, d_emb, n_cond);

    ParamList pl;
    param_list_init(&pl);
    m->parameters(m, &pl);
    m->forward(m, d_in, d_out, batch, &g_ctx); /* warm-up: project MP weights */
    NN_HIP_CHECK(hipDeviceSynchronize());
    float** snap = (float**)calloc((size_t)pl.count, sizeof(float*));
    float** ana = (float**)calloc((size_t)pl.count, sizeof(float*));
    int n_max = n_in > n_cond ? n_in : n_cond;
    for (int k = 0; k < pl.count; ++k) {
        snap[k] = (float*)malloc((size_t)pl.items[k].size * sizeof(float));
        ana[k] = (float*)malloc((size_t)pl.items[k].size * sizeof(float));
        d2h(snap[k], pl.items[k].param, pl.items[k].size);
        NN_HIP_CHECK(hipMemset(pl.items[k].grad, 0, (size_t)pl.items[k].size * sizeof(float)));
        if (pl.items[k].size > n_max) n_max = pl.items[k].size;
    }
    m->forward(m, d_in, d_out, batch, &g_ctx);
    ctx_zero_cond_grad(&g_ctx, batch);
    m->backward(m, d_in, d_out, d_gout, d_gin, batch, &g_ctx);
    NN_HIP_CHECK(hipDeviceSynchronize());
    d2h(h_gin, d_gin, n_in);
    d2h(h_gcond, g_ctx.cond[slot].grad, n_cond);
    for (int k = 0; k < pl.count; ++k) d2h(ana[k], pl.items[k].grad, pl.items[k].size);
    free(h_dir);
    h_dir = (float*)malloc((size_t)n_max * sizeof(float));

    double worst = 0.0;
    for (int i = 0; i < n_in; ++i) h_dir[i] = (float)nn_rng_normal(&g_ctx);
    worst = fmax(worst, dir_group("input", m, &pl, snap, d_in, h_in, h_gin, h_dir, n_in, d_in, d_out, h_out, h_g,
                            batch, n_out, ana_scale, verbose));
    for (int i = 0; i < n_cond; ++i) h_dir[i] = (float)nn_rng_normal(&g_ctx);
    worst = fmax(worst, dir_group("embedding", m, &pl, snap, d_emb, h_cond, h_gcond, h_dir, n_cond, d_in, d_out,
                            h_out, h_g, batch, n_out, ana_scale, verbose));
    for (int k = 0; k < pl.count; ++k) {
        const int n = pl.items[k].size;
        double r = rms_host(snap[k], n);
        if (r < 1e-2) r = 1.0; /* zero-initialised tensors (biases, beta): unit directions */
        for (int i = 0; i < n; ++i) h_dir[i] = (float)(r * nn_rng_normal(&g_ctx));
        char tag[32];
        snprintf(tag, sizeof tag, "param %d", k);
        worst = fmax(worst, dir_group(tag, m, &pl, snap, pl.items[k].param, snap[k], ana[k], h_dir, n, d_in, d_out,
                                h_out, h_g, batch, n_out, ana_scale, verbose));
    }
    if (verbose) {
        printf("  %s block [%d,%d,%d,%d]: worst directional rel error %.2e\n", kind == 0 ? "DDPM" : "EDM", batch, H,
            W, C, worst);
        fflush(stdout);
    }
    for (int k = 0; k < pl.count; ++k) {
        free(snap[k]);
        free(ana[k]);
    }
    free(snap);
    free(ana);
    param_list_free(&pl);
    m->free(m);
    ctx_free_cond(&g_ctx);
    free(h_in);
    free(h_out);
    free(h_g);
    free(h_gin);
    free(h_dir);
    free(h_cond);
    free(h_gcond);
    (void)hipFree(d_in);
    (void)hipFree(d_out);
    (void)hipFree(d_gout);
    (void)hipFree(d_gin);
    (void)hipFree(d_emb);
    nn_context_destroy(&g_ctx);
    return worst;
}

/* Returns the number of failing modules.  Module list: the reference's
 * gradcheck configs on the fused-kernel path (gradcheck.c:290-306), plus the
 * fused GroupNorm+activation module and GroupNorm shapes that take the
 * register-resident kernels. */
int nn_gradcheck_run(int verbose)
{
    g_verbose = verbose;
    nn_context_init(&g_ctx, 42ull, (hipStream_t)0);
    const int B = 2;
    int fails = 0;
    fails += check_module("mp_linear", mp_linear_create(&g_ctx, 12, 8, 1.0f), B, 2e-2);
    fails += check_module("act_silu", activation_create(8, ACT_SILU), B, 2e-2);
    fails += check_module("act_gelu", activation_create(8, ACT_GELU), B, 2e-2);
    fails += check_module("act_tanh", activation_create(8, ACT_TANH), B, 2e-2);
    fails += check_module("act_mp_silu", activation_create(8, ACT_MP_SILU), B, 2e-2);
    fails += check_module("act_relu", activation_create(8, ACT_RELU), B, 2e-2);
    fails += check_module("layernorm", layernorm_create(16, B), B, 2e-2);
    fails += check_module("layernorm_c256", layernorm_create(256, B), B, 2e-2);
    fails += check_module("groupnorm", spatial_groupnorm_create(8, 4, 6, 6, B), B, 2e-2);
    fails += check_module("groupnorm_c32_g8", spatial_groupnorm_create(32, 8, 8, 8, B), B, 2e-2);
    fails += check_module("groupnorm_silu", spatial_groupnorm_act_create(8, 4, 6, 6, B, ACT_SILU), B, 2e-2);
    fails += check_module("groupnorm_silu_c32", spatial_groupnorm_act_create(32, 8, 8, 8, B, ACT_SILU), B, 2e-2);
    fails += check_module("conv3x3", conv2d_create(&g_ctx, 3, 4, 3, 1, 1, 6, 6, B, 0, 1.0f), B, 2e-2);
    fails += check_module("conv3x3_mp", conv2d_create(&g_ctx, 3, 4, 3, 1, 1, 6, 6, B, 1, 1.0f), B, 2e-2);
    fails += check_module("conv1x1_mp", conv2d_create(&g_ctx, 4, 6, 1, 1, 0, 5, 5, B, 1, 1.0f), B, 2e-2);
    fails += check_module("conv3x3_s2", conv2d_create(&g_ctx, 4, 4, 3, 2, 1, 7, 7, B, 0, 1.0f), B, 2e-2);
    fails += check_module("linear", linear_create(&g_ctx, 12, 8), B, 2e-2);
    /* channel counts that take the implicit-GEMM forward, weight gradient and
       (C_in % 128 == 0, stride 1) input gradient; forced, since at these few
       pixels the module's cost model would pick im2col + rocBLAS */
    setenv("NNHIP_CONV_PATH", "implicit", 1);
    fails += check_module("conv3x3_implicit", conv2d_create(&g_ctx, 128, 128, 3, 1, 1, 4, 4, B, 0, 1.0f), B, 2e-2);
    fails += check_module("conv3x3_implicit_mp", conv2d_create(&g_ctx, 128, 128, 3, 1, 1, 4, 4, B, 1, 1.0f), B,
        2e-2);
    fails += check_module("conv3x3_s2_implicit", conv2d_create(&g_ctx, 32, 128, 3, 2, 1, 5, 5, B, 0, 1.0f), B, 2e-2);
    fails += check_module("conv3x3_implicit_c64", conv2d_create(&g_ctx, 64, 64, 3, 1, 1, 4, 4, B, 1, 1.0f), B, 2e-2);
    unsetenv("NNHIP_CONV_PATH");
    /* diffusion blocks with an embedding slot; the EDM block's emb_lin gain is
       zero at creation (src/cond_conv_residual.c:113), so it is set to 0.7
       here to exercise the modulation path */
    {
        const int emb = 6;
        int slot = ctx_add_cond(&g_ctx, emb, B);
        float* d_emb = nn_device_alloc((size_t)B * emb);
        nn_fill_normal(&g_ctx, d_emb, (size_t)B * emb, 0.0f, 1.0f);
        ctx_set_cond(&g_ctx, slot, d_emb);
        fails += check_module_cond("conv_residual", conv_residual_create(&g_ctx, 8, emb, 4, 4, B, 4, slot), B, 2e-2,
            slot);
        fails += check_module_cond("cond_conv_residual",
            with_scalar_param(cond_conv_residual_create(&g_ctx, 4, emb, 4, 4, B, 0.3f, slot), 1, 0.7f), B, 2e-2,
            slot);
        ctx_free_cond(&g_ctx);
        (void)hipFree(d_emb);
    }
    nn_context_destroy(&g_ctx);
    printf("%s (%d failing module%s)\n", fails ? "GRADCHECK FAILED" : "ALL GRADIENTS OK", fails,
        fails == 1 ? "" : "s");
    fflush(stdout);
    return fails;
}
