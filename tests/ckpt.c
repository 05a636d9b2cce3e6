/* ckpt.c -- checkpoint round trips for tests/test_gpu_checkpoint.py (built
 * into _build/libgradcheck.so).  A fixed three-tensor model (sizes 5, 64, 1)
 * with p0[k][i] = 0.01 (i + 1) (k + 1) and g[k][i] = 0.001 (i - 3) (k + 1)
 * takes `steps` fused Adam+EMA steps (lr 1e-3, betas 0.9/0.999, eps 1e-8,
 * decay 0.99), then the training state is written, or a file is loaded into
 * the same lists.  Needs a GPU.
 */
#include <string.h>

#include "nn_modules.h"

#define NT 3
static const int kSizes[NT] = {5, 64, 1};

typedef struct {
    Context ctx;
    ParamList pl, shadow, m, v;
    Optimizer* opt;
    EMA* ema;
    float* p[NT];
    float* g[NT];
} Model;

static void model_init(Model* md)
{
    nn_context_init(&md->ctx, 7ull, (hipStream_t)0);
    param_list_init(&md->pl);
    param_list_init(&md->shadow);
    param_list_init(&md->m);
    param_list_init(&md->v);
    for (int k = 0; k < NT; ++k) {
        const int n = kSizes[k];
        float* hp = (float*)malloc((size_t)n * sizeof(float));
        float* hg = (float*)malloc((size_t)n * sizeof(float));
        for (int i = 0; i < n; ++i) {
            hp[i] = 0.01f * (float)(i + 1) * (float)(k + 1);
            hg[i] = 0.001f * (float)(i - 3) * (float)(k + 1);
        }
        md->p[k] = nn_device_alloc((size_t)n);
        md->g[k] = nn_device_alloc((size_t)n);
        NN_HIP_CHECK(hipMemcpy(md->p[k], hp, (size_t)n * sizeof(float), hipMemcpyHostToDevice));
        NN_HIP_CHECK(hipMemcpy(md->g[k], hg, (size_t)n * sizeof(float), hipMemcpyHostToDevice));
        free(hp);
        free(hg);
        param_list_add(&md->pl, md->p[k], md->g[k], n);
    }
    md->opt = optimizer_adam(&md->pl, 1e-3f, 0.9f, 0.999f, 1e-8f);
    md->ema = ema_create(&md->pl, 0.99f);
    optimizer_moment_lists(md->opt, &md->m, &md->v);
    ema_shadow_list(md->ema, &md->shadow);
}

static void model_free(Model* md)
{
    NN_HIP_CHECK(hipDeviceSynchronize());
    optimizer_free(md->opt);
    ema_free(md->ema);
    for (int k = 0; k < NT; ++k) {
        (void)hipFree(md->p[k]);
        (void)hipFree(md->g[k]);
    }
    param_list_free(&md->pl);
    param_list_free(&md->shadow);
    param_list_free(&md->m);
    param_list_free(&md->v);
    nn_context_destroy(&md->ctx);
}

/* Copy the four lists (params, shadow, m, v) to host, in file order. */
static int dump_lists(Model* md, float* out, int cap)
{
    const ParamList* lists[4] = {&md->pl, &md->shadow, &md->m, &md->v};
    int off = 0;
    NN_HIP_CHECK(hipDeviceSynchronize());
    for (int l = 0; l < 4; ++l)
        for (int k = 0; k < lists[l]->count; ++k) {
            const int n = lists[l]->items[k].size;
            if (off + n > cap) return -1;
            NN_HIP_CHECK(hipMemcpy(out + off, lists[l]->items[k].param, (size_t)n * sizeof(float),
                hipMemcpyDeviceToHost));
            off += n;
        }
    return off;
}

/* Run `steps` steps, save the training state at `path` with the given step
   counter; the state is also copied to `out` (file order).  Returns the
   checkpoint_save_training code, or -100 if out is too small. */
int nn_ckpt_test_save(const char* path, int steps, int step_counter, float* out, int cap)
{
    Model md;
    model_init(&md);
    for (int s = 0; s < steps; ++s) optimizer_step_ema(md.opt, md.ema, &md.pl, &md.ctx);
    NN_HIP_CHECK(hipDeviceSynchronize());
    int rc = checkpoint_save_training(path, step_counter, optimizer_timestep(md.opt), &md.pl, &md.shadow, &md.m,
        &md.v);
    if (!rc && dump_lists(&md, out, cap) < 0) rc = -100;
    model_free(&md);
    return rc;
}

/* Load `path` into a fresh model; out receives the four lists (file order),
   counters[0..1] = step, adam_t.  Returns the checkpoint_load_training code. */
int nn_ckpt_test_load(const char* path, float* out, int cap, int* counters)
{
    Model md;
    model_init(&md);
    int rc = checkpoint_load_training(path, &counters[0], &counters[1], &md.pl, &md.shadow, &md.m, &md.v);
    if (!rc) {
        optimizer_set_timestep(md.opt, counters[1]);
        if (dump_lists(&md, out, cap) < 0) rc = -100;
    }
    model_free(&md);
    return rc;
}

/* Weights-only round trip: save the initial params, clobber, load back.
   Returns 0 when the reloaded bits equal the saved ones. */
int nn_ckpt_test_weights(const char* path)
{
    Model md;
    model_init(&md);
    float before[70], after[70];
    int off = 0;
    for (int k = 0; k < NT; ++k) {
        NN_HIP_CHECK(hipMemcpy(before + off, md.p[k], (size_t)kSizes[k] * sizeof(float), hipMemcpyDeviceToHost));
        off += kSizes[k];
    }
    int rc = checkpoint_save(path, &md.pl);
    for (int k = 0; k < NT && !rc; ++k) NN_HIP_CHECK(hipMemset(md.p[k], 0, (size_t)kSizes[k] * sizeof(float)));
    if (!rc) rc = checkpoint_load(path, &md.pl);
    off = 0;
    for (int k = 0; k < NT && !rc; ++k) {
        NN_HIP_CHECK(hipMemcpy(after + off, md.p[k], (size_t)kSizes[k] * sizeof(float), hipMemcpyDeviceToHost));
        off += kSizes[k];
    }
    if (!rc && memcmp(before, after, (size_t)off * sizeof(float)) != 0) rc = -101;
    model_free(&md);
    return rc;
}

/* Load a weights file into a model whose first tensor has `size0` elements
   (count mismatch when drop_last): exercises the -3 / -4 codes. */
int nn_ckpt_test_load_mismatch(const char* path, int size0, int drop_last)
{
    ParamList pl;
    param_list_init(&pl);
    float* bufs[NT];
    const int n_t = drop_last ? NT - 1 : NT;
    for (int k = 0; k < n_t; ++k) {
        const int n = k == 0 ? size0 : kSizes[k];
        bufs[k] = nn_device_alloc((size_t)n);
        param_list_add(&pl, bufs[k], NULL, n);
    }
    const int rc = checkpoint_load(path, &pl);
    for (int k = 0; k < n_t; ++k) (void)hipFree(bufs[k]);
    param_list_free(&pl);
    return rc;
}

/* Weights round trip of a list with the given tensor sizes: each tensor is
   filled with a pattern of its own, saved, zeroed, loaded and compared bit
   for bit.  Returns the number of tensors that differ, or the load's error
   code when it fails. */
int nn_ckpt_test_roundtrip_sizes(const char* path, const int* sizes, int n)
{
    ParamList pl;
    param_list_init(&pl);
    float** dev = (float**)calloc((size_t)n, sizeof(float*));
    float** want = (float**)calloc((size_t)n, sizeof(float*));
    for (int k = 0; k < n; ++k) {
        const size_t m = (size_t)sizes[k];
        want[k] = (float*)malloc((m ? m : 1) * sizeof(float));
        for (size_t i = 0; i < m; ++i) want[k][i] = (float)(k + 1) + 1e-6f * (float)(i % 1000003);
        dev[k] = nn_device_alloc(m ? m : 1);
        if (m) NN_HIP_CHECK(hipMemcpy(dev[k], want[k], m * sizeof(float), hipMemcpyHostToDevice));
        param_list_add(&pl, dev[k], NULL, sizes[k]);
    }
    int rc = checkpoint_save(path, &pl);
    for (int k = 0; k < n && !rc; ++k)
        if (sizes[k]) NN_HIP_CHECK(hipMemset(dev[k], 0, (size_t)sizes[k] * sizeof(float)));
    if (!rc) rc = checkpoint_load(path, &pl);
    int bad = 0;
    for (int k = 0; k < n; ++k) {
        const size_t m = (size_t)sizes[k];
        if (!rc && m) {
            float* got = (float*)malloc(m * sizeof(float));
            NN_HIP_CHECK(hipMemcpy(got, dev[k], m * sizeof(float), hipMemcpyDeviceToHost));
            bad += memcmp(got, want[k], m * sizeof(float)) != 0;
            free(got);
        }
        (void)hipFree(dev[k]);
        free(want[k]);
    }
    free(dev);
    free(want);
    param_list_free(&pl);
    return rc ? rc : bad;
}
