/* core.c -- device allocation, Context, the host generator and ParamList.
 * Reference: src/nn.h:54-135 (allocation, context, cond slots, normal fill)
 * and src/sequential.c:5-29 (ParamList).
 */
#include <math.h>
#include <string.h>

#include "nn_modules.h"

float* nn_device_alloc(size_t n_floats)
{
    void* p = NULL;
    NN_HIP_CHECK(hipMalloc(&p, (n_floats ? n_floats : 1) * sizeof(float)));
    return (float*)p;
}

/* ---- host generator: SplitMix64 seeding, xoshiro256** (Blackman & Vigna) ---- */

static uint64_t splitmix64(uint64_t* s)
{
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static inline uint64_t rotl64(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

static uint64_t xoshiro_next(uint64_t* s)
{
    const uint64_t result = rotl64(s[1] * 5, 7) * 9;
    const uint64_t t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl64(s[3], 45);
    return result;
}

static double rng_uniform(NnHostRng* g) /* [0, 1) with 53 random bits */
{
    return (double)(xoshiro_next(g->s) >> 11) * (1.0 / 9007199254740992.0);
}

static double rng_normal(NnHostRng* g) /* Box-Muller, cosine branch */
{
    double u1 = 1.0 - rng_uniform(g); /* (0, 1] */
    double u2 = rng_uniform(g);
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}

void nnhip_rng_seed(NnHostRng* g, uint64_t seed)
{
    uint64_t s = seed;
    for (int i = 0; i < 4; ++i) g->s[i] = splitmix64(&s);
}

int nnhip_fill_normal(NnHostRng* g, float* dst, size_t n, float mean, float std)
{
    if (n == 0) return 0;
    float* h = (float*)malloc(n * sizeof(float));
    for (size_t i = 0; i < n; ++i) h[i] = (float)((double)mean + (double)std * rng_normal(g));
    const hipError_t e = hipMemcpy(dst, h, n * sizeof(float), hipMemcpyHostToDevice);
    free(h);
    return (int)e;
}

int nnhip_fill_uniform(NnHostRng* g, float* dst, size_t n)
{
    if (n == 0) return 0;
    float* h = (float*)malloc(n * sizeof(float));
    for (size_t i = 0; i < n; ++i) h[i] = (float)(xoshiro_next(g->s) >> 40) * (1.0f / 16777216.0f);
    const hipError_t e = hipMemcpy(dst, h, n * sizeof(float), hipMemcpyHostToDevice);
    free(h);
    return (int)e;
}

double nn_rng_uniform(Context* ctx) { return rng_uniform(&ctx->rng); }
double nn_rng_normal(Context* ctx) { return rng_normal(&ctx->rng); }

void nn_fill_normal(Context* ctx, float* dst, size_t n, float mean, float std)
{
    NN_HIP_CHECK((hipError_t)nnhip_fill_normal(&ctx->rng, dst, n, mean, std));
}

void nn_fill_uniform(Context* ctx, float* dst, size_t n)
{
    NN_HIP_CHECK((hipError_t)nnhip_fill_uniform(&ctx->rng, dst, n));
}

/* ---- context ---- */

void nn_context_init(Context* ctx, uint64_t seed, hipStream_t stream)
{
    memset(ctx, 0, sizeof *ctx);
    nnhip_rng_seed(&ctx->rng, seed);
    ctx->stream = stream;
    NN_BLAS_CHECK(rocblas_create_handle(&ctx->blas));
    NN_BLAS_CHECK(rocblas_set_stream(ctx->blas, stream));
    NN_BLAS_CHECK(rocblas_set_pointer_mode(ctx->blas, rocblas_pointer_mode_host));
}

void nn_context_destroy(Context* ctx)
{
    ctx_free_cond(ctx);
    if (ctx->blas) rocblas_destroy_handle(ctx->blas);
    ctx->blas = NULL;
}

int ctx_add_cond(Context* ctx, int dim, int max_batch) /* src/nn.h:79-90 */
{
    NN_ASSERT(ctx->n_cond < CTX_MAX_COND, "ctx_add_cond: too many conditioning slots");
    int slot = ctx->n_cond++;
    ctx->cond[slot].dim = dim;
    ctx->cond[slot].fwd = NULL;
    ctx->cond[slot].grad = nn_device_alloc((size_t)max_batch * dim);
    return slot;
}

void ctx_set_cond(Context* ctx, int slot, const float* fwd) { ctx->cond[slot].fwd = fwd; }

void ctx_zero_cond_grad(Context* ctx, int batch) /* src/nn.h:97-103 */
{
    for (int i = 0; i < ctx->n_cond; ++i)
        if (ctx->cond[i].grad)
            nnhip_fill_f32(ctx->cond[i].grad, 0.0f, (size_t)batch * ctx->cond[i].dim, ctx->stream);
}

void ctx_free_cond(Context* ctx)
{
    for (int i = 0; i < ctx->n_cond; ++i) {
        if (ctx->cond[i].grad) (void)hipFree(ctx->cond[i].grad);
        ctx->cond[i].grad = NULL;
        ctx->cond[i].fwd = NULL;
    }
    ctx->n_cond = 0;
}

/* ---- ParamList ---- */

void param_list_init(ParamList* pl)
{
    pl->count = 0;
    pl->capacity = 64;
    pl->items = (Param*)malloc((size_t)pl->capacity * sizeof(Param));
}

void param_list_add(ParamList* pl, float* param, float* grad, int size)
{
    if (pl->count == pl->capacity) {
        pl->capacity *= 2;
        pl->items = (Param*)realloc(pl->items, (size_t)pl->capacity * sizeof(Param));
    }
    pl->items[pl->count].param = param;
    pl->items[pl->count].grad = grad;
    pl->items[pl->count].size = size;
    pl->count++;
}

void param_list_free(ParamList* pl)
{
    free(pl->items);
    pl->items = NULL;
    pl->count = pl->capacity = 0;
}
