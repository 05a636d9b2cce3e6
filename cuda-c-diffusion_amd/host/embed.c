/* embed.c -- the two time/noise embedding modules.
 * mp_fourier: reference src/mp_fourier.c:4-61 (freqs ~ N(0, bandwidth),
 *   phases ~ U[0,1), drawn here from the context's host generator).
 * sinusoidal: reference src/sinusoidal.c:5-58 (C even, logf(max_period)).
 * Neither has a gradient: their backward is a no-op, as in the reference. */
#include <math.h>

#include "nn_modules.h"

typedef struct {
    int C;
    float *freqs, *phases;
} FourierState;

static void mp_fourier_forward(Module* self, const float* in, float* out, int batch, Context* ctx)
{
    FourierState* st = (FourierState*)self->state;
    launch_mp_fourier(out, in, st->freqs, st->phases, batch, st->C, ctx->stream);
}

static void no_backward(Module* self, const float* in, const float* out, const float* grad_out,
    float* grad_in, int batch, Context* ctx)
{
    (void)self;
    (void)in;
    (void)out;
    (void)grad_out;
    (void)grad_in;
    (void)batch;
    (void)ctx;
}

static void mp_fourier_free(Module* self)
{
    FourierState* st = (FourierState*)self->state;
    (void)hipFree(st->freqs);
    (void)hipFree(st->phases);
    free(st);
    free(self);
}

Module* mp_fourier_create(Context* ctx, int num_channels, float bandwidth)
{
    Module* m = (Module*)malloc(sizeof(Module));
    FourierState* st = (FourierState*)malloc(sizeof(FourierState));
    st->C = num_channels;
    st->freqs = nn_device_alloc((size_t)num_channels);
    st->phases = nn_device_alloc((size_t)num_channels);
    nn_fill_normal(ctx, st->freqs, (size_t)num_channels, 0.0f, bandwidth);
    nn_fill_uniform(ctx, st->phases, (size_t)num_channels);
    m->name = "mp_fourier";
    m->in_dim = 1;
    m->out_dim = num_channels;
    m->state = st;
    m->forward = mp_fourier_forward;
    m->backward = no_backward;
    m->parameters = NULL;
    m->free = mp_fourier_free;
    return m;
}

typedef struct {
    int C;
    float log_max_period;
} SinusoidalState;

static void sinusoidal_forward(Module* self, const float* in, float* out, int batch, Context* ctx)
{
    SinusoidalState* st = (SinusoidalState*)self->state;
    launch_sinusoidal(out, in, batch, st->C, st->log_max_period, ctx->stream);
}

static void sinusoidal_free(Module* self)
{
    free(self->state);
    free(self);
}

Module* sinusoidal_create(int num_channels, float max_period)
{
    NN_ASSERT(num_channels % 2 == 0, "sinusoidal_create: num_channels must be even");
    Module* m = (Module*)malloc(sizeof(Module));
    SinusoidalState* st = (SinusoidalState*)malloc(sizeof(SinusoidalState));
    st->C = num_channels;
    st->log_max_period = logf(max_period);
    m->name = "sinusoidal";
    m->in_dim = 1;
    m->out_dim = num_channels;
    m->state = st;
    m->forward = sinusoidal_forward;
    m->backward = no_backward;
    m->parameters = NULL;
    m->free = sinusoidal_free;
    return m;
}
