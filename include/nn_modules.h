/* nn_modules.h -- host modules on the fused-kernel path, behind the reference's
 * Module vtable and Context (reference src/nn.h:61-254).
 *
 * The types keep the reference's shape so that callers written against it
 * (composite blocks, UNets, the training loop) compile unchanged apart from the
 * vendor types: the stream is a hipStream_t, the GEMM handle a rocBLAS handle,
 * and the cuRAND generator is replaced by a seeded host generator
 * (xoshiro256**, filled on the host and uploaded).
 *
 * Ownership and calling conventions are those of the reference: modules own
 * their parameters, gradients, cached statistics and scratch; forward and
 * backward are asynchronous on ctx->stream; parameter gradients are overwritten
 * by every backward (mp gains are accumulated into a buffer the module zeroes).
 */
#ifndef NN_MODULES_H
#define NN_MODULES_H

#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <hip/hip_runtime_api.h>
#include <rocblas/rocblas.h>

#include "nn_hip.h"
#include "nn_hip_rt.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Abort on a failed HIP runtime call, as NN_CUDA_CHECK does (src/nn.h:13-21). */
#define NN_HIP_CHECK(call)                                           \
    do {                                                             \
        hipError_t _e = (call);                                      \
        if (_e != hipSuccess) {                                      \
            fprintf(stderr, "HIP %s:%d: %s\n", __FILE__, __LINE__,   \
                hipGetErrorString(_e));                              \
            exit(1);                                                 \
        }                                                            \
    } while (0)

#define NN_BLAS_CHECK(call)                                              \
    do {                                                                 \
        rocblas_status _s = (call);                                      \
        if (_s != rocblas_status_success) {                              \
            fprintf(stderr, "rocBLAS %s:%d: status %d\n", __FILE__,      \
                __LINE__, (int)_s);                                      \
            exit(1);                                                     \
        }                                                                \
    } while (0)

/* Shape invariant that survives -O3 (src/nn.h:43-52). */
#define NN_ASSERT(cond, msg)                                       \
    do {                                                           \
        if (!(cond)) {                                             \
            fprintf(stderr, "nn assertion failed %s:%d: %s\n",     \
                __FILE__, __LINE__, msg);                          \
            exit(1);                                               \
        }                                                          \
    } while (0)

float* nn_device_alloc(size_t n_floats);

/* ------------------------------ context ------------------------------ */

#define CTX_MAX_COND 4

typedef struct {
    const float* fwd;
    float* grad;
    int dim;
} CondSlot; /* src/nn.h:65-69 */

typedef struct {
    rocblas_handle blas;  /* GEMM outside the fused path */
    NnHostRng rng;        /* host xoshiro256** state (replaces the cuRAND generator) */
    hipStream_t stream;
    CondSlot cond[CTX_MAX_COND];
    int n_cond;
} Context; /* src/nn.h:71-77 */

/* Create the rocBLAS handle (pointer mode host, bound to `stream`) and seed
   the host generator with SplitMix64(seed). */
void nn_context_init(Context* ctx, uint64_t seed, hipStream_t stream);
void nn_context_destroy(Context* ctx);

int ctx_add_cond(Context* ctx, int dim, int max_batch);
void ctx_set_cond(Context* ctx, int slot, const float* fwd);
void ctx_zero_cond_grad(Context* ctx, int batch);
void ctx_free_cond(Context* ctx);

/* Host generator draws: N(mean, std) by Box-Muller in double, U[0,1) from
   the top 24 bits. Both fill a device buffer through a host staging copy. */
double nn_rng_uniform(Context* ctx);
double nn_rng_normal(Context* ctx);
void nn_fill_normal(Context* ctx, float* dst, size_t n, float mean, float std);
void nn_fill_uniform(Context* ctx, float* dst, size_t n);

/* ------------------------ parameters / optimizer view ------------------------ */

typedef struct {
    float* param;
    float* grad;
    int size;
} Param; /* src/nn.h:139-143 */

typedef struct {
    Param* items;
    int count;
    int capacity;
} ParamList; /* src/nn.h:145-149 */

void param_list_init(ParamList* pl);
void param_list_add(ParamList* pl, float* param, float* grad, int size);
void param_list_free(ParamList* pl);

/* ------------------------------ module vtable ------------------------------ */

typedef struct Module Module;
struct Module {
    const char* name;
    int in_dim, out_dim;
    void* state;
    void (*forward)(Module* self, const float* in, float* out, int batch, Context* ctx);
    void (*backward)(Module* self, const float* in, const float* out,
        const float* grad_out, float* grad_in, int batch, Context* ctx);
    void (*parameters)(Module* self, ParamList* pl); /* may be NULL */
    void (*free)(Module* self);
}; /* src/nn.h:159-174 */

/* ------------------------------ modules ------------------------------ */

Module* activation_create(int dim, Activation act);                 /* src/activation.c:31 */
Module* mp_linear_create(Context* ctx, int in_dim, int out_dim, float gain); /* src/mp_linear.c:60 */
Module* mp_fourier_create(Context* ctx, int num_channels, float bandwidth);   /* src/mp_fourier.c:39 */
Module* sinusoidal_create(int num_channels, float max_period);      /* src/sinusoidal.c:37 */
Module* layernorm_create(int dim, int max_batch);                   /* src/layernorm.c:50 */
Module* spatial_groupnorm_create(int C, int num_groups, int H, int W, int max_batch); /* src/groupnorm.c:52 */
Module* conv2d_create(Context* ctx, int C_in, int C_out, int K, int stride, int pad,
    int H, int W, int max_batch, int mp_mode, float gain);         /* src/conv2d.c:95 */

Module* linear_create(Context* ctx, int in_dim, int out_dim);       /* src/linear.c:49 */

/* Diffusion blocks (src/nn.h:279-283), built on the fused kernels: the DDPM
   residual block (src/conv_residual.c:104) with fused GroupNorm+SiLU and the
   parallel embedding broadcast / reduction, and the EDM2 block
   (src/cond_conv_residual.c:96) with the fused modulation + MP-SiLU pair.
   Both read the embedding from ctx->cond[cond_slot].fwd and add its gradient
   into ctx->cond[cond_slot].grad, as the reference's blocks do. */
Module* conv_residual_create(Context* ctx, int C, int emb_dim, int H, int W,
    int max_batch, int num_groups, int cond_slot);                 /* src/conv_residual.c:104 */
Module* cond_conv_residual_create(Context* ctx, int C, int emb_dim, int H, int W,
    int max_batch, float t, int cond_slot);                        /* src/cond_conv_residual.c:96 */

/* GroupNorm followed by an activation in one module (no reference
   counterpart): forward writes act(GN(x)) only, backward takes the gradient
   of the activated output.  Replaces the GroupNorm module + activation
   launches of src/conv_residual.c:28-29, 51-52. */
Module* spatial_groupnorm_act_create(int C, int num_groups, int H, int W, int max_batch,
    Activation act);

/* ------------------------- sequential container ------------------------- */

typedef struct Sequential Sequential;
Sequential* sequential_create(Module** modules, int n, int max_batch);  /* src/sequential.c:46 */
void sequential_forward(Sequential* s, const float* input, int batch, Context* ctx);
void sequential_backward(Sequential* s, const float* grad_output, int batch, Context* ctx);
float* sequential_output(Sequential* s);
float* sequential_input_grad(Sequential* s);
void sequential_parameters(Sequential* s, ParamList* pl);
void sequential_free(Sequential* s);

/* ------------------------------ optimizer ------------------------------ */

typedef struct Optimizer Optimizer;
Optimizer* optimizer_sgd(const ParamList* pl, float lr);             /* src/optimizer.c:16 */
Optimizer* optimizer_adam(const ParamList* pl, float lr,
    float beta1, float beta2, float eps);                            /* src/optimizer.c:29 */
void optimizer_step(Optimizer* o, const ParamList* pl, Context* ctx); /* src/optimizer.c:54 */
void optimizer_set_lr(Optimizer* o, float lr);
void optimizer_free(Optimizer* o);
int optimizer_timestep(const Optimizer* o);
void optimizer_set_timestep(Optimizer* o, int t);
void optimizer_moment_lists(const Optimizer* o, ParamList* m, ParamList* v);

/* ------------------------------ EMA ------------------------------ */

typedef struct EMA EMA;
EMA* ema_create(const ParamList* pl, float decay);                   /* src/ema.c:12 */
void ema_update(EMA* ema, const ParamList* pl, Context* ctx);        /* src/ema.c:29 */
void ema_swap(EMA* ema, ParamList* pl, Context* ctx);                /* src/ema.c:37 */
void ema_free(EMA* ema);
void ema_shadow_list(const EMA* ema, ParamList* shadow);

/* ------------------------------ checkpoints ------------------------------ */

/* The reference's CKPT (weights) and CKTR (params, EMA shadow, Adam m, Adam v,
   step and Adam counters) files, byte for byte (src/checkpoint.c:1-136,
   declared at src/nn.h:256-269).  0 on success; -1 open/write failure, -2 bad
   magic or short file, -3 count mismatch, -4 size mismatch. */
int checkpoint_save(const char* path, const ParamList* pl);
int checkpoint_load(const char* path, ParamList* pl);
int checkpoint_save_training(const char* path, int step, int adam_t,
    const ParamList* params, const ParamList* ema_shadow,
    const ParamList* adam_m, const ParamList* adam_v);
int checkpoint_load_training(const char* path, int* step, int* adam_t,
    ParamList* params, ParamList* ema_shadow,
    ParamList* adam_m, ParamList* adam_v);

/* optimizer_step followed by ema_update in one launch (no reference
   counterpart; replaces src/diffusion/train.c:53-54).  Same results as the
   two calls in sequence.  Adam optimizers only. */
void optimizer_step_ema(Optimizer* o, EMA* ema, const ParamList* pl, Context* ctx);

#ifdef __cplusplus
}
#endif

#endif /* NN_MODULES_H */
