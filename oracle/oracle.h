/* oracle.h -- CPU restatement of the reference's fused-layer maths.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * or the reported CPU baseline; the product path never calls it.
 *
 * Each function cites the reference lines it restates (src/kernels.cu unless
 * another file is named).  Conventions:
 *   - elementwise arithmetic is fp32 in the reference's operation order; the
 *     library is built with -ffp-contract=off, so no fused multiply-adds;
 *   - reductions (means, variances, channel sums, dot products) accumulate in
 *     double and round once ("truth" for the 1e-5 checks);
 *   - the *_f32 variants keep the reference's fp32 serial accumulation and
 *     parallelise over the reference's own units with OpenMP: they are the
 *     CPU baseline of the benchmark, not a checker.
 * Tensors are host arrays in the layouts of the launch layer (NHWC).
 */
#ifndef NN_ORACLE_H
#define NN_ORACLE_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* activation kinds, values of the reference enum (src/nn.h:178-183) */
enum { ORC_IDENTITY = 0, ORC_RELU, ORC_GELU, ORC_SILU, ORC_TANH, ORC_MP_SILU };

/* ---- scalar activation family (kernels.cu:6-68) ---- */
float orc_pade_tanh(float x);
float orc_pade_sigmoid(float x);
float orc_act(float v, int act);
float orc_act_grad(float z, int act);

/* ---- elementwise (kernels.cu:95-117, 163-183, 300-314) ---- */
void orc_activation_forward(float* out, const float* in, long long n, int act);
void orc_activation_backward(float* gin, const float* gout, const float* in, long long n, int act);
void orc_weighted_sum(float* out, const float* a, const float* b, float wa, float wb, long long n);
void orc_mp_sum_weights(float t, float* wa, float* wb);              /* kernels.cu:363-364 */
void orc_mp_cat_weights(float t, int Na, int Nb, float* wa, float* wb); /* kernels.cu:1251-1257 */
void orc_mp_cat(float* out, const float* a, const float* b, float wa, float wb,
    long long rows, int Na, int Nb);                                  /* kernels.cu:318-328 */
void orc_mp_split(float* ga, float* gb, const float* g, float wa, float wb,
    long long rows, int Ca, int Cb);                                  /* kernels.cu:1215-1232 */
void orc_scale_by_scalar(float* x, float s, long long n);              /* kernels.cu:300-306 */
void orc_add_bias(float* Y, const float* b, long long M, int N);       /* kernels.cu:95-101 */
void orc_bias_grad(float* gb, const float* g, long long rows, int N);  /* kernels.cu:148-161 */
void orc_sgd_step(float* p, const float* g, float lr, long long n);    /* kernels.cu:163-168 */
void orc_adam_step(float* p, float* m, float* v, const float* g, float lr, float b1, float b2,
    float eps, float bc1, float bc2, long long n);                    /* kernels.cu:170-183 */
void orc_adam_bias_corrections(float b1, float b2, int t, float* bc1, float* bc2); /* optimizer.c:62-64 */

/* ---- normalisation ---- */
/* GroupNorm (kernels.cu:622-717) with the activation applied after it as the
   DDPM block does (conv_residual.c:28-29, 51-52); act = ORC_IDENTITY gives the
   plain GroupNorm. */
void orc_groupnorm_forward(float* y, float* mu, float* rstd, const float* x, const float* gamma,
    const float* beta, int B, int HW, int C, int G, float eps, int act);
void orc_groupnorm_backward(float* dx, float* ggamma, float* gbeta, const float* dy,
    const float* x, const float* gamma, const float* beta, const float* mu, const float* rstd,
    int B, int HW, int C, int G, int act);
/* LayerNorm (kernels.cu:491-567) */
void orc_layernorm_forward(float* y, float* mu, float* rstd, const float* x, const float* gamma,
    const float* beta, long long rows, int C, float eps);
void orc_layernorm_backward(float* dx, float* ggamma, float* gbeta, const float* dy,
    const float* x, const float* gamma, const float* mu, const float* rstd, long long rows, int C);

/* ---- weight normalisation (kernels.cu:255-297) ---- */
void orc_weight_normalize(float* W, int in, int out, float eps);
void orc_weight_normalize_backward(float* gW, const float* Wn, float gain, float* g_gain,
    int in, int out);

/* ---- embeddings (kernels.cu:385-394, 444-456) ---- */
void orc_mp_fourier(float* out, const float* x, const float* freqs, const float* phases,
    int batch, int C);
void orc_sinusoidal(float* out, const float* t, int batch, int C, float log_max_period);

/* ---- conv helpers (kernels.cu:750-816) ---- */
void orc_im2col(float* col, const float* im, int B, int H, int W, int C, int K, int stride,
    int pad, int Ho, int Wo);
/* The reference kernel's loop run sequentially in ascending index order with
   plain fp32 adds into grad_im (which keeps its incoming values). */
void orc_col2im(float* grad_im, const float* grad_col, int B, int H, int W, int C, int K,
    int stride, int pad, int Ho, int Wo);

/* ---- fp32-faithful OpenMP transcription: the CPU baseline ---- */
void orc_spatial_add(float* x, const float* v, int B, int HW, int C);
void orc_spatial_reduce_sum(float* out, const float* x, int B, int HW, int C);
void orc_spatial_modulate(float* out, const float* x, const float* cond, int B, int HW, int C);
void orc_spatial_modulate_backward(float* gin, float* gcond, const float* gout, const float* x,
    const float* cond, int B, int HW, int C);
void orc_spatial_modulate_act_forward(float* out, const float* x, const float* cond, int B, int HW,
    int C, int act);
void orc_spatial_modulate_act_backward(float* gin, float* gcond, const float* gout, const float* x,
    const float* cond, int B, int HW, int C, int act);
void orc_set_threads(int n);
int orc_get_threads(void);
void orc_groupnorm_forward_f32(float* y, float* mu, float* rstd, const float* x,
    const float* gamma, const float* beta, int B, int HW, int C, int G, float eps, int act);
void orc_groupnorm_backward_f32(float* dx, float* ggamma, float* gbeta, const float* dy,
    const float* x, const float* gamma, const float* beta, const float* mu, const float* rstd,
    int B, int HW, int C, int G, int act);

#ifdef __cplusplus
}
#endif

#endif /* NN_ORACLE_H */
