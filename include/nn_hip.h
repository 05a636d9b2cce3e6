/* nn_hip.h -- the drop-in C-ABI launch layer for the fused layer kernels.
 *
 * Every entry point below replaces one `extern "C"` launcher of the reference's
 * CUDA launch layer (reference src/nn.h:348-466, definitions in src/kernels.cu).
 * Names, argument order and argument meaning are kept; the trailing stream is a
 * HIP stream. All pointers are device pointers unless stated otherwise, sizes are
 * element counts, scalars are host floats. Launchers are asynchronous on the
 * given stream, keep no state between calls and return nothing, as in the
 * reference.
 *
 * Errors: the reference reports nothing from a launcher. Here a launcher that is
 * handed an impossible shape (for example C not divisible by G) refuses to launch
 * and records the reason; a failed launch is recorded too. Read and clear the
 * record with nnhip_get_last_error() (nn_hip_rt.h). Setting NNHIP_CHECK=1 in the
 * environment makes every launcher synchronise its stream and abort the process
 * on any error (a debug mode).
 *
 * Entry points in the "fused additions" block have no reference counterpart;
 * each names the reference call sequence it replaces.
 */
#ifndef NN_HIP_H
#define NN_HIP_H

#include <stddef.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Activation kinds; values as the reference enum (src/nn.h:178-183). */
typedef enum {
    ACT_IDENTITY = 0,
    ACT_RELU,
    ACT_GELU,
    ACT_SILU,
    ACT_TANH,
    ACT_MP_SILU
} Activation;

/* ------------------------------------------------------------------------
 * Support kernels used by on-path host modules
 * ------------------------------------------------------------------------ */

/* Y[m,n] += b[n] for a row-major [M,N] Y.  replaces nn.h:354 / kernels.cu:95-101,193-197 */
void launch_add_bias(float* Y, const float* b, int M, int N, hipStream_t s);

/* gb[n] = sum_r grad_out[r,n] over `batch` rows (overwrites gb).
   replaces nn.h:365-366 / kernels.cu:148-161,225-232 */
void launch_bias_grad(float* gb, const float* grad_out, int batch, int N,
    hipStream_t s);

/* p[i] -= lr * g[i].  replaces nn.h:368 / kernels.cu:163-168,234-239 */
void launch_sgd_step(float* p, const float* g, float lr, int n, hipStream_t s);

/* ------------------------------------------------------------------------
 * Activations (Pade [7/6] tanh family)
 * ------------------------------------------------------------------------ */

/* out[i] = act(in[i]).  replaces nn.h:356-357 / kernels.cu:103-109,199-204 */
void launch_activation_forward(float* out, const float* in, int n,
    Activation act, hipStream_t s);

/* grad_in[i] = grad_out[i] * act'(in[i]), `in` = the pre-activation.
   replaces nn.h:358-360 / kernels.cu:111-117,206-213 */
void launch_activation_backward(float* grad_in, const float* grad_out,
    const float* in, int n, Activation act, hipStream_t s);

/* ------------------------------------------------------------------------
 * Optimizer
 * ------------------------------------------------------------------------ */

/* One Adam update of one tensor; bc1/bc2 are the host-computed bias
   corrections 1-beta^t.  replaces nn.h:369-371 / kernels.cu:170-183,241-248 */
void launch_adam_step(float* p, float* m, float* v, const float* g,
    float lr, float beta1, float beta2, float eps,
    float bc1, float bc2, int n, hipStream_t s);

/* ------------------------------------------------------------------------
 * Magnitude-preserving ops
 * ------------------------------------------------------------------------ */

/* In place: W[:,j] *= rsqrt(sum_i W[i,j]^2 + eps) for W [in,out] row-major.
   replaces nn.h:374 / kernels.cu:255-272,330-335 */
void launch_weight_normalize(float* W, int in, int out, float eps, hipStream_t s);

/* dot_j = <Wn[:,j], gW[:,j]>;  *g_gain += sum_j dot_j;
   gW[:,j] = gain[0] * (gW[:,j] - dot_j * Wn[:,j]).  The caller zeroes g_gain
   when it wants a fresh value, as in the reference.
   replaces nn.h:375-376 / kernels.cu:277-297,337-344 */
void launch_weight_normalize_backward(float* gW, const float* Wn, const float* gain,
    float* g_gain, int in, int out, hipStream_t s);

/* Workspace variant of launch_weight_normalize_backward (no counterpart in
   the reference): identical results, one launch and no pool allocation.  The
   caller lends `workspace` of nnhip_weight_normalize_backward_workspace(out)
   floats, zero-filled before its first use; every launch leaves it re-armed.
   Launches that may run concurrently need separate workspaces. */
size_t nnhip_weight_normalize_backward_workspace(int out);
void launch_weight_normalize_backward_ws(float* gW, const float* Wn, const float* gain,
    float* g_gain, int in, int out, float* workspace, hipStream_t s);

/* x[i] *= s[0] (device-resident scalar).  replaces nn.h:377 / kernels.cu:300-306,346-351 */
void launch_scale_by_scalar(float* x, const float* s, int n, hipStream_t st);

/* out = mp_sum(a, b, t): weights (1-t)/d, t/d with d = sqrt((1-t)^2+t^2),
   computed on the host in float.  replaces nn.h:378-379 / kernels.cu:360-366 */
void launch_mp_sum(float* out, const float* a, const float* b, float t, int n,
    hipStream_t s);

/* out[i] = wa*a[i] + wb*b[i].  replaces nn.h:380-381 / kernels.cu:308-314,353-358 */
void launch_weighted_sum(float* out, const float* a, const float* b,
    float wa, float wb, int n, hipStream_t s);

/* out[r,:] = [wa*a[r,:Na], wb*b[r,:Nb]] with the magnitude-preserving weights of
   blend t.  replaces nn.h:408-409 / kernels.cu:318-328,368-378 */
void launch_mp_cat(float* out, const float* a, const float* b, float t,
    int batch, int Na, int Nb, hipStream_t s);

/* NHWC channel concat with mp_cat weights over `spatial` = N*H*W pixels.
   replaces nn.h:453-454 / kernels.cu:1251-1267 */
void launch_mp_channel_cat(float* out, const float* a, const float* b,
    float t, int spatial, int Ca, int Cb, hipStream_t s);

/* Backward of launch_mp_channel_cat: ga = wa*g[:, :Ca], gb = wb*g[:, Ca:].
   replaces nn.h:455-456 / kernels.cu:1215-1232,1269-1278 */
void launch_mp_channel_split(float* grad_a, float* grad_b, const float* grad_out,
    float t, int spatial, int Ca, int Cb, hipStream_t s);

/* ------------------------------------------------------------------------
 * Embeddings
 * ------------------------------------------------------------------------ */

/* out[b,k] = sqrt(2) * cos(2*pi*(x[b]*freqs[k] + phases[k])).
   replaces nn.h:382-383 / kernels.cu:385-394,416-423 */
void launch_mp_fourier(float* out, const float* x, const float* freqs,
    const float* phases, int batch, int C, hipStream_t s);

/* out[b,c] = c<C/2 ? sin(t[b]*f_c) : cos(t[b]*f_{c-C/2}),
   f_j = exp(-log_max_period*j/(C/2)).  replaces nn.h:387-388 / kernels.cu:444-456,569-575 */
void launch_sinusoidal(float* out, const float* t, int batch, int C,
    float log_max_period, hipStream_t s);

/* ------------------------------------------------------------------------
 * Normalisation
 * ------------------------------------------------------------------------ */

/* Per-row LayerNorm of x [batch, C]; writes y, mu[batch], rstd[batch].
   replaces nn.h:393-395 / kernels.cu:491-516,594-602 */
void launch_layernorm_forward(float* y, float* mu, float* rstd, const float* x,
    const float* gamma, const float* beta,
    int batch, int C, float eps, hipStream_t s);

/* LayerNorm backward from the cached mu/rstd; overwrites ggamma/gbeta [C].
   replaces nn.h:396-399 / kernels.cu:520-567,604-616 */
void launch_layernorm_backward(float* grad_in, float* ggamma, float* gbeta,
    const float* grad_out, const float* x, const float* gamma,
    const float* mu, const float* rstd,
    int batch, int C, hipStream_t s);

/* NHWC GroupNorm of x [batch, HW, C] over G groups of C/G channels; writes y,
   mu[batch*G], rstd[batch*G].  replaces nn.h:400-403 / kernels.cu:622-657,719-729 */
void launch_groupnorm_forward(float* y, float* mu, float* rstd,
    const float* x, const float* gamma, const float* beta,
    int batch, int HW, int C, int G, float eps, hipStream_t s);

/* GroupNorm backward from the cached mu/rstd: dx, and ggamma/gbeta [C]
   (overwritten).  replaces nn.h:404-407 / kernels.cu:659-717,731-745 */
void launch_groupnorm_backward(float* dx, float* ggamma, float* gbeta,
    const float* dy, const float* x, const float* gamma,
    const float* mu, const float* rstd,
    int batch, int HW, int C, int G, hipStream_t s);

/* ------------------------------------------------------------------------
 * Convolution helpers (NHWC)
 * ------------------------------------------------------------------------ */

/* col[(b,oh,ow), (kh,kw,ci)] = im[b, oh*stride+kh-pad, ow*stride+kw-pad, ci]
   or 0 outside the image.  replaces nn.h:412-413 / kernels.cu:750-781,818-827 */
void launch_im2col(float* col, const float* im, int batch, int H, int W, int C,
    int K, int stride, int pad, int H_out, int W_out, hipStream_t s);

/* grad_im += col2im(grad_col): every im element adds its contributions in the
   order of the reference kernel's sequential index (ascending (oh,ow), i.e.
   kh then kw descending), starting from the value already in grad_im. The
   reference caller zeroes grad_im first.  replaces nn.h:414-415 / kernels.cu:785-816,829-838 */
void launch_col2im(float* grad_im, const float* grad_col, int batch, int H, int W, int C,
    int K, int stride, int pad, int H_out, int W_out, hipStream_t s);

/* ------------------------------------------------------------------------
 * Spatial (per sample and channel) broadcasts and reductions, NHWC
 * x [batch, H*W, C], v / cond [batch, C].
 * ------------------------------------------------------------------------ */

/* inout[b,hw,c] += bias[b,c].  replaces nn.h:443-444 / kernels.cu:1132-1142,1160-1168 */
void launch_spatial_add(float* inout, const float* bias, int batch, int H, int W, int C,
    hipStream_t s);

/* out[b,c] = sum over hw of in[b,hw,c] (overwrites out; 0 when HW = 0), summed
   in a fixed order.  replaces nn.h:445-446 / kernels.cu:1145-1158,1170-1178 */
void launch_spatial_reduce_sum(float* out, const float* in, int batch, int HW, int C,
    hipStream_t s);

/* out = in * (cond[b,c] + 1).  replaces nn.h:435-436 / kernels.cu:1055-1067,1103-1111 */
void launch_spatial_modulate(float* out, const float* in, const float* cond,
    int batch, int H, int W, int C, hipStream_t s);

/* grad_in = grad_out * (cond + 1); grad_cond[b,c] = sum over hw of grad_out * in
   (overwrites grad_cond).  replaces nn.h:437-441 / kernels.cu:1070-1101,1113-1126 */
void launch_spatial_modulate_backward(float* grad_in, float* grad_cond,
    const float* grad_out, const float* in, const float* cond,
    int batch, int H, int W, int C, hipStream_t s);

/* ========================================================================
 * Fused additions (no reference counterpart)
 * ======================================================================== */

/* out = act(in * (cond[b,c] + 1)) in one pass; replaces the EDM block's pair
   launch_spatial_modulate + launch_activation_forward
   (src/cond_conv_residual.c:30-33), whose intermediate is not stored. */
void launch_spatial_modulate_act_forward(float* out, const float* in, const float* cond,
    int batch, int H, int W, int C, Activation act, hipStream_t s);

/* Backward of launch_spatial_modulate_act_forward in one pass: with
   g2 = grad_out * act'(in * (cond + 1)), grad_in = g2 * (cond + 1) and
   grad_cond[b,c] = sum over hw of g2 * in.  Replaces the pair
   launch_activation_backward + launch_spatial_modulate_backward
   (src/cond_conv_residual.c:46-49).  `workspace` (may be NULL: library scratch)
   holds nnhip_spatial_reduce_workspace(b, H*W, C) floats for some b >= batch. */
void launch_spatial_modulate_act_backward(float* grad_in, float* grad_cond,
    const float* grad_out, const float* in, const float* cond,
    int batch, int H, int W, int C, Activation act, float* workspace, hipStream_t s);

/* NHWC convolution forward as an implicit GEMM on the matrix cores: the
   im2col matrix is gathered tile by tile from x, never written.  Replaces the
   reference's launch_im2col + gemm_forward + launch_add_bias /
   launch_scale_by_scalar (src/conv2d.c:17-34).  Wt is the reference's
   [K*K*C_in, C_out] weight, read as it is; y [batch*H_out*W_out, C_out] =
   conv + bias[n] (bias non-NULL) or conv * gain[0] (gain non-NULL) or conv.
   Needs C_in % 32 == 0 and C_out % 64 == 0 (nnhip_conv2d_implicit_supported);
   x and Wt 16-byte aligned. */
void launch_conv2d_forward_implicit(float* y, const float* x, const float* Wt, const float* bias,
    const float* gain, int batch, int H, int W, int C_in, int C_out, int K, int stride, int pad,
    int H_out, int W_out, hipStream_t s);
int nnhip_conv2d_implicit_supported(int C_in, int C_out);
/* Convolution weight gradient as an implicit GEMM on the matrix cores:
   gW [K*K*C_in, C_out] = im2col(x)^T dy (overwritten), the im2col matrix
   gathered from x tile by tile.  Replaces the reference's launch_im2col +
   gemm_dW (src/conv2d.c:44-47).  The reduction over the batch*H_out*W_out
   rows is split over workgroups and the partials are added in a fixed order
   (`workspace` of nnhip_conv2d_wgrad_workspace floats, or NULL: library
   scratch).  Needs C_in % 4 == 0 and C_out % 64 == 0; x, dy 16-byte aligned. */
void launch_conv2d_weight_grad_implicit(float* gW, const float* x, const float* dy, int batch, int H,
    int W, int C_in, int C_out, int K, int stride, int pad, int H_out, int W_out, float* workspace,
    hipStream_t s);
int nnhip_conv2d_wgrad_implicit_supported(int C_in, int C_out);
size_t nnhip_conv2d_wgrad_workspace(int batch, int C_in, int C_out, int K, int H_out, int W_out);

/* Input gradient of a stride-1 convolution as an implicit GEMM on the
   matrix cores: dx [batch, H, W, C_in] (overwritten) = the convolution of dy
   [batch, H_out, W_out, C_out] (H_out = H + 2 pad - K + 1) with the kernel of
   the [K*K*C_in, C_out] weight Wt flipped and padding K-1-pad, times gain[0]
   when gain is non-NULL.  Replaces the reference's gemm_dX +
   cudaMemsetAsync + launch_col2im (src/conv2d.c:48-65) for stride 1.  Needs
   pad <= K-1, C_out % 32 == 0 and C_in % 64 == 0
   (nnhip_conv2d_input_grad_implicit_supported); dy and Wt 16-byte aligned. */
void launch_conv2d_input_grad_implicit(float* dx, const float* dy, const float* Wt, const float* gain,
    int batch, int H, int W, int C_in, int C_out, int K, int pad, hipStream_t s);
int nnhip_conv2d_input_grad_implicit_supported(int C_in, int C_out, int K, int stride, int pad);

/* A neighbouring pass folded into an implicit-GEMM convolution kernel, so
   that the tensor between the two is neither stored nor read back.  Each
   fused form computes with the operation order of the pass it replaces, so
   its results are those of the separate launches bit for bit.  Members that a
   launcher does not take must be zero/NULL.
     res, res_w, out_w: y = res_w * res + out_w * y, res shaped as y
       (the block's launch_weighted_sum(y, res, y, res_w, out_w): mp_sum,
       residual add; src/cond_conv_residual.c:35, 61, src/conv_residual.c:39, 65).
     cond, y2, act (forward): y2 = act(y * (cond[b, c] + 1)) besides y
       (launch_spatial_modulate_act_forward after the convolution,
       src/cond_conv_residual.c:31-33); act ACT_SILU or ACT_MP_SILU.
     act_in, act (input gradient): dx = dx * act'(act_in) before the residual
       (launch_activation_backward, src/cond_conv_residual.c:54). */
typedef struct NnConvFusion {
    const float* res;
    float res_w, out_w;
    const float* cond;
    float* y2;
    const float* act_in;
    Activation act;
} NnConvFusion;

/* launch_conv2d_forward_implicit with a fused epilogue: exactly one of
   f->res (residual) and f->cond (modulate + activation into f->y2). */
void launch_conv2d_forward_implicit_fused(float* y, const float* x, const float* Wt, const float* bias,
    const float* gain, int batch, int H, int W, int C_in, int C_out, int K, int stride, int pad,
    int H_out, int W_out, const NnConvFusion* f, hipStream_t s);
/* launch_conv2d_input_grad_implicit with f->act_in and f->res (the EDM
   block's conv0); act_in and res are [batch, H, W, C_in] as dx. */
void launch_conv2d_input_grad_implicit_fused(float* dx, const float* dy, const float* Wt, const float* gain,
    int batch, int H, int W, int C_in, int C_out, int K, int pad, const NnConvFusion* f, hipStream_t s);
/* launch_spatial_reduce_sum with a lent workspace (may be NULL). */
void launch_spatial_reduce_sum_ws(float* out, const float* in, int batch, int HW, int C,
    float* workspace, hipStream_t s);
/* Floats of workspace for the two launchers above, enough for every batch up
   to `batch` at the same HW and C (0 when none needs one). */
size_t nnhip_spatial_reduce_workspace(int batch, int HW, int C);

/* y = act(GroupNorm(x)) in one HBM pass over x.  Replaces the caller sequence
   launch_groupnorm_forward + launch_activation_forward (src/conv_residual.c:28-29,
   35-36); only the activated output is written. */
void launch_groupnorm_act_forward(float* y, float* mu, float* rstd,
    const float* x, const float* gamma, const float* beta,
    int batch, int HW, int C, int G, float eps, Activation act, hipStream_t s);

/* Backward of launch_groupnorm_act_forward.  dy is the gradient of the
   activated output; the pre-activation is recomputed from x, mu, rstd, gamma,
   beta.  Replaces launch_activation_backward + launch_groupnorm_backward
   (src/conv_residual.c:51-52, 62-63).  ggamma/gbeta are overwritten. */
void launch_groupnorm_act_backward(float* dx, float* ggamma, float* gbeta,
    const float* dy, const float* x, const float* gamma, const float* beta,
    const float* mu, const float* rstd,
    int batch, int HW, int C, int G, Activation act, hipStream_t s);

/* Number of floats of device workspace that the *_ws variants need (0 when a
   shape needs none). */
size_t nnhip_groupnorm_forward_workspace(int batch, int HW, int C, int G);
size_t nnhip_groupnorm_backward_workspace(int batch, int HW, int C, int G);
size_t nnhip_layernorm_backward_workspace(int batch, int C);

/* Workspace variants: identical results; the caller lends `workspace` (at least
   the size reported above, 16-byte aligned, zero-filled before first use)
   instead of the launcher drawing it from the stream-ordered pool.  Launches
   that may run concurrently need separate workspaces.  Used by the host
   modules and the benchmark. */
void launch_groupnorm_act_forward_ws(float* y, float* mu, float* rstd,
    const float* x, const float* gamma, const float* beta,
    int batch, int HW, int C, int G, float eps, Activation act,
    float* workspace, hipStream_t s);
void launch_groupnorm_act_backward_ws(float* dx, float* ggamma, float* gbeta,
    const float* dy, const float* x, const float* gamma, const float* beta,
    const float* mu, const float* rstd,
    int batch, int HW, int C, int G, Activation act,
    float* workspace, hipStream_t s);
void launch_layernorm_backward_ws(float* grad_in, float* ggamma, float* gbeta,
    const float* grad_out, const float* x, const float* gamma,
    const float* mu, const float* rstd,
    int batch, int C, float* workspace, hipStream_t s);

/* y = act(GroupNorm(x + shift[b, c])): the DDPM block's broadcast add of the
   embedding projection folded into the GroupNorm that reads it.  Replaces
   launch_spatial_add + launch_groupnorm_forward + launch_activation_forward
   (src/conv_residual.c:34-37); x is not modified and x + shift is not stored
   (each element is the same single fp32 sum the add would store).
   `workspace` as for launch_groupnorm_act_forward_ws
   (nnhip_groupnorm_forward_workspace floats); required. */
void launch_groupnorm_act_shift_forward_ws(float* y, float* mu, float* rstd,
    const float* x, const float* shift, const float* gamma, const float* beta,
    int batch, int HW, int C, int G, float eps, Activation act,
    float* workspace, hipStream_t s);
/* Backward of launch_groupnorm_act_shift_forward_ws: dx = the gradient of
   x + shift (hence of x), gshift[b, c] = the sum over the pixels of dx,
   ggamma/gbeta, all overwritten.  Replaces launch_activation_backward +
   launch_groupnorm_backward + launch_spatial_reduce_sum
   (src/conv_residual.c:51-55).  gshift is summed in a fixed order that differs
   from launch_spatial_reduce_sum's (per 64-pixel tile, then over the tiles);
   dx, ggamma and gbeta are those of launch_groupnorm_act_backward on
   x + shift.  `workspace` holds nnhip_groupnorm_shift_backward_workspace
   floats; required. */
void launch_groupnorm_act_shift_backward_ws(float* dx, float* gshift, float* ggamma, float* gbeta,
    const float* dy, const float* x, const float* shift, const float* gamma, const float* beta,
    const float* mu, const float* rstd,
    int batch, int HW, int C, int G, Activation act,
    float* workspace, hipStream_t s);
/* The two shift launchers run persistent fused kernels only, and allocate
   nothing.  They take SiLU on 16-byte aligned pointers: the forward at 8 or
   16 channels per group, the backward at 4 (up to 2048 pixels) or 8 or 16 (up
   to 4096), where the GroupNorm path policy picks the streaming kernels (from
   4 Mi elements, or NNHIP_GN_PATH=stream).  Any other case is refused with an
   error and nothing is launched; the caller then adds the shift itself
   (launch_spatial_add) and uses the plain launchers, as the reference does.
   Returns bit 0 set when the forward takes the shape, bit 1 when the
   backward does (3: both). */
int nnhip_groupnorm_shift_supported(int batch, int HW, int C, int G, Activation act);
size_t nnhip_groupnorm_shift_backward_workspace(int batch, int HW, int C, int G);

/* Large GroupNorm launches use persistent workgroups that exchange per-tile
   statistics through the workspace and wait for each other with bounded
   polls.  A workspace lent to the GroupNorm launchers must be zero-filled
   before its first use and must not be written by anything else afterwards
   (records of a launch are told apart from earlier ones by a per-launch tag).
   Its first word is the timeout flag: a launch sets it when a wait exceeds its
   bound (that launch's outputs are then not valid), and no launch clears it.
   Returns that word as 1/0 (0: no streaming launch on `workspace` has timed
   out since it was zero-filled), or < 0 on a HIP error.  Synchronous (reads
   one word of device memory). */
int nnhip_groupnorm_workspace_status(const float* workspace);

/* launch_groupnorm_act_backward without any allocation (no counterpart in the
   reference).  For callers that cannot allocate device memory: code under
   HIP graph capture, tight serving loops, harnesses that forbid hipMalloc.
   Same kernels and results as launch_groupnorm_act_backward; instead of a
   pool block its partial sums live in a fixed scratch array of the library
   (16 MiB per device, held until the process ends): up to 12 MiB for the
   streaming kernels' workspace and 4 MiB for the 2*batch*C channel partials
   of the smaller-tensor paths.  The north-star shape [256, 64*64, 256], G=32,
   needs 10.5 MiB.  A larger shape is refused with an error naming the sizes
   (nnhip_get_last_error); nothing is launched then.  Every call on one device
   shares that scratch: calls that may overlap on one device (several streams
   or host threads) race and must be serialised by the caller. */
void launch_groupnorm_act_backward_noalloc(float* dx, float* ggamma, float* gbeta,
    const float* dy, const float* x, const float* gamma, const float* beta,
    const float* mu, const float* rstd,
    int batch, int HW, int C, int G, Activation act, hipStream_t s);

/* grad_im = col2im(grad_col) written, not accumulated: the same fixed order as
   launch_col2im starting from +0.0f.  Replaces the caller's memset + col2im pair
   (src/conv2d.c:61-65). */
void launch_col2im_set(float* grad_im, const float* grad_col, int batch, int H, int W,
    int C, int K, int stride, int pad, int H_out, int W_out, hipStream_t s);

/* Multi-tensor Adam (+ optional EMA) over a tensor list, one launch.
   For every tensor i: the launch_adam_step update of p/m/v from g, then, when
   ema_w1 != 0 and shadow != NULL, shadow = ema_w0*shadow + ema_w1*p_new (the
   update of src/ema.c:29-35 with ema_w0 = decay, ema_w1 = 1-decay in host
   float).  Replaces the per-tensor launch loops of src/optimizer.c:65-68 and
   src/ema.c:31-34.  The plan holds the device-side tensor table; build it once
   per parameter list. */
typedef struct {
    float* p;
    float* m;
    float* v;
    const float* g;
    float* shadow; /* NULL when no EMA shadow */
    long long n;
} NnTensorSlot;

typedef struct NnMultiTensorPlan NnMultiTensorPlan;

NnMultiTensorPlan* nnhip_multi_tensor_plan_create(const NnTensorSlot* slots, int count);
void nnhip_multi_tensor_plan_destroy(NnMultiTensorPlan* plan);

void launch_adam_ema_step(const NnMultiTensorPlan* plan,
    float lr, float beta1, float beta2, float eps, float bc1, float bc2,
    float ema_w0, float ema_w1, hipStream_t s);

/* EMA alone over the plan's tensors: shadow = w0*shadow + w1*p (one launch). */
void launch_ema_update(const NnMultiTensorPlan* plan, float w0, float w1, hipStream_t s);

#ifdef __cplusplus
}
#endif

#endif /* NN_HIP_H */
