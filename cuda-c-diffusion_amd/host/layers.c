/* layers.c -- the single-step host modules as Layer kinds: each kind is a
 * table entry (forward, backward) over the layer's arena buffers, plus a
 * constructor that requests the buffers, declares the exported parameters
 * and initialises them.
 *
 * What the reference fixes, and this keeps (reference file:line):
 *   constructors and their arguments         src/nn.h:185-198, 216-254
 *   ParamList order per module               activation none; layernorm and
 *       groupnorm (gamma, beta) src/layernorm.c:30-35, src/groupnorm.c:32-37;
 *       mp_linear (W, gain) src/mp_linear.c:41-46; linear (W, b)
 *       src/linear.c:32-37; conv2d (W, b) or (W, gain) src/conv2d.c:68-76
 *   init                                      gamma 1, beta 0; mp weights N(0,1),
 *       gain as given (src/mp_linear.c:70-76, src/conv2d.c:124-131); plain
 *       weights He normal sqrt(2/fan_in), bias 0 (src/linear.c:58-61,
 *       src/conv2d.c:133-137); mp_fourier freqs N(0, bandwidth), phases
 *       U[0,1) (src/mp_fourier.c:49-50)
 *   constants                                 eps 1e-5 (norms), 1e-4 (weight
 *       norm, src/mp_linear.c:66, src/conv2d.c:112); logf(max_period)
 *       (src/sinusoidal.c:47)
 *   launch sequences (the maths)              each kind below cites its own
 * Everything else -- one arena per module, lent workspaces so that no call
 * allocates, the fused GroupNorm+activation kind, the implicit-GEMM
 * convolution paths -- is this library's.
 */
#include <math.h>
#include <string.h>

#include "layer.h"
#include "nn_gemm.h"

/* ------------------------------------------------------------------------
 * activation (src/activation.c:8-23): one elementwise launch each way
 * ------------------------------------------------------------------------ */

static void act_fwd(Layer* L, const float* in, float* out, int batch, Context* ctx)
{
    launch_activation_forward(out, in, batch * L->mod.in_dim, L->act, ctx->stream);
}

static void act_bwd(Layer* L, const float* in, const float* out, const float* grad_out, float* grad_in, int batch,
    Context* ctx)
{
    (void)out;
    launch_activation_backward(grad_in, grad_out, in, batch * L->mod.in_dim, L->act, ctx->stream);
}

static const LayerKind kActivation = {"activation", act_fwd, act_bwd};

Module* activation_create(int dim, Activation act)
{
    Layer* L = layer_begin(&kActivation, dim, dim, 0);
    L->act = act;
    return layer_end(L);
}

/* ------------------------------------------------------------------------
 * affine norms: LayerNorm over rows (src/layernorm.c:12-28) and NHWC
 * GroupNorm with an optional fused activation (src/groupnorm.c:12-30; the
 * activation replaces the separate launches of src/conv_residual.c:28-29,
 * 51-52).  Shared buffer layout; statistics cached by the forward for the
 * backward, as in the reference.
 * ------------------------------------------------------------------------ */

enum { NB_GAMMA, NB_BETA, NB_GGAMMA, NB_GBETA, NB_MU, NB_RSTD, NB_BWS, NB_FWS, NB_RED };
enum { ND_C, ND_G, ND_HW, ND_SHIFT_MODULE, ND_SHIFT_FUSED };

static void ln_fwd(Layer* L, const float* in, float* out, int batch, Context* ctx)
{
    launch_layernorm_forward(out, L->buf[NB_MU], L->buf[NB_RSTD], in, L->buf[NB_GAMMA], L->buf[NB_BETA], batch,
        L->dim[ND_C], L->k[0], ctx->stream);
}

static void ln_bwd(Layer* L, const float* in, const float* out, const float* grad_out, float* grad_in, int batch,
    Context* ctx)
{
    (void)out;
    launch_layernorm_backward_ws(grad_in, L->buf[NB_GGAMMA], L->buf[NB_GBETA], grad_out, in, L->buf[NB_GAMMA],
        L->buf[NB_MU], L->buf[NB_RSTD], batch, L->dim[ND_C], L->buf[NB_BWS], ctx->stream);
}

static void gn_fwd(Layer* L, const float* in, float* out, int batch, Context* ctx)
{
    launch_groupnorm_act_forward_ws(out, L->buf[NB_MU], L->buf[NB_RSTD], in, L->buf[NB_GAMMA], L->buf[NB_BETA],
        batch, L->dim[ND_HW], L->dim[ND_C], L->dim[ND_G], L->k[0], L->act, L->buf[NB_FWS], ctx->stream);
}

static void gn_bwd(Layer* L, const float* in, const float* out, const float* grad_out, float* grad_in, int batch,
    Context* ctx)
{
    (void)out;
    launch_groupnorm_act_backward_ws(grad_in, L->buf[NB_GGAMMA], L->buf[NB_GBETA], grad_out, in, L->buf[NB_GAMMA],
        L->buf[NB_BETA], L->buf[NB_MU], L->buf[NB_RSTD], batch, L->dim[ND_HW], L->dim[ND_C], L->dim[ND_G], L->act,
        L->buf[NB_BWS], ctx->stream);
}

static const LayerKind kLayerNorm = {"layernorm", ln_fwd, ln_bwd};
static const LayerKind kGroupNorm = {"groupnorm", gn_fwd, gn_bwd};
static const LayerKind kGroupNormAct = {"groupnorm_act", gn_fwd, gn_bwd};

/* gamma, beta and their gradients, statistics of `rows` rows, the lent
   workspaces (zero-filled: their first word is the wait-timeout flag of the
   streaming GroupNorm; `red` is a spatial-reduction workspace, 0 for none).
   gamma = 1, beta = 0. */
static Module* affine_norm(Layer* L, int C, size_t rows, size_t bws, size_t fws, size_t red)
{
    L->dim[ND_C] = C;
    L->k[0] = 1e-5f;
    layer_buf(L, (size_t)C, 0);
    layer_buf(L, (size_t)C, 1);
    layer_buf(L, (size_t)C, 0);
    layer_buf(L, (size_t)C, 0);
    layer_buf(L, rows, 0);
    layer_buf(L, rows, 0);
    layer_buf(L, bws, 1);
    layer_buf(L, fws, 1);
    layer_buf(L, red, 1);
    layer_param(L, NB_GAMMA, NB_GGAMMA, C);
    layer_param(L, NB_BETA, NB_GBETA, C);
    Module* m = layer_end(L);
    layer_fill_value(L, NB_GAMMA, (size_t)C, 1.0f);
    return m;
}

Module* layernorm_create(int dim, int max_batch)
{
    Layer* L = layer_begin(&kLayerNorm, dim, dim, max_batch);
    return affine_norm(L, dim, (size_t)max_batch, nnhip_layernorm_backward_workspace(max_batch, dim), 0, 0);
}

static Module* groupnorm_make(const LayerKind* kind, int C, int num_groups, int H, int W, int max_batch,
    Activation act, int shift)
{
    NN_ASSERT(num_groups > 0 && C % num_groups == 0, "groupnorm: C must be divisible by num_groups");
    Layer* L = layer_begin(kind, H * W * C, H * W * C, max_batch);
    L->act = act;
    L->dim[ND_G] = num_groups;
    L->dim[ND_HW] = H * W;
    L->dim[ND_SHIFT_MODULE] = shift;
    /* workspaces sized for max_batch serve every smaller batch; a forward that
       needs none gets no buffer (the launcher then works without one).  A
       shift module also keeps a spatial-reduction workspace for the batches
       the fused shift kernels do not take. */
    const int HW = H * W;
    return affine_norm(L, C, (size_t)max_batch * num_groups,
        shift ? nnhip_groupnorm_shift_backward_workspace(max_batch, HW, C, num_groups)
              : nnhip_groupnorm_backward_workspace(max_batch, HW, C, num_groups),
        nnhip_groupnorm_forward_workspace(max_batch, HW, C, num_groups),
        shift ? nnhip_spatial_reduce_workspace(max_batch, HW, C) : 0);
}

Module* spatial_groupnorm_create(int C, int num_groups, int H, int W, int max_batch)
{
    return groupnorm_make(&kGroupNorm, C, num_groups, H, W, max_batch, ACT_IDENTITY, 0);
}

Module* spatial_groupnorm_act_create(int C, int num_groups, int H, int W, int max_batch, Activation act)
{
    return groupnorm_make(&kGroupNormAct, C, num_groups, H, W, max_batch, act, 0);
}

Module* spatial_groupnorm_act_shift_create(int C, int num_groups, int H, int W, int max_batch, Activation act)
{
    return groupnorm_make(&kGroupNormAct, C, num_groups, H, W, max_batch, act, 1);
}

/* The fused shift launchers when they take the batch (both directions, so
   that forward and backward agree); otherwise the reference's sequence, the
   in-place broadcast add followed by the plain module (src/conv_residual.c:34-37)
   and, backward, the plain module and the pixel sum (:53-55).  The forward
   records which one ran; the backward follows it. */
void groupnorm_shift_forward(Module* gn, float* x, const float* shift, float* y, int batch, Context* ctx)
{
    Layer* L = as_layer(gn);
    NN_ASSERT(batch <= L->max_batch, L->kind->name);
    NN_ASSERT(L->dim[ND_SHIFT_MODULE], "groupnorm_shift_forward: not a shift module");
    const int HW = L->dim[ND_HW], C = L->dim[ND_C], G = L->dim[ND_G];
    L->dim[ND_SHIFT_FUSED] = nnhip_groupnorm_shift_supported(batch, HW, C, G, L->act) == 3;
    if (L->dim[ND_SHIFT_FUSED]) {
        launch_groupnorm_act_shift_forward_ws(y, L->buf[NB_MU], L->buf[NB_RSTD], x, shift, L->buf[NB_GAMMA],
            L->buf[NB_BETA], batch, HW, C, G, L->k[0], L->act, L->buf[NB_FWS], ctx->stream);
    } else {
        launch_spatial_add(x, shift, batch, HW, 1, C, ctx->stream);
        gn_fwd(L, x, y, batch, ctx);
    }
}

void groupnorm_shift_backward(Module* gn, const float* x, const float* shift, const float* g_y, float* g_x,
    float* g_shift, int batch, Context* ctx)
{
    Layer* L = as_layer(gn);
    NN_ASSERT(batch <= L->max_batch, L->kind->name);
    NN_ASSERT(L->dim[ND_SHIFT_MODULE], "groupnorm_shift_backward: not a shift module");
    const int HW = L->dim[ND_HW], C = L->dim[ND_C], G = L->dim[ND_G];
    if (L->dim[ND_SHIFT_FUSED]) {
        launch_groupnorm_act_shift_backward_ws(g_x, g_shift, L->buf[NB_GGAMMA], L->buf[NB_GBETA], g_y, x, shift,
            L->buf[NB_GAMMA], L->buf[NB_BETA], L->buf[NB_MU], L->buf[NB_RSTD], batch, HW, C, G, L->act,
            L->buf[NB_BWS], ctx->stream);
    } else {
        gn_bwd(L, x, NULL, g_y, g_x, batch, ctx);  /* x holds x + shift since the forward */
        launch_spatial_reduce_sum_ws(g_shift, g_x, batch, HW, C, L->buf[NB_RED], ctx->stream);
    }
}

/* ------------------------------------------------------------------------
 * dense layers around a rocBLAS GEMM (the GEMM is outside the fused path):
 *   mp_linear (src/mp_linear.c:12-39): W normalised in place every forward,
 *     Y = X W * gain; backward gW = X^T dY, g_gain zeroed then accumulated,
 *     gW projected and scaled, dX = dY W^T * gain;
 *   linear (src/linear.c:12-30): Y = X W + b; gW = X^T dY, gb = column sums,
 *     dX = dY W^T.
 * ------------------------------------------------------------------------ */

enum { DB_W, DB_GW, DB_AUX, DB_GAUX, DB_WNWS };
enum { DD_IN, DD_OUT };

static void mpl_fwd(Layer* L, const float* in, float* out, int batch, Context* ctx)
{
    const int ni = L->dim[DD_IN], no = L->dim[DD_OUT];
    launch_weight_normalize(L->buf[DB_W], ni, no, L->k[0], ctx->stream);
    nn_gemm_forward(ctx->blas, 1.0f, in, L->buf[DB_W], out, batch, ni, no);
    launch_scale_by_scalar(out, L->buf[DB_AUX], batch * no, ctx->stream);
}

static void mpl_bwd(Layer* L, const float* in, const float* out, const float* grad_out, float* grad_in, int batch,
    Context* ctx)
{
    (void)out;
    const int ni = L->dim[DD_IN], no = L->dim[DD_OUT];
    nn_gemm_dW(ctx->blas, 1.0f, in, grad_out, L->buf[DB_GW], batch, ni, no);
    nnhip_fill_f32(L->buf[DB_GAUX], 0.0f, 1, ctx->stream);
    launch_weight_normalize_backward_ws(L->buf[DB_GW], L->buf[DB_W], L->buf[DB_AUX], L->buf[DB_GAUX], ni, no,
        L->buf[DB_WNWS], ctx->stream);
    if (!grad_in) return;
    nn_gemm_dX(ctx->blas, 1.0f, L->buf[DB_W], grad_out, grad_in, batch, ni, no);
    launch_scale_by_scalar(grad_in, L->buf[DB_AUX], batch * ni, ctx->stream);
}

static void lin_fwd(Layer* L, const float* in, float* out, int batch, Context* ctx)
{
    const int ni = L->dim[DD_IN], no = L->dim[DD_OUT];
    nn_gemm_forward(ctx->blas, 1.0f, in, L->buf[DB_W], out, batch, ni, no);
    launch_add_bias(out, L->buf[DB_AUX], batch, no, ctx->stream);
}

static void lin_bwd(Layer* L, const float* in, const float* out, const float* grad_out, float* grad_in, int batch,
    Context* ctx)
{
    (void)out;
    const int ni = L->dim[DD_IN], no = L->dim[DD_OUT];
    nn_gemm_dW(ctx->blas, 1.0f, in, grad_out, L->buf[DB_GW], batch, ni, no);
    launch_bias_grad(L->buf[DB_GAUX], grad_out, batch, no, ctx->stream);
    if (grad_in) nn_gemm_dX(ctx->blas, 1.0f, L->buf[DB_W], grad_out, grad_in, batch, ni, no);
}

static const LayerKind kMpLinear = {"mp_linear", mpl_fwd, mpl_bwd};
static const LayerKind kLinear = {"linear", lin_fwd, lin_bwd};

/* W [in, out] and its gradient, then the per-output-layer term (gain [1] or
   bias [out]) and its gradient; the weight-norm workspace in mp mode. */
static Layer* dense(const LayerKind* kind, int in_dim, int out_dim, int aux_n, size_t wn_ws)
{
    Layer* L = layer_begin(kind, in_dim, out_dim, 0);
    L->dim[DD_IN] = in_dim;
    L->dim[DD_OUT] = out_dim;
    const size_t nw = (size_t)in_dim * out_dim;
    layer_buf(L, nw, 0);
    layer_buf(L, nw, 0);
    layer_buf(L, (size_t)aux_n, 1);
    layer_buf(L, (size_t)aux_n, 0);
    layer_buf(L, wn_ws, 1);
    layer_param(L, DB_W, DB_GW, (int)nw);
    layer_param(L, DB_AUX, DB_GAUX, aux_n);
    return L;
}

Module* mp_linear_create(Context* ctx, int in_dim, int out_dim, float gain)
{
    Layer* L = dense(&kMpLinear, in_dim, out_dim, 1, nnhip_weight_normalize_backward_workspace(out_dim));
    L->k[0] = 1e-4f;
    Module* m = layer_end(L);
    nn_fill_normal(ctx, L->buf[DB_W], (size_t)in_dim * out_dim, 0.0f, 1.0f);
    layer_fill_value(L, DB_AUX, 1, gain);
    return m;
}

Module* linear_create(Context* ctx, int in_dim, int out_dim)
{
    Layer* L = dense(&kLinear, in_dim, out_dim, out_dim, 0);
    Module* m = layer_end(L);
    nn_fill_normal(ctx, L->buf[DB_W], (size_t)in_dim * out_dim, 0.0f, sqrtf(2.0f / (float)in_dim));
    return m;
}

/* ------------------------------------------------------------------------
 * embeddings, forward only (their backward is a no-op in the reference,
 * src/mp_fourier.c:16-28, src/sinusoidal.c:17-29):
 *   mp_fourier (src/mp_fourier.c:9-14), sinusoidal (src/sinusoidal.c:10-15)
 * ------------------------------------------------------------------------ */

enum { EB_FREQ, EB_PHASE };

static void fourier_fwd(Layer* L, const float* in, float* out, int batch, Context* ctx)
{
    launch_mp_fourier(out, in, L->buf[EB_FREQ], L->buf[EB_PHASE], batch, L->mod.out_dim, ctx->stream);
}

static void sinusoidal_fwd(Layer* L, const float* in, float* out, int batch, Context* ctx)
{
    launch_sinusoidal(out, in, batch, L->mod.out_dim, L->k[0], ctx->stream);
}

static const LayerKind kMpFourier = {"mp_fourier", fourier_fwd, NULL};
static const LayerKind kSinusoidal = {"sinusoidal", sinusoidal_fwd, NULL};

Module* mp_fourier_create(Context* ctx, int num_channels, float bandwidth)
{
    Layer* L = layer_begin(&kMpFourier, 1, num_channels, 0);
    layer_buf(L, (size_t)num_channels, 0);
    layer_buf(L, (size_t)num_channels, 0);
    Module* m = layer_end(L);
    nn_fill_normal(ctx, L->buf[EB_FREQ], (size_t)num_channels, 0.0f, bandwidth);
    nn_fill_uniform(ctx, L->buf[EB_PHASE], (size_t)num_channels);
    return m;
}

Module* sinusoidal_create(int num_channels, float max_period)
{
    NN_ASSERT(num_channels % 2 == 0, "sinusoidal_create: num_channels must be even");
    Layer* L = layer_begin(&kSinusoidal, 1, num_channels, 0);
    L->k[0] = logf(max_period);
    return layer_end(L);
}

/* ------------------------------------------------------------------------
 * conv2d, NHWC, plain (bias) or magnitude-preserving (forced weight norm and
 * gain), weights [K*K*C_in, C_out] row-major (src/conv2d.c:17-66).
 * Forward: the implicit-GEMM kernel on the matrix cores when the channel
 * counts allow it (C_in % 32 == 0, C_out % 64 == 0), bias or gain in its
 * epilogue; otherwise im2col + rocBLAS + the bias/gain pass, as the
 * reference.  Backward: the weight gradient as an implicit GEMM (C_in % 4,
 * C_out % 64), the stride-1 input gradient as the implicit convolution of
 * grad_out with the flipped kernel (C_out % 32, C_in % 64); otherwise
 * im2col + rocBLAS and the gather col2im, which needs no memset of grad_in.
 * The implicit kernels read the weight in its own layout.
 * NNHIP_CONV_PATH=gemm forces the reference's sequence.  Its im2col matrix
 * (max_batch * H_out * W_out * K*K*C_in floats, 604 MB at cfg3) is allocated
 * only for a path the implicit kernels do not take, or when the variable is
 * set as the module is created; forcing the sequence later is refused.
 * ------------------------------------------------------------------------ */

enum { CB_W, CB_GW, CB_AUX, CB_GAUX, CB_COL, CB_WGWS, CB_WNWS };
enum { CD_CIN, CD_COUT, CD_K, CD_S, CD_P, CD_HI, CD_WI, CD_HO, CD_WO, CD_MP, CD_FWD, CD_WGRAD, CD_DGRAD };

static int conv_gemm_forced(void)
{
    const char* e = getenv("NNHIP_CONV_PATH");
    return e && strcmp(e, "gemm") == 0;
}

static int conv_implicit_forced(void)
{
    const char* e = getenv("NNHIP_CONV_PATH");
    return e && strcmp(e, "implicit") == 0;
}

/* Whether the implicit-GEMM kernel (igemm_fwd: the forward, and the stride-1
   input gradient) beats im2col + rocBLAS for an M x N x K product, by a cost
   model fitted on MI355X.  A 128 x BN output tile takes ~2.25 us per 32-deep k
   slice with one workgroup per CU (cfg3's forward: 36 slices, 1024 tiles,
   four tiles per CU: 320 us), so few tiles leave the device idle: at the
   reference DDPM's 7 x 7 x 128 level (M = 392 at batch 8, 4 tiles) the kernel
   takes ~83 us where the GEMM path takes ~10.  The GEMM path: ~10 us of fixed
   cost, the GEMM at ~70 TFLOP/s (rocBLAS fp32, measured at cfg3) and the
   im2col matrix written and read at ~6 TB/s. */
static int conv_implicit_wins(long long M, int N, int K)
{
    const int bn = N % 128 == 0 ? 128 : 64;
    const double tiles = (double)((M + 127) / 128) * ((N + bn - 1) / bn);
    const double t_impl = (K / 32.0) * 2.25 * ceil(tiles / 256.0);
    const double t_gemm = 10.0 + 2.0 * (double)M * N * K / 70e6 + 8.0 * (double)M * K / 6e6;
    return t_impl <= t_gemm;
}

/* the reference's sequence asked for at this call (needs the im2col buffer) */
static int conv_gemm_path(const Layer* L)
{
    if (!conv_gemm_forced()) return 0;
    NN_ASSERT(L->buf[CB_COL], "conv2d: NNHIP_CONV_PATH=gemm must be set when the module is created "
                              "(its im2col buffer is allocated then)");
    return 1;
}

/* The implicit-GEMM kernels take 128-bit loads of the activations they
   gather; a misaligned tensor would make them refuse and leave the output
   unwritten, so the module stops with a message instead. */
static void conv_require_aligned(const float* p, const char* what)
{
    if (((uintptr_t)p & 15u) != 0) {
        fprintf(stderr, "conv2d: %s at %p is not 16-byte aligned (the implicit-GEMM path needs it)\n", what,
            (const void*)p);
        exit(1);
    }
}

static void conv_fwd(Layer* L, const float* in, float* out, int batch, Context* ctx)
{
    const int* d = L->dim;
    const int kg = d[CD_K] * d[CD_K] * d[CD_CIN], rows = batch * d[CD_HO] * d[CD_WO];
    float *w = L->buf[CB_W], *aux = L->buf[CB_AUX];
    if (d[CD_MP]) launch_weight_normalize(w, kg, d[CD_COUT], L->k[0], ctx->stream);
    if (d[CD_FWD] && !conv_gemm_path(L)) {
        conv_require_aligned(in, "the forward input");
        launch_conv2d_forward_implicit(out, in, w, d[CD_MP] ? NULL : aux, d[CD_MP] ? aux : NULL, batch,
            d[CD_HI], d[CD_WI], d[CD_CIN], d[CD_COUT], d[CD_K], d[CD_S], d[CD_P], d[CD_HO], d[CD_WO], ctx->stream);
        return;
    }
    launch_im2col(L->buf[CB_COL], in, batch, d[CD_HI], d[CD_WI], d[CD_CIN], d[CD_K], d[CD_S], d[CD_P], d[CD_HO],
        d[CD_WO], ctx->stream);
    nn_gemm_forward(ctx->blas, 1.0f, L->buf[CB_COL], w, out, rows, kg, d[CD_COUT]);
    if (d[CD_MP]) launch_scale_by_scalar(out, aux, rows * d[CD_COUT], ctx->stream);
    else launch_add_bias(out, aux, rows, d[CD_COUT], ctx->stream);
}

static void conv_bwd(Layer* L, const float* in, const float* out, const float* grad_out, float* grad_in, int batch,
    Context* ctx)
{
    (void)out;
    const int* d = L->dim;
    const int kg = d[CD_K] * d[CD_K] * d[CD_CIN], rows = batch * d[CD_HO] * d[CD_WO];
    const int forced = conv_gemm_path(L);
    float *w = L->buf[CB_W], *gw = L->buf[CB_GW], *col = L->buf[CB_COL];
    if (d[CD_WGRAD] && !forced) {
        conv_require_aligned(in, "the forward input");
        conv_require_aligned(grad_out, "the output gradient");
        launch_conv2d_weight_grad_implicit(gw, in, grad_out, batch, d[CD_HI], d[CD_WI], d[CD_CIN], d[CD_COUT],
            d[CD_K], d[CD_S], d[CD_P], d[CD_HO], d[CD_WO], L->buf[CB_WGWS], ctx->stream);
    } else {
        launch_im2col(col, in, batch, d[CD_HI], d[CD_WI], d[CD_CIN], d[CD_K], d[CD_S], d[CD_P], d[CD_HO], d[CD_WO],
            ctx->stream);
        nn_gemm_dW(ctx->blas, 1.0f, col, grad_out, gw, rows, kg, d[CD_COUT]);
    }
    if (d[CD_MP]) {
        nnhip_fill_f32(L->buf[CB_GAUX], 0.0f, 1, ctx->stream);
        launch_weight_normalize_backward_ws(gw, w, L->buf[CB_AUX], L->buf[CB_GAUX], kg, d[CD_COUT],
            L->buf[CB_WNWS], ctx->stream);
    } else {
        launch_bias_grad(L->buf[CB_GAUX], grad_out, rows, d[CD_COUT], ctx->stream);
    }
    if (!grad_in) return;
    const float* gain = d[CD_MP] ? L->buf[CB_AUX] : NULL;
    if (d[CD_DGRAD] && !forced) {
        /* stride 1: dx = conv(dy, flipped kernel, pad K-1-pad), times the gain in mp mode */
        conv_require_aligned(grad_out, "the output gradient");
        launch_conv2d_input_grad_implicit(grad_in, grad_out, w, gain, batch, d[CD_HI], d[CD_WI], d[CD_CIN],
            d[CD_COUT], d[CD_K], d[CD_P], ctx->stream);
        return;
    }
    nn_gemm_dX(ctx->blas, 1.0f, w, grad_out, col, rows, kg, d[CD_COUT]);
    if (gain) launch_scale_by_scalar(col, gain, rows * kg, ctx->stream);
    launch_col2im_set(grad_in, col, batch, d[CD_HI], d[CD_WI], d[CD_CIN], d[CD_K], d[CD_S], d[CD_P], d[CD_HO],
        d[CD_WO], ctx->stream);
}

static const LayerKind kConv2d = {"conv2d", conv_fwd, conv_bwd};

/* The convolution with a neighbouring pass of the diffusion blocks folded into
   its implicit-GEMM kernels (launch_conv2d_*_implicit_fused), so that the
   tensor between the two never goes through HBM.  Where the implicit kernels
   do not take the convolution (channel counts, NNHIP_CONV_PATH=gemm), the
   module's own forward/backward runs and the pass follows as a launch of its
   own, the reference's sequence.  The results are the same either way. */

static int conv_fused_fwd(const Layer* L) { return L->dim[CD_FWD] && !conv_gemm_path(L); }
static int conv_fused_bwd(const Layer* L) { return L->dim[CD_WGRAD] && L->dim[CD_DGRAD] && !conv_gemm_path(L); }

static void conv_fused_forward(Layer* L, const float* in, float* out, int batch, const NnConvFusion* f, Context* ctx)
{
    const int* d = L->dim;
    float *w = L->buf[CB_W], *aux = L->buf[CB_AUX];
    if (d[CD_MP]) launch_weight_normalize(w, d[CD_K] * d[CD_K] * d[CD_CIN], d[CD_COUT], L->k[0], ctx->stream);
    conv_require_aligned(in, "the forward input");
    launch_conv2d_forward_implicit_fused(out, in, w, d[CD_MP] ? NULL : aux, d[CD_MP] ? aux : NULL, batch, d[CD_HI],
        d[CD_WI], d[CD_CIN], d[CD_COUT], d[CD_K], d[CD_S], d[CD_P], d[CD_HO], d[CD_WO], f, ctx->stream);
}

void conv2d_forward_residual(Module* m, const float* in, float* out, const float* res, float res_w, float out_w,
    int batch, Context* ctx)
{
    Layer* L = as_layer(m);
    const int* d = L->dim;
    if (!conv_fused_fwd(L)) {
        conv_fwd(L, in, out, batch, ctx);
        launch_weighted_sum(out, res, out, res_w, out_w, batch * d[CD_HO] * d[CD_WO] * d[CD_COUT], ctx->stream);
        return;
    }
    NnConvFusion f;
    memset(&f, 0, sizeof f);
    f.res = res;
    f.res_w = res_w;
    f.out_w = out_w;
    conv_fused_forward(L, in, out, batch, &f, ctx);
}

void conv2d_forward_modulate_act(Module* m, const float* in, float* out, float* out2, const float* cond,
    Activation act, int batch, Context* ctx)
{
    Layer* L = as_layer(m);
    const int* d = L->dim;
    if (!conv_fused_fwd(L) || (act != ACT_SILU && act != ACT_MP_SILU)) {
        conv_fwd(L, in, out, batch, ctx);
        launch_spatial_modulate_act_forward(out2, out, cond, batch, d[CD_HO] * d[CD_WO], 1, d[CD_COUT], act,
            ctx->stream);
        return;
    }
    NnConvFusion f;
    memset(&f, 0, sizeof f);
    f.cond = cond;
    f.y2 = out2;
    f.act = act;
    conv_fused_forward(L, in, out, batch, &f, ctx);
}

void conv2d_backward_act_residual(Module* m, const float* in, const float* grad_out, float* grad_in,
    const float* act_in, Activation act, const float* res, float res_w, float* tmp, int batch, Context* ctx)
{
    Layer* L = as_layer(m);
    const int* d = L->dim;
    const int n_in = batch * d[CD_HI] * d[CD_WI] * d[CD_CIN];
    if (!conv_fused_bwd(L) || (act != ACT_SILU && act != ACT_MP_SILU)) {
        conv_bwd(L, in, NULL, grad_out, tmp, batch, ctx);
        launch_activation_backward(grad_in, tmp, act_in, n_in, act, ctx->stream);
        launch_weighted_sum(grad_in, res, grad_in, res_w, 1.0f, n_in, ctx->stream);
        return;
    }
    NN_ASSERT(grad_in != grad_out, "conv2d_backward_act_residual: grad_in must not alias grad_out");
    conv_bwd(L, in, NULL, grad_out, NULL, batch, ctx); /* parameter gradients */
    NnConvFusion f;
    memset(&f, 0, sizeof f);
    f.act_in = act_in;
    f.act = act;
    f.res = res;
    f.res_w = res_w;
    f.out_w = 1.0f;
    conv_require_aligned(grad_out, "the output gradient");
    launch_conv2d_input_grad_implicit_fused(grad_in, grad_out, L->buf[CB_W], d[CD_MP] ? L->buf[CB_AUX] : NULL, batch,
        d[CD_HI], d[CD_WI], d[CD_CIN], d[CD_COUT], d[CD_K], d[CD_P], &f, ctx->stream);
}

Module* conv2d_create(Context* ctx, int C_in, int C_out, int K, int stride, int pad, int H, int W, int max_batch,
    int mp_mode, float gain)
{
    const int Ho = (H + 2 * pad - K) / stride + 1, Wo = (W + 2 * pad - K) / stride + 1;
    const int kg = K * K * C_in;
    const size_t nw = (size_t)kg * C_out;
    Layer* L = layer_begin(&kConv2d, H * W * C_in, Ho * Wo * C_out, max_batch);
    int* d = L->dim;
    d[CD_CIN] = C_in;
    d[CD_COUT] = C_out;
    d[CD_K] = K;
    d[CD_S] = stride;
    d[CD_P] = pad;
    d[CD_HI] = H;
    d[CD_WI] = W;
    d[CD_HO] = Ho;
    d[CD_WO] = Wo;
    d[CD_MP] = mp_mode != 0;
    /* the implicit kernels where the channel counts allow them and, for the
       forward and input gradient, where they beat the GEMM path at max_batch
       (NNHIP_CONV_PATH=implicit at creation: wherever allowed) */
    const int forced = conv_implicit_forced();
    d[CD_FWD] = nnhip_conv2d_implicit_supported(C_in, C_out) &&
                (forced || conv_implicit_wins((long long)max_batch * Ho * Wo, C_out, kg));
    d[CD_WGRAD] = nnhip_conv2d_wgrad_implicit_supported(C_in, C_out);
    d[CD_DGRAD] = nnhip_conv2d_input_grad_implicit_supported(C_in, C_out, K, stride, pad) &&
                  (forced || conv_implicit_wins((long long)max_batch * H * W, C_in, K * K * C_out));
    L->k[0] = 1e-4f;
    const int aux_n = mp_mode ? 1 : C_out;
    layer_buf(L, nw, 0);
    layer_buf(L, nw, 0);
    layer_buf(L, (size_t)aux_n, 1);
    layer_buf(L, (size_t)aux_n, 0);
    /* the im2col matrix, for the paths the implicit kernels do not take */
    const int need_col = !d[CD_FWD] || !d[CD_WGRAD] || !d[CD_DGRAD] || conv_gemm_forced();
    layer_buf(L, need_col ? (size_t)max_batch * Ho * Wo * kg : 0, 0);
    layer_buf(L, d[CD_WGRAD] ? nnhip_conv2d_wgrad_workspace(max_batch, C_in, C_out, K, Ho, Wo) : 0, 0);
    layer_buf(L, mp_mode ? nnhip_weight_normalize_backward_workspace(C_out) : 0, 1);
    layer_param(L, CB_W, CB_GW, (int)nw);
    layer_param(L, CB_AUX, CB_GAUX, aux_n);
    Module* m = layer_end(L);
    nn_fill_normal(ctx, L->buf[CB_W], nw, 0.0f, mp_mode ? 1.0f : sqrtf(2.0f / (float)kg));
    if (mp_mode) layer_fill_value(L, CB_AUX, 1, gain);
    return m;
}
