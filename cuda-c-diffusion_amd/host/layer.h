/* layer.h -- the record behind every host module of this library.
 *
 * A Layer is what a Module* points at: the Module vtable the callers use is its
 * first member, and the four vtable entries are the same for every kind (they
 * dispatch through the kind's table entry).  All device memory a layer owns
 * (parameters, their gradients, cached statistics, lent workspaces, scratch)
 * is carved out of ONE device allocation, the arena, described by a list of
 * buffer requests made at construction time; the ParamList entries are
 * (value buffer, gradient buffer, size) triples in the order the module
 * exports them, and composite layers own child modules whose parameters
 * follow the layer's own.
 *
 * Construction: layer_begin -> layer_buf / layer_param / layer_sub ->
 * layer_end, which makes the single allocation, zero-fills the buffers asked
 * for zeroed and wires the vtable.  Only after layer_end are the buffers
 * addressable (L->buf[i]).
 */
#ifndef NN_LAYER_H
#define NN_LAYER_H

#include "nn_modules.h"

#define LAYER_MAX_BUFS 16
#define LAYER_MAX_PARAMS 3
#define LAYER_MAX_SUBS 6
#define LAYER_MAX_DIMS 16

typedef struct Layer Layer;

typedef struct {
    const char* name;
    void (*fwd)(Layer* L, const float* in, float* out, int batch, Context* ctx);
    void (*bwd)(Layer* L, const float* in, const float* out, const float* grad_out, float* grad_in,
        int batch, Context* ctx);
} LayerKind;

struct Layer {
    Module mod; /* must stay first: a Module* of this library is a Layer* */
    const LayerKind* kind;
    int max_batch;
    int dim[LAYER_MAX_DIMS]; /* the kind's geometry, indexed by the kind's own enum */
    float k[4];              /* the kind's constants (eps, blend weights, ...) */
    Activation act;
    /* device buffers: requests, then the carved views */
    int nbuf;
    size_t want[LAYER_MAX_BUFS];
    unsigned char zero[LAYER_MAX_BUFS];
    float* buf[LAYER_MAX_BUFS];
    float* arena;
    /* ParamList export */
    int nparam;
    int pval[LAYER_MAX_PARAMS], pgrad[LAYER_MAX_PARAMS], pn[LAYER_MAX_PARAMS];
    /* owned child modules, exported after this layer's own parameters */
    int nsub;
    Module* sub[LAYER_MAX_SUBS];
};

/* Start a layer of `kind` with the Module's in/out dimensions. */
Layer* layer_begin(const LayerKind* kind, int in_dim, int out_dim, int max_batch);
/* Request a device buffer of `floats` floats (0: none, its view stays NULL);
   zero != 0 zero-fills it at layer_end.  Returns its index. */
int layer_buf(Layer* L, size_t floats, int zero);
/* Export (value, gradient) buffers of n floats as the next ParamList entry. */
void layer_param(Layer* L, int value_buf, int grad_buf, int n);
/* Take ownership of a child module (freed with the layer). */
void layer_sub(Layer* L, Module* child);
/* Allocate and carve the arena, zero-fill the buffers asked for, wire the
   vtable; returns the Module callers hold. */
Module* layer_end(Layer* L);

static inline Layer* as_layer(Module* m) { return (Layer*)m; }

/* Host-to-device fill of a buffer with one value (construction time). */
void layer_fill_value(Layer* L, int b, size_t n, float value);

/* A fused GroupNorm+activation layer whose input may carry a per-(sample,
   channel) shift: an ordinary spatial_groupnorm_act module (same parameters,
   ParamList and vtable) whose workspaces also fit the shift path.
   groupnorm_shift_forward / _backward run it on x + shift[b, c] (shift
   [batch, C]): y = act(GN(x + shift)); g_x = the gradient of x + shift,
   g_shift[b, c] = its sum over the pixels (both overwritten; the parameter
   gradients too, as in the plain backward).  Where the fused shift kernels
   take the batch, x + shift is formed in registers and x is left as it is;
   elsewhere the forward adds the shift into x in place, as the reference
   block does.  Either way the backward must be given the same x, shift and
   batch as the most recent forward. */
Module* spatial_groupnorm_act_shift_create(int C, int num_groups, int H, int W, int max_batch, Activation act);
void groupnorm_shift_forward(Module* gn, float* x, const float* shift, float* y, int batch, Context* ctx);
void groupnorm_shift_backward(Module* gn, const float* x, const float* shift, const float* g_y, float* g_x,
    float* g_shift, int batch, Context* ctx);

/* conv2d modules (conv2d_create) with the pass that follows them in the
   diffusion blocks folded into their kernels where the implicit-GEMM path
   takes them (elsewhere the module runs and the pass follows as its own
   launch, the reference's sequence):
     conv2d_forward_residual:     out = res_w * res + out_w * conv(in)
     conv2d_forward_modulate_act: out = conv(in), out2 = act(out * (cond[b, c] + 1))
     conv2d_backward_act_residual: parameter gradients, and
                                  grad_in = res_w * res + (dx * act'(act_in))
   `tmp` holds the unfused path's intermediate (the module's input size);
   act is ACT_SILU or ACT_MP_SILU for the fused kernels. */
void conv2d_forward_residual(Module* m, const float* in, float* out, const float* res, float res_w, float out_w,
    int batch, Context* ctx);
void conv2d_forward_modulate_act(Module* m, const float* in, float* out, float* out2, const float* cond,
    Activation act, int batch, Context* ctx);
void conv2d_backward_act_residual(Module* m, const float* in, const float* grad_out, float* grad_in,
    const float* act_in, Activation act, const float* res, float res_w, float* tmp, int batch, Context* ctx);

#endif /* NN_LAYER_H */
