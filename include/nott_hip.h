/*
 * nott_hip.h — C ABI of libnott_hip.so, the MI355X (gfx950) backward-pass
 * library behind Nott's layer, loss and optimizer modules.
 *
 * The reference (MoonFlowww/Thot, namespace Nott) has no C ABI: every
 * backward op is a libtorch autograd node recorded by a torch::nn module
 * that Nott builds.  Each entry point below replaces the ATen kernel that
 * one of those nodes dispatches; the comment on each names the Nott call
 * site (reference file:line, relative to the reference's src/) whose
 * backward it computes.
 *
 * Conventions (all entry points):
 *   - Return an int status: NOTT_OK (0) or a negative NOTT_ERR_* code.
 *     Nothing throws across the ABI.  nott_last_error(ctx) gives the text.
 *   - Every pointer is a device pointer owned by the caller unless the
 *     comment says otherwise.  Tensors are dense and contiguous in the
 *     layout named.  Launches are asynchronous on the context's stream
 *     (nott_set_stream); nothing synchronises unless stated.
 *   - `dtype` names the storage type of activations and activation
 *     gradients (x, y, dy, dx, logits, q/k/v …).  Arithmetic is fp32 for
 *     both dtypes.  Parameter gradients (dw, db, dgamma, dbeta) and
 *     per-row / per-channel statistics are always fp32.
 *   - `accumulate` = 0 overwrites a parameter-gradient output, 1 adds into
 *     it (libtorch AccumulateGrad semantics on a zero_grad'ed .grad()).
 *   - A context is bound to one device and is not re-entrant; calls that
 *     share a context must be serialised by the caller.
 */
#ifndef NOTT_HIP_H
#define NOTT_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NOTT_ABI_VERSION 1

enum {
    NOTT_OK = 0,
    NOTT_ERR_INVALID_ARG = -1,   /* shape / option error  -> std::invalid_argument */
    NOTT_ERR_UNSUPPORTED = -2,   /* valid but not built    -> std::invalid_argument */
    NOTT_ERR_HIP = -3,           /* HIP runtime failure    -> std::runtime_error    */
    NOTT_ERR_ALLOC = -4,         /* workspace allocation   -> std::runtime_error    */
    NOTT_ERR_DEVICE = -5         /* kernel-detected data error (e.g. label out of range) */
};

typedef enum { NOTT_F32 = 0, NOTT_BF16 = 1 } nott_dtype;
typedef enum { NOTT_NCHW = 0, NOTT_NHWC = 1 } nott_layout;

typedef struct nott_ctx_s* nott_ctx;

/* ---- context --------------------------------------------------------- */
/* Owns: device id, the launch stream, a workspace arena and a device error
 * word.  When a call needs more workspace, a new arena (at least twice the
 * size) is allocated and the old one is kept, not freed, until nott_destroy:
 * a HIP graph captured earlier keeps its workspace pointer valid, and no
 * stream is synchronised for growth.  The workspace is shared by every call
 * on the context, so calls on different streams that overlap race on it.
 * Replaces nothing in the reference (libtorch keeps this state in its
 * caching allocator and per-device stream pool). */
int nott_create(int device, nott_ctx* out);
int nott_destroy(nott_ctx ctx);
int nott_set_stream(nott_ctx ctx, void* hip_stream);   /* NULL = legacy default stream */
void* nott_get_stream(nott_ctx ctx);
const char* nott_last_error(nott_ctx ctx);
const char* nott_status_string(int status);
int nott_abi_version(void);
/* Synchronises the stream and returns the number of data errors kernels
 * reported since the last call (labels out of range), then clears it. */
int nott_device_errors(nott_ctx ctx, int64_t* count);
/* Device memory the context holds for workspace, in bytes: the live arena
 * plus the smaller arenas retired when it grew (kept until nott_destroy,
 * since a graph captured earlier may still use them).  The static scratch
 * of nott_layernorm_bwd_noalloc is per GPU and not counted. */
int nott_workspace_bytes(nott_ctx ctx, int64_t* bytes);

/* ---- conv2d ------------------------------------------------------------
 * Replaces the autograd node of torch::nn::Conv2d built by
 * Nott::Layer::Details::build_registered_layer(Owner&, const Conv2dDescriptor&, size_t)
 * (layer/details/conv.hpp:140-191, module created at :177; options :39-49).
 * Layout NCHW is the reference default; NHWC is its ChannelsLast mode
 * (core.hpp:2546-2561, conv.hpp:178-182).  groups must be 1, padding_mode
 * "zeros".  Output size p = (h + 2*pad_h - dil_h*(r-1) - 1)/stride_h + 1. */
typedef struct nott_conv2d_desc {
    int64_t n, c, h, w;        /* input  x  [n, c, h, w] (logical)          */
    int64_t k;                 /* output channels; weight [k, c, r, s]      */
    int64_t r, s;              /* kernel height, width                      */
    int64_t stride_h, stride_w;
    int64_t pad_h, pad_w;
    int64_t dil_h, dil_w;
    int64_t groups;            /* must be 1 */
    int32_t layout;            /* nott_layout of x, y, dx, dy; weight always KCRS */
    int32_t reserved;
} nott_conv2d_desc;

/* y = conv(x, w) + b (b fp32, nullable); w in dtype.  Forward that feeds the
 * backward (conv.hpp:177 forward). */
int nott_conv2d_fwd(nott_ctx ctx, const nott_conv2d_desc* d, nott_dtype dtype,
                    const void* x, const void* w, const float* b, void* y);
/* y = relu(conv(x, w) + b) when relu = 1 (0: as nott_conv2d_fwd): the layer
 * with the activation Nott applies after it (apply.hpp:24-57, relu.hpp:13;
 * src/core.hpp:1933), fused into the convolution's epilogue where it has one. */
int nott_conv2d_fwd_act(nott_ctx ctx, const nott_conv2d_desc* d, nott_dtype dtype,
                        const void* x, const void* w, const float* b, int relu, void* y);
/* dgrad: dx = conv_transpose(dy, w).  (ATen convolution_backward, input grad) */
int nott_conv2d_bwd_data(nott_ctx ctx, const nott_conv2d_desc* d, nott_dtype dtype,
                         const void* dy, const void* w, void* dx);
/* A 3x3 stride-1 layer's weights, re-laid out for the data gradient by the
 * forward's own weight prep (one launch for both layouts) and kept by the
 * caller until the backward: no counterpart in the reference (libtorch
 * transforms the weights inside each convolution call); for host layers that
 * run a layer's forward and backward in one step.
 * nott_conv2d_dgrad_prep_bytes: size of wd for d (0 when the convolution does
 * not take this path: then use nott_conv2d_fwd_act / nott_conv2d_bwd_data).
 * nott_conv2d_fwd_prep: as nott_conv2d_fwd_act, and writes wd (16-byte aligned).
 * nott_conv2d_bwd_data_prepped: as nott_conv2d_bwd_data, from wd. */
int nott_conv2d_dgrad_prep_bytes(const nott_conv2d_desc* d, nott_dtype dtype, int64_t* bytes);
int nott_conv2d_fwd_prep(nott_ctx ctx, const nott_conv2d_desc* d, nott_dtype dtype,
                         const void* x, const void* w, const float* b, int relu, void* y, void* wd);
int nott_conv2d_bwd_data_prepped(nott_ctx ctx, const nott_conv2d_desc* d, nott_dtype dtype,
                                 const void* dy, const void* wd, void* dx);
/* wgrad: dw[k,c,r,s] = sum_{n,p,q} dy * x(shifted); db[k] = sum dy (db nullable).
 * dw, db fp32.  (ATen convolution_backward, weight and bias grads) */
int nott_conv2d_bwd_weight(nott_ctx ctx, const nott_conv2d_desc* d, nott_dtype dtype,
                           const void* x, const void* dy, float* dw, float* db,
                           int accumulate);

/* ---- linear ------------------------------------------------------------
 * Replaces torch::nn::Linear built by build_registered_layer(Owner&, const
 * FCDescriptor&, size_t) (layer/details/fc.hpp:32-49, module at :40) and the
 * q/k/v/out projections of MultiHeadAttentionImpl (attention/details/head.hpp:38-41).
 * x [m, kin], w [nout, kin] (dtype), b [nout] fp32 nullable, y [m, nout]. */
int nott_linear_fwd(nott_ctx ctx, nott_dtype dtype, int64_t m, int64_t kin, int64_t nout,
                    const void* x, const void* w, const float* b, void* y);
/* dx = dy·w (nullable), dw = dyᵀ·x (fp32, nullable), db = Σ_rows dy (fp32, nullable). */
int nott_linear_bwd(nott_ctx ctx, nott_dtype dtype, int64_t m, int64_t kin, int64_t nout,
                    const void* dy, const void* x, const void* w,
                    void* dx, float* dw, float* db, int accumulate);
/* An FC layer with its ReLU activation (fc.hpp:40 with the activation node of
 * activation/apply.hpp:24-57, relu.hpp:13): relu = 1 gives y = relu(x·wᵀ + b)
 * in the GEMM's epilogue, bit-identical to nott_linear_fwd then nott_relu_fwd. */
int nott_linear_fwd_act(nott_ctx ctx, nott_dtype dtype, int64_t m, int64_t kin, int64_t nout,
                        const void* x, const void* w, const float* b, int relu, void* y);
/* nott_linear_bwd where x is the output of the previous layer's ReLU
 * (relu_input = 1): dx also takes that ReLU's backward, dx = (x <= 0) ? 0 : dy·w,
 * bit-identical to nott_linear_bwd then nott_relu_bwd(y = x). */
int nott_linear_bwd_act(nott_ctx ctx, nott_dtype dtype, int64_t m, int64_t kin, int64_t nout,
                        const void* dy, const void* x, const void* w,
                        void* dx, float* dw, float* db, int accumulate, int relu_input);

/* ---- ReLU -------------------------------------------------------------
 * Replaces the relu node applied after every layer by
 * Nott::Activation::Details::apply (activation/apply.hpp:24-57, ReLU at
 * activation/details/relu.hpp:13).  dx = (y <= 0) ? 0 : dy  (y = relu output). */
int nott_relu_fwd(nott_ctx ctx, nott_dtype dtype, int64_t n, const void* x, void* y);
int nott_relu_bwd(nott_ctx ctx, nott_dtype dtype, int64_t n, const void* y, const void* dy, void* dx);

/* ---- max-pool / global average pool -------------------------------------
 * Replaces torch::nn::MaxPool2d / AdaptiveAvgPool2d({1,1}) built by
 * build_registered_layer(Owner&, const PoolingDescriptor&, size_t)
 * (layer/details/pooling.hpp:132-149 and :164-167; options :41-57). */
typedef struct nott_pool2d_desc {
    int64_t n, c, h, w;
    int64_t kh, kw;
    int64_t stride_h, stride_w;
    int64_t pad_h, pad_w;
    int64_t dil_h, dil_w;
    int32_t ceil_mode;
    int32_t layout;            /* NOTT_NCHW only */
} nott_pool2d_desc;
/* y = max over window, argmax = flat index ih*w+iw within the (n,c) plane
 * (int64).  Tie rule: first maximum in scan order; a NaN always wins. */
int nott_maxpool2d_fwd(nott_ctx ctx, const nott_pool2d_desc* d, nott_dtype dtype,
                       const void* x, void* y, int64_t* argmax);
/* dx[argmax] += dy, summed in output scan order for overlapping windows. */
int nott_maxpool2d_bwd(nott_ctx ctx, const nott_pool2d_desc* d, nott_dtype dtype,
                       const int64_t* argmax, const void* dy, void* dx);
/* The same pair (the same torch::nn::MaxPool2d, pooling.hpp:132-149) with the
 * argmax kept as the window tap, one byte per output:
 *   tap = ((ih - oh*stride_h + pad_h) / dil_h) * kw + (iw - ow*stride_w + pad_w) / dil_w,
 * for callers that keep the indices to themselves (the host models' MaxPool2d
 * layers); 1/8 of the index traffic.  y and dx are bit-identical to the int64
 * pair's.  Requires kh*kw <= 256. */
int nott_maxpool2d_fwd_tap(nott_ctx ctx, const nott_pool2d_desc* d, nott_dtype dtype,
                           const void* x, void* y, uint8_t* tap);
int nott_maxpool2d_bwd_tap(nott_ctx ctx, const nott_pool2d_desc* d, nott_dtype dtype,
                           const uint8_t* tap, const void* dy, void* dx);
/* Max-pool backward followed by the backward of the ReLU whose output y is
 * the pool's input (the Conv2d + ReLU + MaxPool2d layers of the small CNN:
 * conv.hpp:177 with activation/details/relu.hpp:13, then pooling.hpp:144):
 * dx = (y <= 0) ? 0 : maxpool_bwd(dy), bit-identical to nott_maxpool2d_bwd_tap
 * then nott_relu_bwd, in one pass where the tiled kernels apply. */
int nott_maxpool2d_bwd_tap_relu(nott_ctx ctx, const nott_pool2d_desc* d, nott_dtype dtype,
                                const uint8_t* tap, const void* dy, const void* y, void* dx);
/* The max-pool of a BatchNorm2d + ReLU output (ResNet-18's stem: batchnorm.hpp:50
 * with its ReLU activation, then pooling.hpp:144) without that output in
 * memory: the pool reads the BatchNorm's input x and forms relu(a·x + c) per
 * channel, coef = {a_c, c_c} from nott_batchnorm2d_fwd_coef, as the BatchNorm's
 * apply pass would store it; y and tap are bit-identical to
 * nott_batchnorm2d_fwd_act (relu) then nott_maxpool2d_fwd_tap.  Stride-2 3x3
 * (pad 1) or 2x2 (pad 0) windows on rows of whole 4-element groups only
 * (NOTT_ERR_UNSUPPORTED otherwise). */
int nott_maxpool2d_fwd_tap_bnrelu(nott_ctx ctx, const nott_pool2d_desc* d, nott_dtype dtype,
                                  const void* x, const float* coef, void* y, uint8_t* tap);
/* Its backward (the BatchNorm2d + ReLU backward of batchnorm.hpp:50 taking the
 * max-pool backward of pooling.hpp:144 as its dy): dx, dgamma and dbeta of
 * nott_maxpool2d_bwd_tap then nott_batchnorm2d_bwd_act (relu), d the pool's
 * descriptor (x [n, c, h, w] the BatchNorm's input, tap and dy the pooled
 * shape).  On the stride-2 shapes of nott_maxpool2d_fwd_tap_bnrelu the routed
 * gradient is never stored: the BatchNorm's sums run over the pooled outputs
 * and the routing carries the apply, so results agree with the two calls to
 * rounding (each routed term enters the sums unrounded); other shapes run the
 * two calls.  dx nullable (dgamma, dbeta only); accumulate adds into them. */
int nott_batchnorm2d_relu_maxpool2d_bwd(nott_ctx ctx, const nott_pool2d_desc* d, nott_dtype dtype,
                                        const void* x, const uint8_t* tap, const void* dy,
                                        const float* mean, const float* rstd, const float* gamma,
                                        const float* beta, void* dx, float* dgamma, float* dbeta,
                                        int accumulate);
/* y[nc] = mean over hw; dx[nc, i] = dy[nc] / hw. */
int nott_avgpool_global_fwd(nott_ctx ctx, nott_dtype dtype, int64_t nc, int64_t hw,
                            const void* x, void* y);
int nott_avgpool_global_bwd(nott_ctx ctx, nott_dtype dtype, int64_t nc, int64_t hw,
                            const void* dy, void* dx);

/* ---- batch norm (training mode) -----------------------------------------
 * Replaces torch::nn::BatchNorm2d built by build_registered_layer(Owner&,
 * const BatchNorm2dDescriptor&, size_t) (layer/details/batchnorm.hpp:38-59).
 * x [n, c, hw] NCHW; gamma, beta, mean, rstd, running stats fp32 [c].
 * Forward saves mean and rstd = 1/sqrt(var_biased + eps); running stats are
 * updated with momentum and the unbiased variance (nullable). */
/* The statistics of the forward alone (mean, rstd, running stats) and the
 * affine coefficients of its apply pass, y = coef[2c]·x + coef[2c+1] per
 * channel (fp32 [2c]), for a consumer that applies them itself
 * (nott_maxpool2d_fwd_tap_bnrelu). */
int nott_batchnorm2d_fwd_coef(nott_ctx ctx, nott_dtype dtype, int64_t n, int64_t c, int64_t hw,
                              const void* x, const float* gamma, const float* beta, double eps,
                              double momentum, float* running_mean, float* running_var, float* mean,
                              float* rstd, float* coef);
int nott_batchnorm2d_fwd(nott_ctx ctx, nott_dtype dtype, int64_t n, int64_t c, int64_t hw,
                         const void* x, const float* gamma, const float* beta,
                         double eps, double momentum, float* running_mean, float* running_var,
                         void* y, float* mean, float* rstd);
int nott_batchnorm2d_bwd(nott_ctx ctx, nott_dtype dtype, int64_t n, int64_t c, int64_t hw,
                         const void* x, const void* dy, const float* mean, const float* rstd,
                         const float* gamma, void* dx, float* dgamma, float* dbeta,
                         int accumulate);
/* BatchNorm2d fused with what Nott applies right after it: the layer's own
 * activation (ReLU; block/details/blocks/residual.hpp:94-96, the BN layer
 * then Activation::Details::apply) and, for the second BN of a residual
 * branch, the skip addition and the block's final activation (residual.hpp:
 * 130-132).  Forward: y = act(BN(x) [+ residual]), act = ReLU when relu != 0
 * (residual nullable).  Backward with relu != 0: dy is the gradient w.r.t.
 * relu(BN(x)) (no residual), the ReLU mask is recomputed from x, gamma, beta,
 * mean and rstd; with relu == 0 it is nott_batchnorm2d_bwd. */
int nott_batchnorm2d_fwd_act(nott_ctx ctx, nott_dtype dtype, int64_t n, int64_t c, int64_t hw,
                             const void* x, const float* gamma, const float* beta,
                             double eps, double momentum, float* running_mean, float* running_var,
                             const void* residual, int relu, void* y, float* mean, float* rstd);
int nott_batchnorm2d_bwd_act(nott_ctx ctx, nott_dtype dtype, int64_t n, int64_t c, int64_t hw,
                             const void* x, const void* dy, const float* mean, const float* rstd,
                             const float* gamma, const float* beta, int relu, void* dx,
                             float* dgamma, float* dbeta, int accumulate);

/* ---- layer norm ---------------------------------------------------------
 * Replaces torch::nn::LayerNorm of TransformerEncoderLayerImpl
 * (block/details/transformers/classic.hpp:403-404, final norm :495).
 * x, y, dy, dx [rows, d] (dtype); gamma, beta [d] (dtype); mean, rstd
 * [rows] fp32; dgamma, dbeta [d] fp32. */
int nott_layernorm_fwd(nott_ctx ctx, nott_dtype dtype, int64_t rows, int64_t d,
                       const void* x, const void* gamma, const void* beta, double eps,
                       void* y, float* mean, float* rstd);
int nott_layernorm_bwd(nott_ctx ctx, nott_dtype dtype, int64_t rows, int64_t d,
                       const void* x, const void* dy, const float* mean, const float* rstd,
                       const void* gamma, void* dx, float* dgamma, float* dbeta,
                       int accumulate);
/* nott_layernorm_bwd without any allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, serving loops, harnesses that forbid hipMalloc).
 * Same arguments and results as nott_layernorm_bwd (the same kernels); the
 * dgamma/dbeta column partials live in a static 16 MiB device array, one per
 * GPU, instead of the context workspace.  That bounds the problem.  On the
 * vector path (d <= 2048 and a multiple of 8 bf16 / 4 fp32 elements, every
 * row pointer 16-byte aligned) the partials take 2·16·ceil(d/16)·4 bytes for
 * each of at most (number of CUs) blocks, at most 4 MiB on a 256-CU MI355X,
 * so every row count fits.  Otherwise the generic path needs 8·d·rows bytes
 * (rows·d <= 2^21 elements).  Larger problems return NOTT_ERR_UNSUPPORTED
 * with the sizes in the message.  Every call on a GPU
 * shares that GPU's array: calls that overlap on one GPU (two streams, two
 * contexts) race.  The partials are written in full before they are read,
 * so no clearing is needed between calls. */
int nott_layernorm_bwd_noalloc(nott_ctx ctx, nott_dtype dtype, int64_t rows, int64_t d,
                               const void* x, const void* dy, const float* mean, const float* rstd,
                               const void* gamma, void* dx, float* dgamma, float* dbeta,
                               int accumulate);

/* ---- softmax cross-entropy ------------------------------------------------
 * Replaces F::cross_entropy called by Nott::Loss::Details::compute(const
 * CrossEntropyDescriptor&, ...) (loss/details/ce.hpp:21-37), mean reduction,
 * ignore_index -100, optional label smoothing, no class weights.
 * logits, dlogits [n, c] (dtype); labels int64 [n].  One pass computes
 * dlogits = grad_scale·(softmax − (1−ε)·onehot − ε/c)/n_valid and, if loss
 * is non-NULL, the mean loss (fp32 scalar). */
int nott_softmax_xent_bwd(nott_ctx ctx, nott_dtype dtype, int64_t n, int64_t c,
                          const void* logits, const int64_t* labels,
                          double label_smoothing, double grad_scale,
                          void* dlogits, float* loss);

/* ---- scaled dot-product attention -----------------------------------------
 * Replaces ScaledDotProductKernelImpl::forward (attention/details/kernel.hpp:20-96):
 * s = q·kᵀ·scale, causal mask triu(1) -> -inf, p = softmax(s), o = p·v.
 * lse [b, h, t] fp32 = log Σ exp(s).  Dropout must be 0.
 * Layouts (dtype elements):
 *   NOTT_ATTN_HEAD_MAJOR: q, o, dO, dq [b, h, t, dh]; k, v, dk, dv [b, h, s, dh],
 *     contiguous (the tensors after head.hpp:70-75's view + transpose);
 *   NOTT_ATTN_TOKEN_MAJOR: q, dq [b, t, h, dh] and k, v, dk, dv [b, s, h, dh]
 *     with row stride ld_qkv between consecutive tokens, o, dO [b, t, h, dh]
 *     with row stride ld_o (0 = h·dh): the projections' outputs as they are,
 *     e.g. q, k, v = qkv, qkv + h·dh, qkv + 2·h·dh of a packed [b·t, 3·h·dh]
 *     buffer with ld_qkv = 3·h·dh, so no head split or merge copies. */
#define NOTT_ATTN_HEAD_MAJOR 0
#define NOTT_ATTN_TOKEN_MAJOR 1
typedef struct nott_attn_desc {
    int64_t b, h, t, s, dh;
    int32_t causal;
    int32_t layout;            /* NOTT_ATTN_HEAD_MAJOR or NOTT_ATTN_TOKEN_MAJOR */
    double scale;              /* reference: 1/sqrt(dh) */
    int64_t ld_qkv, ld_o;      /* token-major row strides (elements); 0 = h·dh */
} nott_attn_desc;
int nott_attention_fwd(nott_ctx ctx, const nott_attn_desc* d, nott_dtype dtype,
                       const void* q, const void* k, const void* v, void* o, float* lse);
int nott_attention_bwd(nott_ctx ctx, const nott_attn_desc* d, nott_dtype dtype,
                       const void* q, const void* k, const void* v, const void* o,
                       const void* dO, const float* lse, void* dq, void* dk, void* dv);

/* ---- Adam / AdamW --------------------------------------------------------
 * Replaces torch::optim::Adam::step / AdamW::step inherited by
 * Nott::Optimizer::Details::Adam / AdamW (optimizer/details/adam.hpp:63-154,
 * 159-250; options :18-60), stepped by Model::step_optimizers
 * (core.hpp:3820, 5049-5057).  One launch updates a flat buffer of n
 * parameters.  p and g are p_dtype / g_dtype; m, v fp32.  `step` is the
 * post-increment step count t (>= 1).  decoupled = 0: Adam (L2 into g);
 * 1: AdamW (p *= 1 - lr·wd first).  zero_grad_after = 1 also writes g = 0
 * (Model::zero_grad, core.hpp:2425-2442).  amsgrad is not supported. */
int nott_adam_step(nott_ctx ctx, int decoupled, int64_t n,
                   void* p, nott_dtype p_dtype, void* g, nott_dtype g_dtype,
                   float* m, float* v,
                   double lr, double beta1, double beta2, double eps, double weight_decay,
                   int64_t step, int zero_grad_after);

/* The same update as nott_adam_step with its scalars taken from memory at
 * launch time, so that the launch can be captured once into a HIP graph
 * that is replayed every step (the reference's CUDA-graph step path,
 * core.hpp:3829-3945, with the optimizer inside the graph).  Each launch
 * first increments state->step (device memory, the per-tensor step count of
 * torch::optim::Adam[W]; 0 before the first update) and forms the bias
 * corrections from the new count, in the same double arithmetic as
 * nott_adam_step, then runs the update.  hparams = {lr, beta1, beta2, eps,
 * weight_decay} (5 doubles) is read by the device at launch time: device
 * memory, or pinned host memory (hipHostMalloc) that the host rewrites
 * between replays, e.g. after a scheduler writes a new lr
 * (lrscheduler/details/cosineannealing.hpp:52-63).  Whether the weight
 * decay term runs is fixed by weight_decay_nonzero at the call (libtorch
 * skips it when weight_decay == 0). */
typedef struct nott_adam_device_state {
    int64_t step;
    int64_t reserved[7];       /* the launch's scalar block; written by the library */
} nott_adam_device_state;
int nott_adam_step_graph(nott_ctx ctx, int decoupled, int64_t n,
                         void* p, nott_dtype p_dtype, void* g, nott_dtype g_dtype,
                         float* m, float* v, const double* hparams, nott_adam_device_state* state,
                         int weight_decay_nonzero, int zero_grad_after);

/* ---- utilities used by the host modules ---------------------------------- */
/* dst = a + b elementwise (residual gradient fan-in, block/details/blocks/residual.hpp:131). */
int nott_add(nott_ctx ctx, nott_dtype dtype, int64_t n, const void* a, const void* b, void* dst);
/* The gradient of a residual block's output, which is a ReLU output (the
 * block's final activation, residual.hpp:130-132) used twice by the next
 * block (branch and skip, residual.hpp:87-141): dz = (y <= 0) ? 0 : a + b,
 * bit-identical to nott_add then nott_relu_bwd, in one pass. */
int nott_add_relu_bwd(nott_ctx ctx, nott_dtype dtype, int64_t n, const void* a, const void* b, const void* y,
                      void* dz);
/* Dtype conversion fp32 <-> bf16 (round to nearest even). */
int nott_cast(nott_ctx ctx, int64_t n, const void* src, nott_dtype src_dtype, void* dst, nott_dtype dst_dtype);
/* Fill `bytes` bytes with zero using a kernel (safe under graph capture). */
int nott_zero(nott_ctx ctx, int64_t bytes, void* dst);
/* y = x · scale[0] with scale a device fp32 scalar: the chain-rule product
 * of a loss gradient with the upstream gradient of the scalar loss, which
 * libtorch's engine hands over as a device tensor. */
int nott_scale(nott_ctx ctx, nott_dtype dtype, int64_t n, const void* x, const float* scale, void* y);
/* acc[0] += (double)loss[0] · weight, in double on the device: the epoch
 * loss accumulation of Model::run_epochs (core.hpp:4481-4487: the step's
 * detached loss in float64, times the batch size, added to a device
 * accumulator), so a training loop needs no host read per step. */
int nott_loss_accumulate(nott_ctx ctx, const float* loss, double weight, double* acc);

#ifdef __cplusplus
}
#endif
#endif /* NOTT_HIP_H */
