/*
 * oracle.h — CPU restatement of the reference's training-backward path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load liboracle.so, and only as the
 * checker.  The product path (libnott_hip.so and thot_amd) never calls it.
 *
 * Every function is a brute-force loop nest over fp32 host buffers with
 * double accumulation, restating the libtorch op that the Nott module at the
 * cited reference file:line dispatches.  Shapes and options use the
 * descriptor structs of include/nott_hip.h (NCHW only).
 *
 * Pinning (tests/test_oracle.py): every function is checked against golden
 * vectors written by the reference's own modules compiled from source
 * (oracle/_ref, tests/golden/), and against invariants / closed forms that
 * a dropped term, wrong sign or transposed operand would break.
 */
#ifndef NOTT_ORACLE_H
#define NOTT_ORACLE_H

#include <stdint.h>

#include "../include/nott_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

int64_t oracle_conv_out(int64_t in, int64_t k, int64_t stride, int64_t pad, int64_t dil);
int64_t oracle_pool_out(int64_t in, int64_t k, int64_t stride, int64_t pad, int64_t dil, int ceil_mode);

/* conv.hpp:177 (torch::nn::Conv2d) */
void oracle_conv2d_fwd(const nott_conv2d_desc* d, const float* x, const float* w, const float* b, float* y);
void oracle_conv2d_bwd_data(const nott_conv2d_desc* d, const float* dy, const float* w, float* dx);
void oracle_conv2d_bwd_weight(const nott_conv2d_desc* d, const float* x, const float* dy, float* dw, float* db);

/* fc.hpp:40 (torch::nn::Linear) */
void oracle_linear_fwd(int64_t m, int64_t kin, int64_t nout, const float* x, const float* w, const float* b, float* y);
void oracle_linear_bwd(int64_t m, int64_t kin, int64_t nout, const float* dy, const float* x, const float* w,
                       float* dx, float* dw, float* db);

/* activation/details/relu.hpp:13 */
void oracle_relu_fwd(int64_t n, const float* x, float* y);
void oracle_relu_bwd(int64_t n, const float* y, const float* dy, float* dx);

/* pooling.hpp:144 (MaxPool2d), :164 (AdaptiveAvgPool2d {1,1}) */
void oracle_maxpool2d_fwd(const nott_pool2d_desc* d, const float* x, float* y, int64_t* argmax);
void oracle_maxpool2d_bwd(const nott_pool2d_desc* d, const int64_t* argmax, const float* dy, float* dx);
void oracle_avgpool_global_fwd(int64_t nc, int64_t hw, const float* x, float* y);
void oracle_avgpool_global_bwd(int64_t nc, int64_t hw, const float* dy, float* dx);

/* batchnorm.hpp:44-50 (torch::nn::BatchNorm2d, training mode) */
void oracle_batchnorm2d_fwd(int64_t n, int64_t c, int64_t hw, const float* x, const float* gamma, const float* beta,
                            double eps, double momentum, float* running_mean, float* running_var,
                            float* y, float* mean, float* rstd);
void oracle_batchnorm2d_bwd(int64_t n, int64_t c, int64_t hw, const float* x, const float* dy, const float* mean,
                            const float* rstd, const float* gamma, float* dx, float* dgamma, float* dbeta);

/* classic.hpp:403-404 (torch::nn::LayerNorm, eps 1e-5, affine) */
void oracle_layernorm_fwd(int64_t rows, int64_t d, const float* x, const float* gamma, const float* beta, double eps,
                          float* y, float* mean, float* rstd);
void oracle_layernorm_bwd(int64_t rows, int64_t d, const float* x, const float* dy, const float* mean,
                          const float* rstd, const float* gamma, float* dx, float* dgamma, float* dbeta);

/* ce.hpp:21-37 (F::cross_entropy, mean, ignore_index -100) */
void oracle_softmax_xent(int64_t n, int64_t c, const float* logits, const int64_t* labels, double label_smoothing,
                         double grad_scale, float* dlogits, float* loss);

/* kernel.hpp:20-96 (scaled dot-product attention) */
void oracle_attention_fwd(const nott_attn_desc* d, const float* q, const float* k, const float* v, float* o, float* lse);
void oracle_attention_bwd(const nott_attn_desc* d, const float* q, const float* k, const float* v, const float* o,
                          const float* dO, float* dq, float* dk, float* dv);

/* adam.hpp:63,159 (torch::optim::Adam / AdamW step); fp32 in libtorch's op order */
void oracle_adam_step(int decoupled, int64_t n, float* p, const float* g, float* m, float* v, double lr, double beta1,
                      double beta2, double eps, double weight_decay, int64_t step);

/* bf16 round-to-nearest-even (c10::BFloat16 semantics) applied in place */
void oracle_round_bf16(int64_t n, float* x);

#ifdef __cplusplus
}
#endif
#endif
