/*
 * oracle.c — CPU restatement of the reference path (TEST INFRASTRUCTURE ONLY;
 * see oracle.h).  The reference (Nott) computes every op below through
 * libtorch 2.10.0 ATen CPU kernels (third-party; no version pin in the
 * reference's CMakeLists.txt:13-19, the image's wheel is torch 2.10.0).
 * Each function restates the op's published semantics as a loop nest, with
 * double accumulation; comments cite the Nott call site that reaches it.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- shapes */
int64_t oracle_conv_out(int64_t in, int64_t k, int64_t stride, int64_t pad, int64_t dil) {
    return (in + 2 * pad - dil * (k - 1) - 1) / stride + 1;
}

/* ATen pooling_output_shape: floor or ceil division; with ceil_mode the last
 * window must start inside the input or its left padding. */
int64_t oracle_pool_out(int64_t in, int64_t k, int64_t stride, int64_t pad, int64_t dil, int ceil_mode) {
    int64_t num = in + 2 * pad - dil * (k - 1) - 1 + (ceil_mode ? stride - 1 : 0);
    int64_t out = (num >= 0 ? num / stride : -((-num + stride - 1) / stride)) + 1;
    if (ceil_mode && (out - 1) * stride >= in + pad) --out;
    return out;
}

/* ------------------------------------------------------------------ conv
 * Conv2d forward (reference conv.hpp:177 -> torch::nn::Conv2d, zero padding,
 * groups 1):  y[n,k,p,q] = b[k] + Σ_{c,r,s} w[k,c,r,s]·x[n,c,p·sh−ph+r·dh, q·sw−pw+s·dw]. */
void oracle_conv2d_fwd(const nott_conv2d_desc* d, const float* x, const float* w, const float* b, float* y) {
    const int64_t P = oracle_conv_out(d->h, d->r, d->stride_h, d->pad_h, d->dil_h);
    const int64_t Q = oracle_conv_out(d->w, d->s, d->stride_w, d->pad_w, d->dil_w);
    for (int64_t n = 0; n < d->n; ++n)
        for (int64_t k = 0; k < d->k; ++k)
            for (int64_t p = 0; p < P; ++p)
                for (int64_t q = 0; q < Q; ++q) {
                    double acc = b ? b[k] : 0.0;
                    for (int64_t c = 0; c < d->c; ++c)
                        for (int64_t r = 0; r < d->r; ++r) {
                            const int64_t ih = p * d->stride_h - d->pad_h + r * d->dil_h;
                            if (ih < 0 || ih >= d->h) continue;
                            for (int64_t s = 0; s < d->s; ++s) {
                                const int64_t iw = q * d->stride_w - d->pad_w + s * d->dil_w;
                                if (iw < 0 || iw >= d->w) continue;
                                acc += (double)w[((k * d->c + c) * d->r + r) * d->s + s] *
                                       (double)x[((n * d->c + c) * d->h + ih) * d->w + iw];
                            }
                        }
                    y[((n * d->k + k) * P + p) * Q + q] = (float)acc;
                }
}

/* dgrad: the adjoint of the forward in x:
 * dx[n,c,ih,iw] = Σ_{k,p,q,r,s : p·sh−ph+r·dh = ih, q·sw−pw+s·dw = iw} w[k,c,r,s]·dy[n,k,p,q]. */
void oracle_conv2d_bwd_data(const nott_conv2d_desc* d, const float* dy, const float* w, float* dx) {
    const int64_t P = oracle_conv_out(d->h, d->r, d->stride_h, d->pad_h, d->dil_h);
    const int64_t Q = oracle_conv_out(d->w, d->s, d->stride_w, d->pad_w, d->dil_w);
    const int64_t nx = d->n * d->c * d->h * d->w;
    double* acc = (double*)calloc((size_t)nx, sizeof(double));
    for (int64_t n = 0; n < d->n; ++n)
        for (int64_t k = 0; k < d->k; ++k)
            for (int64_t p = 0; p < P; ++p)
                for (int64_t q = 0; q < Q; ++q) {
                    const double g = dy[((n * d->k + k) * P + p) * Q + q];
                    for (int64_t c = 0; c < d->c; ++c)
                        for (int64_t r = 0; r < d->r; ++r) {
                            const int64_t ih = p * d->stride_h - d->pad_h + r * d->dil_h;
                            if (ih < 0 || ih >= d->h) continue;
                            for (int64_t s = 0; s < d->s; ++s) {
                                const int64_t iw = q * d->stride_w - d->pad_w + s * d->dil_w;
                                if (iw < 0 || iw >= d->w) continue;
                                acc[((n * d->c + c) * d->h + ih) * d->w + iw] +=
                                    g * (double)w[((k * d->c + c) * d->r + r) * d->s + s];
                            }
                        }
                }
    for (int64_t i = 0; i < nx; ++i) dx[i] = (float)acc[i];
    free(acc);
}

/* wgrad: dw[k,c,r,s] = Σ_{n,p,q} dy[n,k,p,q]·x[n,c,p·sh−ph+r·dh, q·sw−pw+s·dw];  db[k] = Σ_{n,p,q} dy. */
void oracle_conv2d_bwd_weight(const nott_conv2d_desc* d, const float* x, const float* dy, float* dw, float* db) {
    const int64_t P = oracle_conv_out(d->h, d->r, d->stride_h, d->pad_h, d->dil_h);
    const int64_t Q = oracle_conv_out(d->w, d->s, d->stride_w, d->pad_w, d->dil_w);
    for (int64_t k = 0; k < d->k; ++k) {
        for (int64_t c = 0; c < d->c; ++c)
            for (int64_t r = 0; r < d->r; ++r)
                for (int64_t s = 0; s < d->s; ++s) {
                    double acc = 0.0;
                    for (int64_t n = 0; n < d->n; ++n)
                        for (int64_t p = 0; p < P; ++p) {
                            const int64_t ih = p * d->stride_h - d->pad_h + r * d->dil_h;
                            if (ih < 0 || ih >= d->h) continue;
                            for (int64_t q = 0; q < Q; ++q) {
                                const int64_t iw = q * d->stride_w - d->pad_w + s * d->dil_w;
                                if (iw < 0 || iw >= d->w) continue;
                                acc += (double)dy[((n * d->k + k) * P + p) * Q + q] *
                                       (double)x[((n * d->c + c) * d->h + ih) * d->w + iw];
                            }
                        }
                    dw[((k * d->c + c) * d->r + r) * d->s + s] = (float)acc;
                }
        if (db) {
            double acc = 0.0;
            for (int64_t n = 0; n < d->n; ++n)
                for (int64_t i = 0; i < P * Q; ++i) acc += dy[(n * d->k + k) * P * Q + i];
            db[k] = (float)acc;
        }
    }
}

/* ---------------------------------------------------------------- linear
 * fc.hpp:40 -> torch::nn::Linear:  y = x·wᵀ + b;  dx = dy·w;  dw = dyᵀ·x;  db = Σ_rows dy. */
void oracle_linear_fwd(int64_t m, int64_t kin, int64_t nout, const float* x, const float* w, const float* b, float* y) {
    for (int64_t i = 0; i < m; ++i)
        for (int64_t j = 0; j < nout; ++j) {
            double acc = b ? b[j] : 0.0;
            for (int64_t t = 0; t < kin; ++t) acc += (double)x[i * kin + t] * (double)w[j * kin + t];
            y[i * nout + j] = (float)acc;
        }
}

void oracle_linear_bwd(int64_t m, int64_t kin, int64_t nout, const float* dy, const float* x, const float* w,
                       float* dx, float* dw, float* db) {
    if (dx)
        for (int64_t i = 0; i < m; ++i)
            for (int64_t t = 0; t < kin; ++t) {
                double acc = 0.0;
                for (int64_t j = 0; j < nout; ++j) acc += (double)dy[i * nout + j] * (double)w[j * kin + t];
                dx[i * kin + t] = (float)acc;
            }
    if (dw)
        for (int64_t j = 0; j < nout; ++j)
            for (int64_t t = 0; t < kin; ++t) {
                double acc = 0.0;
                for (int64_t i = 0; i < m; ++i) acc += (double)dy[i * nout + j] * (double)x[i * kin + t];
                dw[j * kin + t] = (float)acc;
            }
    if (db)
        for (int64_t j = 0; j < nout; ++j) {
            double acc = 0.0;
            for (int64_t i = 0; i < m; ++i) acc += dy[i * nout + j];
            db[j] = (float)acc;
        }
}

/* ------------------------------------------------------------------ relu
 * relu.hpp:13 -> torch::relu; autograd threshold_backward(grad, result, 0):
 * dx = (y <= 0) ? 0 : dy  (a NaN output passes the gradient through). */
void oracle_relu_fwd(int64_t n, const float* x, float* y) {
    for (int64_t i = 0; i < n; ++i) y[i] = (x[i] > 0.f || isnan(x[i])) ? x[i] : 0.f;
}

void oracle_relu_bwd(int64_t n, const float* y, const float* dy, float* dx) {
    for (int64_t i = 0; i < n; ++i) dx[i] = (y[i] <= 0.f) ? 0.f : dy[i];
}

/* --------------------------------------------------------------- maxpool
 * pooling.hpp:144 -> torch::nn::MaxPool2d -> max_pool2d_with_indices (CPU).
 * Window scan: rows then columns, starting at the first in-bounds tap; the
 * index starts at that tap and moves on a strictly greater value or a NaN. */
void oracle_maxpool2d_fwd(const nott_pool2d_desc* d, const float* x, float* y, int64_t* argmax) {
    const int64_t OH = oracle_pool_out(d->h, d->kh, d->stride_h, d->pad_h, d->dil_h, d->ceil_mode);
    const int64_t OW = oracle_pool_out(d->w, d->kw, d->stride_w, d->pad_w, d->dil_w, d->ceil_mode);
    for (int64_t pl = 0; pl < d->n * d->c; ++pl) {
        const float* xp = x + pl * d->h * d->w;
        for (int64_t oh = 0; oh < OH; ++oh)
            for (int64_t ow = 0; ow < OW; ++ow) {
                int64_t ih0 = oh * d->stride_h - d->pad_h;
                int64_t iw0 = ow * d->stride_w - d->pad_w;
                const int64_t ih1 = ih0 + (d->kh - 1) * d->dil_h + 1 < d->h ? ih0 + (d->kh - 1) * d->dil_h + 1 : d->h;
                const int64_t iw1 = iw0 + (d->kw - 1) * d->dil_w + 1 < d->w ? iw0 + (d->kw - 1) * d->dil_w + 1 : d->w;
                while (ih0 < 0) ih0 += d->dil_h;
                while (iw0 < 0) iw0 += d->dil_w;
                int64_t best = ih0 * d->w + iw0;
                float bv = -INFINITY;
                for (int64_t ih = ih0; ih < ih1; ih += d->dil_h)
                    for (int64_t iw = iw0; iw < iw1; iw += d->dil_w) {
                        const float v = xp[ih * d->w + iw];
                        if (v > bv || isnan(v)) {
                            bv = v;
                            best = ih * d->w + iw;
                        }
                    }
                y[(pl * OH + oh) * OW + ow] = bv;
                argmax[(pl * OH + oh) * OW + ow] = best;
            }
    }
}

/* Backward: dx = 0; dx[plane, argmax] += dy in output scan order (fp32 adds). */
void oracle_maxpool2d_bwd(const nott_pool2d_desc* d, const int64_t* argmax, const float* dy, float* dx) {
    const int64_t OH = oracle_pool_out(d->h, d->kh, d->stride_h, d->pad_h, d->dil_h, d->ceil_mode);
    const int64_t OW = oracle_pool_out(d->w, d->kw, d->stride_w, d->pad_w, d->dil_w, d->ceil_mode);
    memset(dx, 0, sizeof(float) * (size_t)(d->n * d->c * d->h * d->w));
    for (int64_t pl = 0; pl < d->n * d->c; ++pl)
        for (int64_t o = 0; o < OH * OW; ++o) {
            const int64_t idx = argmax[pl * OH * OW + o];
            dx[pl * d->h * d->w + idx] += dy[pl * OH * OW + o];
        }
}

/* pooling.hpp:164 -> AdaptiveAvgPool2d({1,1}): mean over the plane; grad dy/hw. */
void oracle_avgpool_global_fwd(int64_t nc, int64_t hw, const float* x, float* y) {
    for (int64_t i = 0; i < nc; ++i) {
        double acc = 0.0;
        for (int64_t j = 0; j < hw; ++j) acc += x[i * hw + j];
        y[i] = (float)(acc / (double)hw);
    }
}

void oracle_avgpool_global_bwd(int64_t nc, int64_t hw, const float* dy, float* dx) {
    for (int64_t i = 0; i < nc; ++i)
        for (int64_t j = 0; j < hw; ++j) dx[i * hw + j] = dy[i] / (float)hw;
}

/* ------------------------------------------------------------- batchnorm
 * batchnorm.hpp:44-50 -> torch::nn::BatchNorm2d in training mode:
 * per channel over (n, hw): mean, biased var -> rstd = 1/sqrt(var+eps);
 * running stats: r = (1−mom)·r + mom·stat with the unbiased variance. */
void oracle_batchnorm2d_fwd(int64_t n, int64_t c, int64_t hw, const float* x, const float* gamma, const float* beta,
                            double eps, double momentum, float* running_mean, float* running_var,
                            float* y, float* mean, float* rstd) {
    const double M = (double)(n * hw);
    for (int64_t ch = 0; ch < c; ++ch) {
        double s = 0.0;
        for (int64_t i = 0; i < n; ++i)
            for (int64_t j = 0; j < hw; ++j) s += x[(i * c + ch) * hw + j];
        const double mu = s / M;
        double ss = 0.0;
        for (int64_t i = 0; i < n; ++i)
            for (int64_t j = 0; j < hw; ++j) {
                const double t = x[(i * c + ch) * hw + j] - mu;
                ss += t * t;
            }
        const double var = ss / M;
        const double rs = 1.0 / sqrt(var + eps);
        mean[ch] = (float)mu;
        rstd[ch] = (float)rs;
        const double g = gamma ? gamma[ch] : 1.0, b = beta ? beta[ch] : 0.0;
        for (int64_t i = 0; i < n; ++i)
            for (int64_t j = 0; j < hw; ++j) {
                const int64_t o = (i * c + ch) * hw + j;
                y[o] = (float)((x[o] - mu) * rs * g + b);
            }
        if (running_mean) running_mean[ch] = (float)((1.0 - momentum) * running_mean[ch] + momentum * mu);
        if (running_var) {
            const double unbiased = M > 1 ? ss / (M - 1.0) : var;
            running_var[ch] = (float)((1.0 - momentum) * running_var[ch] + momentum * unbiased);
        }
    }
}

/* dβ = Σ dy; dγ = Σ dy·x̂; dx = γ·rstd·(dy − Σdy/M − x̂·Σ(dy·x̂)/M). */
void oracle_batchnorm2d_bwd(int64_t n, int64_t c, int64_t hw, const float* x, const float* dy, const float* mean,
                            const float* rstd, const float* gamma, float* dx, float* dgamma, float* dbeta) {
    const double M = (double)(n * hw);
    for (int64_t ch = 0; ch < c; ++ch) {
        const double mu = mean[ch], rs = rstd[ch];
        double sdy = 0.0, sdyx = 0.0;
        for (int64_t i = 0; i < n; ++i)
            for (int64_t j = 0; j < hw; ++j) {
                const int64_t o = (i * c + ch) * hw + j;
                sdy += dy[o];
                sdyx += dy[o] * (x[o] - mu) * rs;
            }
        if (dgamma) dgamma[ch] = (float)sdyx;
        if (dbeta) dbeta[ch] = (float)sdy;
        const double g = gamma ? gamma[ch] : 1.0;
        if (dx)
            for (int64_t i = 0; i < n; ++i)
                for (int64_t j = 0; j < hw; ++j) {
                    const int64_t o = (i * c + ch) * hw + j;
                    const double xh = (x[o] - mu) * rs;
                    dx[o] = (float)(g * rs * (dy[o] - sdy / M - xh * sdyx / M));
                }
    }
}

/* ------------------------------------------------------------- layernorm
 * classic.hpp:403-404 -> torch::nn::LayerNorm({d}) (eps 1e-5, affine):
 * per row x̂ = (x−μ)·rstd, biased variance; y = x̂·γ + β.
 * Backward with g = dy·γ: dx = rstd·(g − Σg/d − x̂·Σ(g·x̂)/d);
 * dγ = Σ_rows dy·x̂; dβ = Σ_rows dy. */
void oracle_layernorm_fwd(int64_t rows, int64_t d, const float* x, const float* gamma, const float* beta, double eps,
                          float* y, float* mean, float* rstd) {
    for (int64_t i = 0; i < rows; ++i) {
        const float* xr = x + i * d;
        double s = 0.0;
        for (int64_t j = 0; j < d; ++j) s += xr[j];
        const double mu = s / (double)d;
        double ss = 0.0;
        for (int64_t j = 0; j < d; ++j) ss += (xr[j] - mu) * (xr[j] - mu);
        const double rs = 1.0 / sqrt(ss / (double)d + eps);
        mean[i] = (float)mu;
        rstd[i] = (float)rs;
        for (int64_t j = 0; j < d; ++j)
            y[i * d + j] = (float)((xr[j] - mu) * rs * (gamma ? gamma[j] : 1.0) + (beta ? beta[j] : 0.0));
    }
}

void oracle_layernorm_bwd(int64_t rows, int64_t d, const float* x, const float* dy, const float* mean,
                          const float* rstd, const float* gamma, float* dx, float* dgamma, float* dbeta) {
    double* dg = (double*)calloc((size_t)d, sizeof(double));
    double* db = (double*)calloc((size_t)d, sizeof(double));
    for (int64_t i = 0; i < rows; ++i) {
        const double mu = mean[i], rs = rstd[i];
        double sg = 0.0, sgx = 0.0;
        for (int64_t j = 0; j < d; ++j) {
            const double xh = (x[i * d + j] - mu) * rs;
            const double g = (double)dy[i * d + j] * (gamma ? gamma[j] : 1.0);
            sg += g;
            sgx += g * xh;
            dg[j] += (double)dy[i * d + j] * xh;
            db[j] += dy[i * d + j];
        }
        if (dx)
            for (int64_t j = 0; j < d; ++j) {
                const double xh = (x[i * d + j] - mu) * rs;
                const double g = (double)dy[i * d + j] * (gamma ? gamma[j] : 1.0);
                dx[i * d + j] = (float)(rs * (g - sg / (double)d - xh * sgx / (double)d));
            }
    }
    for (int64_t j = 0; j < d; ++j) {
        if (dgamma) dgamma[j] = (float)dg[j];
        if (dbeta) dbeta[j] = (float)db[j];
    }
    free(dg);
    free(db);
}

/* ---------------------------------------------------------- cross-entropy
 * ce.hpp:36 -> F::cross_entropy(pred, target, {reduction Mean, label_smoothing ε}),
 * ignore_index −100:  loss = Σ_valid[(1−ε)·(−log p_y) + (ε/c)·(−Σ_j log p_j)] / n_valid;
 * dz = grad_scale·(p − (1−ε)·onehot(y) − ε/c)/n_valid on valid rows, 0 on ignored rows. */
void oracle_softmax_xent(int64_t n, int64_t c, const float* logits, const int64_t* labels, double label_smoothing,
                         double grad_scale, float* dlogits, float* loss) {
    int64_t nvalid = 0;
    for (int64_t i = 0; i < n; ++i) nvalid += labels[i] != -100;
    double total = 0.0;
    for (int64_t i = 0; i < n; ++i) {
        const float* z = logits + i * c;
        float* dz = dlogits ? dlogits + i * c : NULL;
        const int64_t y = labels[i];
        if (y == -100) {
            if (dz)
                for (int64_t j = 0; j < c; ++j) dz[j] = 0.f;
            continue;
        }
        double mx = -INFINITY;
        for (int64_t j = 0; j < c; ++j) mx = z[j] > mx ? z[j] : mx;
        double se = 0.0, sz = 0.0;
        for (int64_t j = 0; j < c; ++j) {
            se += exp((double)z[j] - mx);
            sz += z[j];
        }
        const double lse = mx + log(se);
        const double nll = lse - z[y];
        const double smooth = (double)c * lse - sz; /* −Σ_j log p_j */
        total += (1.0 - label_smoothing) * nll + (label_smoothing / (double)c) * smooth;
        if (dz)
            for (int64_t j = 0; j < c; ++j) {
                const double p = exp((double)z[j] - lse);
                const double t = (j == y ? (1.0 - label_smoothing) : 0.0) + label_smoothing / (double)c;
                dz[j] = (float)(grad_scale * (p - t) / (double)nvalid);
            }
    }
    if (loss) *loss = nvalid > 0 ? (float)(total / (double)nvalid) : NAN;
}

/* ------------------------------------------------------------- attention
 * kernel.hpp:26-95: s = (q·kᵀ)/sqrt(d) [here ·scale], causal triu(1) -> −inf,
 * p = softmax_j(s), o = p·v.  lse = log Σ_j exp(s_j).
 * Backward: dv = pᵀ·dO; dp = dO·vᵀ; ds = p∘(dp − rowsum(dp∘p)); dq = ds·k·scale; dk = dsᵀ·q·scale. */
static void attn_probs(const nott_attn_desc* d, const float* q, const float* k, int64_t bh, int64_t i, double* p,
                       double* lse_out) {
    const int64_t T = d->t, S = d->s, D = d->dh;
    double mx = -INFINITY;
    for (int64_t j = 0; j < S; ++j) {
        if (d->causal && j > i) {
            p[j] = -INFINITY;
            continue;
        }
        double acc = 0.0;
        for (int64_t e = 0; e < D; ++e) acc += (double)q[(bh * T + i) * D + e] * (double)k[(bh * S + j) * D + e];
        p[j] = acc * d->scale;
        if (p[j] > mx) mx = p[j];
    }
    double se = 0.0;
    for (int64_t j = 0; j < S; ++j) se += (p[j] == -INFINITY) ? 0.0 : exp(p[j] - mx);
    for (int64_t j = 0; j < S; ++j) p[j] = (p[j] == -INFINITY) ? 0.0 : exp(p[j] - mx) / se;
    if (lse_out) *lse_out = mx + log(se);
}

void oracle_attention_fwd(const nott_attn_desc* d, const float* q, const float* k, const float* v, float* o, float* lse) {
    const int64_t T = d->t, S = d->s, D = d->dh;
    double* p = (double*)malloc(sizeof(double) * (size_t)S);
    for (int64_t bh = 0; bh < d->b * d->h; ++bh)
        for (int64_t i = 0; i < T; ++i) {
            double l;
            attn_probs(d, q, k, bh, i, p, &l);
            if (lse) lse[bh * T + i] = (float)l;
            for (int64_t e = 0; e < D; ++e) {
                double acc = 0.0;
                for (int64_t j = 0; j < S; ++j) acc += p[j] * (double)v[(bh * S + j) * D + e];
                o[(bh * T + i) * D + e] = (float)acc;
            }
        }
    free(p);
}

void oracle_attention_bwd(const nott_attn_desc* d, const float* q, const float* k, const float* v, const float* o,
                          const float* dO, float* dq, float* dk, float* dv) {
    const int64_t T = d->t, S = d->s, D = d->dh;
    (void)o;
    double* p = (double*)malloc(sizeof(double) * (size_t)S);
    double* dp = (double*)malloc(sizeof(double) * (size_t)S);
    double* adk = (double*)calloc((size_t)(S * D), sizeof(double));
    double* adv = (double*)calloc((size_t)(S * D), sizeof(double));
    for (int64_t bh = 0; bh < d->b * d->h; ++bh) {
        memset(adk, 0, sizeof(double) * (size_t)(S * D));
        memset(adv, 0, sizeof(double) * (size_t)(S * D));
        for (int64_t i = 0; i < T; ++i) {
            attn_probs(d, q, k, bh, i, p, NULL);
            double rs = 0.0;
            for (int64_t j = 0; j < S; ++j) {
                double acc = 0.0;
                for (int64_t e = 0; e < D; ++e) acc += (double)dO[(bh * T + i) * D + e] * (double)v[(bh * S + j) * D + e];
                dp[j] = acc;
                rs += acc * p[j];
            }
            for (int64_t e = 0; e < D; ++e) {
                double acc = 0.0;
                for (int64_t j = 0; j < S; ++j) {
                    const double ds = p[j] * (dp[j] - rs);
                    acc += ds * (double)k[(bh * S + j) * D + e];
                }
                dq[(bh * T + i) * D + e] = (float)(acc * d->scale);
            }
            for (int64_t j = 0; j < S; ++j) {
                const double ds = p[j] * (dp[j] - rs);
                for (int64_t e = 0; e < D; ++e) {
                    adk[j * D + e] += ds * (double)q[(bh * T + i) * D + e] * d->scale;
                    adv[j * D + e] += p[j] * (double)dO[(bh * T + i) * D + e];
                }
            }
        }
        for (int64_t j = 0; j < S * D; ++j) {
            dk[bh * S * D + j] = (float)adk[j];
            dv[bh * S * D + j] = (float)adv[j];
        }
    }
    free(p);
    free(dp);
    free(adk);
    free(adv);
}

/* ------------------------------------------------------------------ adam
 * adam.hpp:63/159 -> torch::optim::Adam/AdamW::step, per element in fp32
 * with the scalars rounded from double as libtorch's tensor-scalar ops do.
 * The fused multiply-adds are where libtorch's vectorised CPU kernels use
 * them (add with alpha, addcmul); this order reproduces its outputs bit for
 * bit on the golden fixtures:
 *   AdamW: p = p·(1 − lr·wd)               Adam: g = fma(p, wd, g)   (wd != 0)
 *   m = fma(g, 1−β1, m·β1);  v = fma((1−β2)·g, g, v·β2)
 *   p = p + (−lr/bc1 · m) / (sqrt(v)/sqrt(bc2) + eps),  bc_i = 1 − β_i^t. */
void oracle_adam_step(int decoupled, int64_t n, float* p, const float* g, float* m, float* v, double lr, double beta1,
                      double beta2, double eps, double weight_decay, int64_t step) {
    const double bc1 = 1.0 - pow(beta1, (double)step);
    const double bc2 = 1.0 - pow(beta2, (double)step);
    const float fb1 = (float)beta1, fb2 = (float)beta2;
    const float a1 = (float)(1.0 - beta1), a2 = (float)(1.0 - beta2);
    const float fwd = (float)weight_decay, decay = (float)(1.0 - lr * weight_decay);
    const float neg_step = (float)(-(lr / bc1)), bc2s = (float)sqrt(bc2), feps = (float)eps;
    for (int64_t i = 0; i < n; ++i) {
        float pi = p[i], gi = g[i];
        if (weight_decay != 0.0) {
            if (decoupled)
                pi = pi * decay;
            else
                gi = fmaf(pi, fwd, gi);
        }
        const float mi = fmaf(gi, a1, m[i] * fb1);
        const float vi = fmaf(a2 * gi, gi, v[i] * fb2);
        const float denom = sqrtf(vi) / bc2s + feps;
        pi = pi + (neg_step * mi) / denom;
        p[i] = pi;
        m[i] = mi;
        v[i] = vi;
    }
}

void oracle_round_bf16(int64_t n, float* x) {
    for (int64_t i = 0; i < n; ++i) {
        uint32_t u;
        memcpy(&u, &x[i], 4);
        if ((u & 0x7fffffffu) > 0x7f800000u) {
            u = (u | 0x00400000u) & 0xffff0000u;
        } else {
            u += 0x7fffu + ((u >> 16) & 1u);
            u &= 0xffff0000u;
        }
        memcpy(&x[i], &u, 4);
    }
}
