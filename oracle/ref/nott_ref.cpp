// nott_ref.cpp — drives the REFERENCE's own modules (compiled from the
// headers under /root/reference/src, see oracle/ref/Makefile) on the CPU and
// exposes each hot-path op through a plain C ABI over host fp32 buffers.
//
// TEST INFRASTRUCTURE ONLY: built into oracle/_ref/libnott_ref.so, loaded by
// tests/golden/make_golden.py (to write fixtures), by tests when present, and
// by bench.py's cpu_baseline leg (kind "reference").  Nothing in the product
// path links or loads it.
//
// Each function builds the layer the way Nott's Model::add does
// (Layer::Details::build_registered_layer on an owner module), loads the given
// weights, runs forward + autograd backward exactly as libtorch does for the
// reference, and copies results out.
#include <torch/torch.h>

#include "activation/activation.hpp"
#include "activation/apply.hpp"
#include "initialization/initialization.hpp"
#include "initialization/apply.hpp"
#include "common/local.hpp"
#include "layer/details/conv.hpp"
#include "layer/details/fc.hpp"
#include "layer/details/pooling.hpp"
#include "layer/details/batchnorm.hpp"
#include "layer/details/flatten.hpp"
#include "loss/details/ce.hpp"
#include "optimizer/details/adam.hpp"
#include "attention/details/head.hpp"

#include <chrono>
#include <cstring>
#include <stdexcept>

#include "../../include/nott_hip.h"

namespace {

struct Owner : torch::nn::Module {};

torch::Tensor in(const float* p, std::vector<int64_t> shape) {
    return torch::from_blob(const_cast<float*>(p), shape, torch::kFloat32).clone();
}

torch::Tensor in64(const int64_t* p, std::vector<int64_t> shape) {
    return torch::from_blob(const_cast<int64_t*>(p), shape, torch::kInt64).clone();
}

void out(const torch::Tensor& t, float* dst) {
    if (!dst) return;
    auto c = t.detach().to(torch::kFloat32).contiguous();
    std::memcpy(dst, c.data_ptr<float>(), sizeof(float) * (size_t)c.numel());
}

void set_param(torch::nn::Module& m, const std::string& name, const torch::Tensor& v) {
    torch::NoGradGuard g;
    auto params = m.named_parameters(true);
    auto* p = params.find(name);
    if (!p) throw std::runtime_error("no parameter " + name);
    p->copy_(v);
}

torch::Tensor grad_of(torch::nn::Module& m, const std::string& name) {
    auto params = m.named_parameters(true);
    auto* p = params.find(name);
    if (!p) throw std::runtime_error("no parameter " + name);
    return p->grad();
}

template <class F>
int guarded(F&& f) {
    try {
        f();
        return 0;
    } catch (const std::exception& e) {
        fprintf(stderr, "nott_ref: %s\n", e.what());
        return -1;
    }
}

Nott::Layer::Details::Conv2dDescriptor conv_descriptor(const nott_conv2d_desc* d, bool bias) {
    Nott::Layer::Details::Conv2dDescriptor desc;
    desc.options.in_channels = d->c;
    desc.options.out_channels = d->k;
    desc.options.kernel_size = {d->r, d->s};
    desc.options.stride = {d->stride_h, d->stride_w};
    desc.options.padding = {d->pad_h, d->pad_w};
    desc.options.dilation = {d->dil_h, d->dil_w};
    desc.options.bias = bias;
    return desc;
}

// A chain of registered layers applied in order, each followed by its
// activation (Model::forward applies registered_layer.activation after the
// module, core.hpp:1719-1790).
struct Chain {
    Owner owner;
    std::vector<Nott::Layer::Details::RegisteredLayer> layers;
    size_t next = 0;
    template <class D>
    size_t add(const D& d) {
        layers.push_back(Nott::Layer::Details::build_registered_layer(owner, d, next++));
        return layers.size() - 1;
    }
    torch::Tensor run(size_t i, torch::Tensor x) {
        auto y = layers[i].forward(std::move(x));
        return Nott::Activation::Details::apply(layers[i].activation, std::move(y));
    }
};

Nott::Layer::Details::Conv2dDescriptor conv_d(int64_t ci, int64_t co, int64_t k, int64_t stride, int64_t pad,
                                              bool bias, bool relu) {
    Nott::Layer::Details::Conv2dDescriptor d;
    d.options.in_channels = ci;
    d.options.out_channels = co;
    d.options.kernel_size = {k, k};
    d.options.stride = {stride, stride};
    d.options.padding = {pad, pad};
    d.options.bias = bias;
    d.activation = relu ? Nott::Activation::ReLU : Nott::Activation::Identity;
    d.initialization = Nott::Initialization::HeUniform;
    return d;
}

Nott::Layer::Details::BatchNorm2dDescriptor bn_d(int64_t c, bool relu) {
    Nott::Layer::Details::BatchNorm2dDescriptor d;
    d.options.num_features = c;
    d.activation = relu ? Nott::Activation::ReLU : Nott::Activation::Identity;
    return d;
}

Nott::Layer::Details::FCDescriptor fc_d(int64_t in, int64_t out, bool relu) {
    Nott::Layer::Details::FCDescriptor d;
    d.options.in_features = in;
    d.options.out_features = out;
    d.activation = relu ? Nott::Activation::ReLU : Nott::Activation::Identity;
    d.initialization = Nott::Initialization::HeUniform;
    return d;
}

Nott::Layer::Details::PoolingDescriptor maxpool_d(int64_t k, int64_t stride, int64_t pad) {
    Nott::Layer::Details::MaxPool2dOptions o;
    o.kernel_size = {k, k};
    o.stride = {stride, stride};
    o.padding = {pad, pad};
    return Nott::Layer::Details::PoolingDescriptor{o};
}

// Conv(1->32)+ReLU+MaxPool2 -> Conv(32->64)+ReLU+MaxPool2 -> FC(3136->128)+ReLU -> FC(128->10).
struct SmallCnnRef {
    Chain c;
    SmallCnnRef() {
        c.add(conv_d(1, 32, 3, 1, 1, true, true));
        c.add(maxpool_d(2, 2, 0));
        c.add(conv_d(32, 64, 3, 1, 1, true, true));
        c.add(maxpool_d(2, 2, 0));
        c.add(Nott::Layer::Details::FlattenDescriptor{});
        c.add(fc_d(3136, 128, true));
        c.add(fc_d(128, 10, false));
    }
    torch::Tensor forward(torch::Tensor x) {
        for (size_t i = 0; i < c.layers.size(); ++i) x = c.run(i, x);
        return x;
    }
};

// ResNet-18 (7x7/2 stem + BN + ReLU + 3x3/2 max-pool, 4 stages of
// 2 basic blocks, global average pool, FC 512->1000) from the same layer
// descriptors; the residual add and the post-add ReLU are what Nott's
// residual block applies (block/details/blocks/residual.hpp:131-132).
struct ResNet18Ref {
    Chain c;
    struct Block { size_t c0, b0, c1, b1; long sc = -1, sb = -1; };
    size_t stem, stem_bn, pool, gap, flat, fc;
    std::vector<Block> blocks;
    ResNet18Ref() {
        stem = c.add(conv_d(3, 64, 7, 2, 3, false, false));
        stem_bn = c.add(bn_d(64, true));
        pool = c.add(maxpool_d(3, 2, 1));
        int64_t in = 64;
        const int64_t widths[4] = {64, 128, 256, 512};
        for (int st = 0; st < 4; ++st) {
            for (int j = 0; j < 2; ++j) {
                const int64_t out = widths[st], stride = (st > 0 && j == 0) ? 2 : 1;
                Block b;
                b.c0 = c.add(conv_d(in, out, 3, stride, 1, false, false));
                b.b0 = c.add(bn_d(out, true));
                b.c1 = c.add(conv_d(out, out, 3, 1, 1, false, false));
                b.b1 = c.add(bn_d(out, false));
                if (stride != 1 || in != out) {
                    b.sc = (long)c.add(conv_d(in, out, 1, stride, 0, false, false));
                    b.sb = (long)c.add(bn_d(out, false));
                }
                blocks.push_back(b);
                in = out;
            }
        }
        Nott::Layer::Details::AdaptiveAvgPool2dOptions ao;
        ao.output_size = {1, 1};
        gap = c.add(Nott::Layer::Details::PoolingDescriptor{ao});
        flat = c.add(Nott::Layer::Details::FlattenDescriptor{});
        fc = c.add(fc_d(512, 1000, false));
    }
    torch::Tensor forward(torch::Tensor x) {
        x = c.run(pool, c.run(stem_bn, c.run(stem, x)));
        for (auto& b : blocks) {
            auto y = c.run(b.b1, c.run(b.c1, c.run(b.b0, c.run(b.c0, x))));
            auto s = b.sc >= 0 ? c.run((size_t)b.sb, c.run((size_t)b.sc, x)) : x;
            x = torch::relu(y + s);
        }
        return c.run(fc, c.run(flat, c.run(gap, x)));
    }
};

template <class Net>
double time_train_steps(Net& net, torch::Tensor x, torch::Tensor y, bool decoupled, int iters) {
    net.c.owner.train();
    std::vector<torch::Tensor> params = net.c.owner.parameters();
    Nott::Loss::Details::CrossEntropyDescriptor ce;
    auto run = [&](auto& opt) {
        auto step = [&] {   // core.hpp:3757-3823: forward, loss, backward, step, zero_grad
            auto loss = Nott::Loss::Details::compute(ce, net.forward(x), y);
            loss.backward();
            opt.step();
            opt.zero_grad(false);
        };
        step();   // warm-up (also initialises the optimizer state)
        auto t0 = std::chrono::steady_clock::now();
        for (int i = 0; i < iters; ++i) step();
        auto t1 = std::chrono::steady_clock::now();
        return std::chrono::duration<double>(t1 - t0).count() / iters;
    };
    if (decoupled) {
        Nott::Optimizer::Details::AdamWOptions o;
        Nott::Optimizer::Details::AdamW opt(params, Nott::Optimizer::Details::to_torch_options(o));
        return run(opt);
    }
    Nott::Optimizer::Details::AdamOptions o;
    Nott::Optimizer::Details::Adam opt(params, Nott::Optimizer::Details::to_torch_options(o));
    return run(opt);
}

}  // namespace

extern "C" {

void ref_set_threads(int n) { torch::set_num_threads(n); }
int ref_get_threads(void) { return torch::get_num_threads(); }

// conv.hpp:140-191.  y = conv(x); then backward with dy.  Any output may be NULL.
int ref_conv2d(const nott_conv2d_desc* d, int with_bias, const float* x, const float* w, const float* b,
               const float* dy, float* y, float* dx, float* dw, float* db) {
    return guarded([&] {
        Owner owner;
        auto layer = Nott::Layer::Details::build_registered_layer(owner, conv_descriptor(d, with_bias != 0), 0);
        set_param(owner, "conv2d_0.weight", in(w, {d->k, d->c, d->r, d->s}));
        if (with_bias) set_param(owner, "conv2d_0.bias", in(b, {d->k}));
        auto xt = in(x, {d->n, d->c, d->h, d->w}).requires_grad_(true);
        auto yt = layer.forward(xt);
        out(yt, y);
        if (dy) {
            yt.backward(in(dy, yt.sizes().vec()));
            out(xt.grad(), dx);
            out(grad_of(owner, "conv2d_0.weight"), dw);
            if (with_bias) out(grad_of(owner, "conv2d_0.bias"), db);
        }
    });
}

// Times `iters` conv backward passes (dgrad + wgrad) on the CPU; returns
// seconds per pass in *sec.  Inputs as ref_conv2d (no bias).
int ref_conv2d_bwd_time(const nott_conv2d_desc* d, const float* x, const float* w, const float* dy, int iters,
                        double* sec) {
    return guarded([&] {
        Owner owner;
        auto layer = Nott::Layer::Details::build_registered_layer(owner, conv_descriptor(d, false), 0);
        set_param(owner, "conv2d_0.weight", in(w, {d->k, d->c, d->r, d->s}));
        auto xt = in(x, {d->n, d->c, d->h, d->w}).requires_grad_(true);
        auto yt = layer.forward(xt);
        auto g = in(dy, yt.sizes().vec());
        yt.backward(g, /*retain_graph=*/true);  // warm-up
        auto t0 = std::chrono::steady_clock::now();
        for (int i = 0; i < iters; ++i) yt.backward(g, /*retain_graph=*/true);
        auto t1 = std::chrono::steady_clock::now();
        *sec = std::chrono::duration<double>(t1 - t0).count() / iters;
    });
}

// fc.hpp:32-49.
int ref_linear(int64_t m, int64_t kin, int64_t nout, int with_bias, const float* x, const float* w, const float* b,
               const float* dy, float* y, float* dx, float* dw, float* db) {
    return guarded([&] {
        Owner owner;
        Nott::Layer::Details::FCDescriptor desc;
        desc.options.in_features = kin;
        desc.options.out_features = nout;
        desc.options.bias = with_bias != 0;
        auto layer = Nott::Layer::Details::build_registered_layer(owner, desc, 0);
        set_param(owner, "fc_0.weight", in(w, {nout, kin}));
        if (with_bias) set_param(owner, "fc_0.bias", in(b, {nout}));
        auto xt = in(x, {m, kin}).requires_grad_(true);
        auto yt = layer.forward(xt);
        out(yt, y);
        if (dy) {
            yt.backward(in(dy, {m, nout}));
            out(xt.grad(), dx);
            out(grad_of(owner, "fc_0.weight"), dw);
            if (with_bias) out(grad_of(owner, "fc_0.bias"), db);
        }
    });
}

// activation/apply.hpp:24 with Type::ReLU (relu.hpp:13).
int ref_relu(int64_t n, const float* x, const float* dy, float* y, float* dx) {
    return guarded([&] {
        auto xt = in(x, {n}).requires_grad_(true);
        auto yt = Nott::Activation::Details::apply(Nott::Activation::Type::ReLU, xt);
        out(yt, y);
        if (dy) {
            yt.backward(in(dy, {n}));
            out(xt.grad(), dx);
        }
    });
}

// pooling.hpp:132-149 (MaxPool2d).  argmax comes from the same module's
// forward_with_indices (the op its forward dispatches).
int ref_maxpool2d(const nott_pool2d_desc* d, const float* x, const float* dy, float* y, int64_t* argmax, float* dx) {
    return guarded([&] {
        Owner owner;
        Nott::Layer::Details::MaxPool2dOptions o;
        o.kernel_size = {d->kh, d->kw};
        o.stride = {d->stride_h, d->stride_w};
        o.padding = {d->pad_h, d->pad_w};
        o.dilation = {d->dil_h, d->dil_w};
        o.ceil_mode = d->ceil_mode != 0;
        Nott::Layer::Details::PoolingDescriptor desc{o};
        auto layer = Nott::Layer::Details::build_registered_layer(owner, desc, 0);
        auto* impl = dynamic_cast<torch::nn::MaxPool2dImpl*>(layer.module.get());
        if (!impl) throw std::runtime_error("not a MaxPool2d");
        auto xt = in(x, {d->n, d->c, d->h, d->w}).requires_grad_(true);
        auto yt = layer.forward(xt);
        out(yt, y);
        if (argmax) {
            torch::NoGradGuard ng;
            auto pair = impl->forward_with_indices(xt.detach());
            auto idx = std::get<1>(pair).contiguous();
            std::memcpy(argmax, idx.data_ptr<int64_t>(), sizeof(int64_t) * (size_t)idx.numel());
        }
        if (dy) {
            yt.backward(in(dy, yt.sizes().vec()));
            out(xt.grad(), dx);
        }
    });
}

// pooling.hpp:164-167 (AdaptiveAvgPool2d {1,1}).
int ref_avgpool_global(int64_t n, int64_t c, int64_t h, int64_t w, const float* x, const float* dy, float* y, float* dx) {
    return guarded([&] {
        Owner owner;
        Nott::Layer::Details::AdaptiveAvgPool2dOptions o;
        o.output_size = {1, 1};
        Nott::Layer::Details::PoolingDescriptor desc{o};
        auto layer = Nott::Layer::Details::build_registered_layer(owner, desc, 0);
        auto xt = in(x, {n, c, h, w}).requires_grad_(true);
        auto yt = layer.forward(xt);
        out(yt, y);
        if (dy) {
            yt.backward(in(dy, {n, c, 1, 1}));
            out(xt.grad(), dx);
        }
    });
}

// batchnorm.hpp:38-59, training mode.  Running stats in/out (may be NULL).
int ref_batchnorm2d(int64_t n, int64_t c, int64_t h, int64_t w, double eps, double momentum, const float* x,
                    const float* gamma, const float* beta, const float* dy, float* running_mean, float* running_var,
                    float* y, float* dx, float* dgamma, float* dbeta) {
    return guarded([&] {
        Owner owner;
        Nott::Layer::Details::BatchNorm2dDescriptor desc;
        desc.options.num_features = c;
        desc.options.eps = eps;
        desc.options.momentum = momentum;
        auto layer = Nott::Layer::Details::build_registered_layer(owner, desc, 0);
        owner.train();
        set_param(owner, "batchnorm2d_0.weight", in(gamma, {c}));
        set_param(owner, "batchnorm2d_0.bias", in(beta, {c}));
        auto* impl = dynamic_cast<torch::nn::BatchNorm2dImpl*>(layer.module.get());
        if (!impl) throw std::runtime_error("not a BatchNorm2d");
        if (running_mean) {
            torch::NoGradGuard ng;
            impl->running_mean.copy_(in(running_mean, {c}));
            impl->running_var.copy_(in(running_var, {c}));
        }
        auto xt = in(x, {n, c, h, w}).requires_grad_(true);
        auto yt = layer.forward(xt);
        out(yt, y);
        if (running_mean) {
            out(impl->running_mean, running_mean);
            out(impl->running_var, running_var);
        }
        if (dy) {
            yt.backward(in(dy, {n, c, h, w}));
            out(xt.grad(), dx);
            out(grad_of(owner, "batchnorm2d_0.weight"), dgamma);
            out(grad_of(owner, "batchnorm2d_0.bias"), dbeta);
        }
    });
}

// LayerNorm as TransformerEncoderLayerImpl builds it
// (block/details/transformers/classic.hpp:399-404; options :54-57).
int ref_layernorm(int64_t rows, int64_t d, double eps, const float* x, const float* gamma, const float* beta,
                  const float* dy, float* y, float* dx, float* dgamma, float* dbeta) {
    return guarded([&] {
        auto norm_options = torch::nn::LayerNormOptions(std::vector<int64_t>{d}).eps(eps).elementwise_affine(true);
        torch::nn::LayerNorm ln(norm_options);
        {
            torch::NoGradGuard ng;
            ln->weight.copy_(in(gamma, {d}));
            ln->bias.copy_(in(beta, {d}));
        }
        auto xt = in(x, {rows, d}).requires_grad_(true);
        auto yt = ln->forward(xt);
        out(yt, y);
        if (dy) {
            yt.backward(in(dy, {rows, d}));
            out(xt.grad(), dx);
            out(ln->weight.grad(), dgamma);
            out(ln->bias.grad(), dbeta);
        }
    });
}

// ce.hpp:21-37, mean reduction; loss.backward() as core.hpp:3819 does.
int ref_cross_entropy(int64_t n, int64_t c, double label_smoothing, const float* logits, const int64_t* labels,
                      float* loss, float* dlogits) {
    return guarded([&] {
        Nott::Loss::Details::CrossEntropyDescriptor desc;
        desc.options.label_smoothing = label_smoothing;
        auto z = in(logits, {n, c}).requires_grad_(true);
        auto l = Nott::Loss::Details::compute(desc, z, in64(labels, {n}));
        if (loss) *loss = l.item<float>();
        l.backward();
        out(z.grad(), dlogits);
    });
}

// adam.hpp:63-154 / 159-250.  State is initialised by the wrapper's
// ensure_state_initialized (step 0, zero moments), then set to (step-1, m, v)
// so that the call performs step number `step`.  p, m, v updated in place.
int ref_adam_step(int decoupled, int64_t n, float* p, const float* g, float* m, float* v, double lr, double beta1,
                  double beta2, double eps, double weight_decay, int64_t step) {
    return guarded([&] {
        auto pt = in(p, {n}).requires_grad_(true);
        pt.mutable_grad() = in(g, {n});
        auto run = [&](auto& opt) {
            opt.ensure_state_initialized();
            auto& st = opt.state();
            auto it = st.find(pt.unsafeGetTensorImpl());
            if (it == st.end()) throw std::runtime_error("adam state missing");
            using State = std::conditional_t<std::is_same_v<std::decay_t<decltype(opt)>, Nott::Optimizer::Details::AdamW>,
                                             torch::optim::AdamWParamState, torch::optim::AdamParamState>;
            auto& s = static_cast<State&>(*it->second);
            s.step(step - 1);
            s.exp_avg().copy_(in(m, {n}));
            s.exp_avg_sq().copy_(in(v, {n}));
            opt.step();
            out(pt, p);
            out(s.exp_avg(), m);
            out(s.exp_avg_sq(), v);
        };
        if (decoupled) {
            Nott::Optimizer::Details::AdamWOptions o;
            o.learning_rate = lr;
            o.beta1 = beta1;
            o.beta2 = beta2;
            o.eps = eps;
            o.weight_decay = weight_decay;
            Nott::Optimizer::Details::AdamW opt(std::vector<at::Tensor>{pt}, Nott::Optimizer::Details::to_torch_options(o));
            run(opt);
        } else {
            Nott::Optimizer::Details::AdamOptions o;
            o.learning_rate = lr;
            o.beta1 = beta1;
            o.beta2 = beta2;
            o.eps = eps;
            o.weight_decay = weight_decay;
            Nott::Optimizer::Details::Adam opt(std::vector<at::Tensor>{pt}, Nott::Optimizer::Details::to_torch_options(o));
            run(opt);
        }
    });
}

// Times `iters` AdamW steps over a flat n-element buffer; seconds per step.
int ref_adamw_time(int64_t n, int iters, double* sec) {
    return guarded([&] {
        auto pt = (torch::randn({n}) * 0.02).requires_grad_(true);
        pt.mutable_grad() = torch::randn({n}) * 1e-3;
        Nott::Optimizer::Details::AdamWOptions o;
        o.learning_rate = 3e-4;
        o.weight_decay = 0.01;
        Nott::Optimizer::Details::AdamW opt(std::vector<at::Tensor>{pt}, Nott::Optimizer::Details::to_torch_options(o));
        opt.ensure_state_initialized();
        opt.step();
        auto t0 = std::chrono::steady_clock::now();
        for (int i = 0; i < iters; ++i) opt.step();
        auto t1 = std::chrono::steady_clock::now();
        *sec = std::chrono::duration<double>(t1 - t0).count() / iters;
    });
}

// kernel.hpp:20-96 (ScaledDotProductKernel; Variant::Causal when causal).
int ref_attention(const nott_attn_desc* d, const float* q, const float* k, const float* v, const float* dO, float* o,
                  float* dq, float* dk, float* dv) {
    return guarded([&] {
        Nott::Attention::Details::ScaledDotProductKernel kernel(
            0.0, d->causal ? Nott::Attention::Variant::Causal : Nott::Attention::Variant::Full);
        auto qt = in(q, {d->b, d->h, d->t, d->dh}).requires_grad_(true);
        auto kt = in(k, {d->b, d->h, d->s, d->dh}).requires_grad_(true);
        auto vt = in(v, {d->b, d->h, d->s, d->dh}).requires_grad_(true);
        auto ot = kernel->forward(qt, kt, vt);
        out(ot, o);
        if (dO) {
            ot.backward(in(dO, {d->b, d->h, d->t, d->dh}));
            out(qt.grad(), dq);
            out(kt.grad(), dk);
            out(vt.grad(), dv);
        }
    });
}

// head.hpp:22-98 (MultiHeadAttention, self-attention x=q=k=v, batch_first).
// Weights: wq, wk, wv, wo [e, e], biases bq.. [e] (nullable when !with_bias).
int ref_mha(int64_t b, int64_t t, int64_t e, int64_t heads, int causal, int with_bias, const float* x,
            const float* wq, const float* wk, const float* wv, const float* wo, const float* bq, const float* bk,
            const float* bv, const float* bo, const float* dy, float* y, float* dx, float* dwq, float* dwk, float* dwv,
            float* dwo, float* dbq, float* dbk, float* dbv, float* dbo) {
    return guarded([&] {
        Nott::Attention::Details::MultiHeadAttentionOptions o;
        o.embed_dim = e;
        o.num_heads = heads;
        o.dropout = 0.0;
        o.bias = with_bias != 0;
        o.batch_first = true;
        o.variant = causal ? Nott::Attention::Variant::Causal : Nott::Attention::Variant::Full;
        Nott::Attention::Details::MultiHeadAttention mha(o);
        set_param(*mha, "q_proj.weight", in(wq, {e, e}));
        set_param(*mha, "k_proj.weight", in(wk, {e, e}));
        set_param(*mha, "v_proj.weight", in(wv, {e, e}));
        set_param(*mha, "out_proj.weight", in(wo, {e, e}));
        if (with_bias) {
            set_param(*mha, "q_proj.bias", in(bq, {e}));
            set_param(*mha, "k_proj.bias", in(bk, {e}));
            set_param(*mha, "v_proj.bias", in(bv, {e}));
            set_param(*mha, "out_proj.bias", in(bo, {e}));
        }
        auto xt = in(x, {b, t, e}).requires_grad_(true);
        auto yt = mha->forward(xt, xt, xt);
        out(yt, y);
        if (dy) {
            yt.backward(in(dy, {b, t, e}));
            out(xt.grad(), dx);
            out(grad_of(*mha, "q_proj.weight"), dwq);
            out(grad_of(*mha, "k_proj.weight"), dwk);
            out(grad_of(*mha, "v_proj.weight"), dwv);
            out(grad_of(*mha, "out_proj.weight"), dwo);
            if (with_bias) {
                out(grad_of(*mha, "q_proj.bias"), dbq);
                out(grad_of(*mha, "k_proj.bias"), dbk);
                out(grad_of(*mha, "v_proj.bias"), dbv);
                out(grad_of(*mha, "out_proj.bias"), dbo);
            }
        }
    });
}

// Loads a parameters.binary archive (torch::nn::Module::save layout, keys by
// Nott's registration names) into the configs[0] model built from the
// reference's descriptors and runs its forward on x[batch,1,28,28]; logits
// [batch,10].  Checks that a checkpoint written by another implementation
// loads into the reference (core.hpp:2188-2236 reads the same archive).
int ref_small_cnn_forward_archive(const char* path, int64_t batch, const float* x, float* logits) {
    return guarded([&] {
        SmallCnnRef net;
        torch::serialize::InputArchive ar;
        ar.load_from(std::string(path));
        net.c.owner.load(ar);
        torch::NoGradGuard ng;
        auto y = net.forward(in(x, {batch, 1, 28, 28}));
        out(y, logits);
    });
}

// Times `iters` full fp32 training steps on the CPU (forward, CE mean,
// backward, Adam (model 0, configs[0]) or AdamW (model 1, configs[4]) step,
// zero_grad) at the given batch; seconds per step in *sec.  Inputs
// uniform[0,1), labels uniform, weights HeUniform from torch's CPU generator.
int ref_train_step_time(int model, int64_t batch, int iters, double* sec) {
    return guarded([&] {
        torch::manual_seed(0);
        if (model == 0) {
            SmallCnnRef net;
            auto x = torch::rand({batch, 1, 28, 28});
            auto y = torch::randint(0, 10, {batch}, torch::kInt64);
            *sec = time_train_steps(net, x, y, false, iters);
        } else if (model == 1) {
            ResNet18Ref net;
            auto x = torch::rand({batch, 3, 224, 224});
            auto y = torch::randint(0, 1000, {batch}, torch::kInt64);
            *sec = time_train_steps(net, x, y, true, iters);
        } else {
            throw std::invalid_argument("model must be 0 (small CNN) or 1 (ResNet-18)");
        }
    });
}

}  // extern "C"
