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

#include <algorithm>
#include <chrono>
#include <optional>
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

// Rounds a tensor to bf16 and back in the forward, and its gradient the same
// way in the backward: placed where a bf16 mixed-precision implementation
// stores activations (and, in the backward, the gradients of those
// activations), it turns the fp32 reference into the same computation with
// bf16 storage.
struct RoundBF16 : torch::autograd::Function<RoundBF16> {
    static torch::Tensor forward(torch::autograd::AutogradContext*, torch::Tensor x) {
        return x.to(torch::kBFloat16).to(x.scalar_type());
    }
    static torch::autograd::variable_list backward(torch::autograd::AutogradContext*,
                                                   torch::autograd::variable_list g) {
        return {g[0].to(torch::kBFloat16).to(g[0].scalar_type())};
    }
};
inline torch::Tensor store(torch::Tensor t, bool bf16) { return bf16 ? RoundBF16::apply(t) : t; }

// Nott's residual block (block/details/blocks/residual.hpp:37-141) cannot be
// compiled here: residual.hpp includes layer/layer.hpp, whose
// details/recurrent.hpp:14 includes <ATen/cuda/CUDAContext.h>, which needs
// the CUDA runtime headers this ROCm image does not have.  ResidualRef
// restates the block over the reference's own layer factories, which do
// compile: one repeat of its layers registered by build_registered_layer on
// the block with running indices, then the projection (residual.hpp:49-62),
// and the forward of residual.hpp:87-132 — the branch through every layer
// and its activation, the skip through the projection and its activation,
// their sum, then the final activation (dropout 0 registers nothing).
struct ResidualRef : torch::nn::Module {
    std::vector<Nott::Layer::Details::RegisteredLayer> layers;
    std::optional<Nott::Layer::Details::RegisteredLayer> projection;
    Nott::Activation::Type final_activation;
    template <class... D>
    ResidualRef(Nott::Activation::Type final_act, const std::optional<Nott::Layer::Details::Conv2dDescriptor>& proj,
                const D&... ds)
        : final_activation(final_act) {
        size_t index = 0;
        (layers.push_back(Nott::Layer::Details::build_registered_layer(*this, ds, index++)), ...);
        if (proj) projection = Nott::Layer::Details::build_registered_layer(*this, *proj, index++);
    }
    // bf16: activations stored in bf16 after each layer but the last (whose
    // output is summed with the skip before one rounding), after the
    // projection and after the final activation.
    torch::Tensor forward(torch::Tensor input, bool bf16 = false) {
        auto branch = input;
        for (size_t i = 0; i < layers.size(); ++i) {
            branch = Nott::Activation::Details::apply(layers[i].activation, layers[i].forward(branch));
            if (i + 1 < layers.size()) branch = store(branch, bf16);
        }
        auto skip = input;
        if (projection)
            skip = store(Nott::Activation::Details::apply(projection->activation, projection->forward(skip)), bf16);
        return store(Nott::Activation::Details::apply(final_activation, branch + skip), bf16);
    }
};

// ResNet-18 assembled the way a Nott model registers it
// (core.hpp:516-523 layers, 576-592 residual blocks): the stem Conv2d,
// BatchNorm2d with ReLU and MaxPool2d under conv2d_0 / batchnorm2d_1 /
// maxpool2d_2, eight residual blocks under residual_block_3 ..
// residual_block_10 ({Conv2d, BatchNorm2d+ReLU, Conv2d, BatchNorm2d}, a 1×1
// stride-2 Conv2d projection on each down-sampling block, final ReLU), then
// adaptive_avgpool2d_11, flatten_12 and fc_13.
struct ResNet18Ref {
    Owner owner;
    std::vector<Nott::Layer::Details::RegisteredLayer> head, tail;
    std::vector<std::shared_ptr<ResidualRef>> blocks;
    size_t index = 0;
    ResNet18Ref() {
        head.push_back(Nott::Layer::Details::build_registered_layer(owner, conv_d(3, 64, 7, 2, 3, false, false), index++));
        head.push_back(Nott::Layer::Details::build_registered_layer(owner, bn_d(64, true), index++));
        head.push_back(Nott::Layer::Details::build_registered_layer(owner, maxpool_d(3, 2, 1), index++));
        int64_t in = 64;
        const int64_t widths[4] = {64, 128, 256, 512};
        for (int st = 0; st < 4; ++st)
            for (int j = 0; j < 2; ++j) {
                const int64_t out = widths[st], stride = (st > 0 && j == 0) ? 2 : 1;
                std::optional<Nott::Layer::Details::Conv2dDescriptor> proj;
                if (stride != 1 || in != out) proj = conv_d(in, out, 1, stride, 0, false, false);
                auto block = std::make_shared<ResidualRef>(Nott::Activation::Type::ReLU, proj,
                                                           conv_d(in, out, 3, stride, 1, false, false), bn_d(out, true),
                                                           conv_d(out, out, 3, 1, 1, false, false), bn_d(out, false));
                blocks.push_back(owner.register_module("residual_block_" + std::to_string(index++), block));
                in = out;
            }
        Nott::Layer::Details::AdaptiveAvgPool2dOptions ao;
        ao.output_size = {1, 1};
        tail.push_back(Nott::Layer::Details::build_registered_layer(owner, Nott::Layer::Details::PoolingDescriptor{ao}, index++));
        tail.push_back(Nott::Layer::Details::build_registered_layer(owner, Nott::Layer::Details::FlattenDescriptor{}, index++));
        tail.push_back(Nott::Layer::Details::build_registered_layer(owner, fc_d(512, 1000, false), index++));
    }
    static torch::Tensor run(const Nott::Layer::Details::RegisteredLayer& l, torch::Tensor x) {
        return Nott::Activation::Details::apply(l.activation, l.forward(std::move(x)));
    }
    // Model::forward over the registered layers (core.hpp:1926-1936); the
    // stem output and every block output go to `outs` when given.
    // bf16: every layer's output stored in bf16 (the flatten is a view).
    torch::Tensor forward(torch::Tensor x, std::vector<torch::Tensor>* outs = nullptr, bool bf16 = false) {
        for (auto& l : head) x = store(run(l, x), bf16);
        if (outs) outs->push_back(x);
        for (auto& b : blocks) {
            x = b->forward(x, bf16);
            if (outs) outs->push_back(x);
        }
        for (auto& l : tail) x = store(run(l, x), bf16);
        return x;
    }
};

torch::nn::Module& owner_of(SmallCnnRef& n) { return n.c.owner; }
torch::nn::Module& owner_of(ResNet18Ref& n) { return n.owner; }

// Median seconds of `iters` timed calls of fn after 5 untimed warm-up calls.
constexpr int kTimingWarmup = 5;
template <class F>
double median_seconds(int iters, F&& fn) {
    for (int i = 0; i < kTimingWarmup; ++i) fn();
    std::vector<double> t(std::max(iters, 1));
    for (auto& s : t) {
        const auto t0 = std::chrono::steady_clock::now();
        fn();
        s = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    }
    std::sort(t.begin(), t.end());
    const size_t m = t.size() / 2;
    return t.size() % 2 ? t[m] : 0.5 * (t[m - 1] + t[m]);
}

template <class Net>
double time_train_steps(Net& net, torch::Tensor x, torch::Tensor y, bool decoupled, int iters) {
    owner_of(net).train();
    std::vector<torch::Tensor> params = owner_of(net).parameters();
    Nott::Loss::Details::CrossEntropyDescriptor ce;
    auto run = [&](auto& opt) {
        auto step = [&] {   // core.hpp:3757-3823: forward, loss, backward, step, zero_grad
            auto loss = Nott::Loss::Details::compute(ce, net.forward(x), y);
            loss.backward();
            opt.step();
            opt.zero_grad(false);
        };
        return median_seconds(iters, step);   // the warm-ups also initialise the optimizer state
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

// Times conv backward passes (dgrad + wgrad) on the CPU; *sec is the median
// seconds of `iters` timed passes after 5 warm-ups (as every *_time below).  Inputs as ref_conv2d (no bias).
int ref_conv2d_bwd_time(const nott_conv2d_desc* d, const float* x, const float* w, const float* dy, int iters,
                        double* sec) {
    return guarded([&] {
        Owner owner;
        auto layer = Nott::Layer::Details::build_registered_layer(owner, conv_descriptor(d, false), 0);
        set_param(owner, "conv2d_0.weight", in(w, {d->k, d->c, d->r, d->s}));
        auto xt = in(x, {d->n, d->c, d->h, d->w}).requires_grad_(true);
        auto yt = layer.forward(xt);
        auto g = in(dy, yt.sizes().vec());
        *sec = median_seconds(iters, [&] { yt.backward(g, /*retain_graph=*/true); });
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

// Times AdamW steps over a flat n-element buffer; median seconds per step.
int ref_adamw_time(int64_t n, int iters, double* sec) {
    return guarded([&] {
        auto pt = (torch::randn({n}) * 0.02).requires_grad_(true);
        pt.mutable_grad() = torch::randn({n}) * 1e-3;
        Nott::Optimizer::Details::AdamWOptions o;
        o.learning_rate = 3e-4;
        o.weight_decay = 0.01;
        Nott::Optimizer::Details::AdamW opt(std::vector<at::Tensor>{pt}, Nott::Optimizer::Details::to_torch_options(o));
        opt.ensure_state_initialized();
        *sec = median_seconds(iters, [&] { opt.step(); });
    });
}

// Seconds per call of the ATen op LayerNorm's autograd node runs backward
// (native_layer_norm_backward, for the norms of classic.hpp:403-404) on
// x ~ N(0,1) [rows, d], gamma ~ N(1, 0.1), beta = 0, dy ~ N(0,1).
int ref_layernorm_bwd_time(int64_t rows, int64_t d, int iters, double* sec) {
    return guarded([&] {
        torch::manual_seed(1);
        auto x = torch::randn({rows, d});
        auto gamma = 1 + 0.1 * torch::randn({d});
        auto beta = torch::zeros({d});
        auto dy = torch::randn({rows, d});
        auto fwd = at::native_layer_norm(x, {d}, gamma, beta, 1e-5);
        const auto& mean = std::get<1>(fwd);
        const auto& rstd = std::get<2>(fwd);
        auto once = [&] { return at::native_layer_norm_backward(dy, x, {d}, mean, rstd, gamma, beta, {true, true, true}); };
        *sec = median_seconds(iters, once);
    });
}

// Seconds per forward + backward of Nott's CrossEntropy loss (ce.hpp:21-37,
// mean reduction; log_softmax + nll_loss and their backward, as
// core.hpp:3777-3819 runs them) on logits ~ N(0, 2) [n, c], labels uniform.
int ref_cross_entropy_time(int64_t n, int64_t c, int iters, double* sec) {
    return guarded([&] {
        torch::manual_seed(2);
        auto z = (2 * torch::randn({n, c})).requires_grad_(true);
        auto y = torch::randint(0, c, {n}, torch::kInt64);
        Nott::Loss::Details::CrossEntropyDescriptor desc;
        auto once = [&] {
            auto l = Nott::Loss::Details::compute(desc, z, y);
            l.backward();
            z.mutable_grad().reset();
        };
        *sec = median_seconds(iters, once);
    });
}

// Seconds per backward pass of Nott's MultiHeadAttention (head.hpp:22-98,
// self-attention, batch_first, with bias) through its saved graph: x ~ N(0,1)
// [b, t, e], weights ~ N(0, 0.02), dy ~ N(0,1).  The graph is kept between
// passes (retain_graph), so only the backward is timed.
int ref_mha_bwd_time(int64_t b, int64_t t, int64_t e, int64_t heads, int causal, int iters, double* sec) {
    return guarded([&] {
        torch::manual_seed(5);
        Nott::Attention::Details::MultiHeadAttentionOptions o;
        o.embed_dim = e;
        o.num_heads = heads;
        o.dropout = 0.0;
        o.bias = true;
        o.batch_first = true;
        o.variant = causal ? Nott::Attention::Variant::Causal : Nott::Attention::Variant::Full;
        Nott::Attention::Details::MultiHeadAttention mha(o);
        for (const char* w : {"q_proj.weight", "k_proj.weight", "v_proj.weight", "out_proj.weight"})
            set_param(*mha, w, 0.02 * torch::randn({e, e}));
        auto xt = torch::randn({b, t, e}).requires_grad_(true);
        auto yt = mha->forward(xt, xt, xt);
        auto dy = torch::randn({b, t, e});
        *sec = median_seconds(iters, [&] { yt.backward(dy, /*retain_graph=*/true); });
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

// One configs[4] training step of the reference's ResNet-18 (ResNet18Ref) on
// the CPU, in the order of Model::run_training_step (core.hpp:3757-3823):
// forward in training mode, CrossEntropy mean (ce.hpp:21-37), backward,
// AdamW(lr, weight_decay) step (adam.hpp:159-250).  Tensors are exchanged by
// their registration keys: for each of the `count` names, init[i] (nullable)
// sets the parameter or float buffer before the step, grads_out[i]
// (nullable) receives the parameter's gradient, after_out[i] (nullable) its
// value after the step (buffers: after the forward).  block_outs (nullable)
// receives the stem output and the 8 block outputs, in that order.
//
// precision 1 runs the same step with the model, input, loss and optimizer
// in double precision (the exact-arithmetic yardstick both fp32 paths are
// measured against); results are still returned as fp32.  precision 2 runs
// it in fp32 with every activation and activation gradient rounded to bf16
// where a bf16 mixed-precision step stores them (RoundBF16).
int ref_resnet18_step(int64_t batch, const float* x, const int64_t* labels, double lr, double weight_decay,
                      int64_t count, const char* const* names, const float* const* init, float* const* grads_out,
                      float* const* after_out, float* loss, float* logits, float* const* block_outs, int precision) {
    return guarded([&] {
        ResNet18Ref net;
        net.owner.train();
        auto params = net.owner.named_parameters(true);
        auto bufs = net.owner.named_buffers(true);
        auto find = [&](const char* name) -> torch::Tensor* {
            if (auto* p = params.find(name)) return p;
            if (auto* b = bufs.find(name)) return b;
            throw std::runtime_error(std::string("no parameter or buffer ") + name);
        };
        {
            torch::NoGradGuard ng;
            for (int64_t i = 0; i < count; ++i)
                if (init && init[i]) {
                    torch::Tensor* t = find(names[i]);
                    t->copy_(in(init[i], t->sizes().vec()));
                }
        }
        auto xt = in(x, {batch, 3, 224, 224});
        if (precision == 1) {
            net.owner.to(torch::kDouble);
            xt = xt.to(torch::kDouble);
            params = net.owner.named_parameters(true);
            bufs = net.owner.named_buffers(true);
        }
        std::vector<torch::Tensor> outs;
        auto z = net.forward(xt, block_outs ? &outs : nullptr, precision == 2);
        out(z, logits);
        Nott::Loss::Details::CrossEntropyDescriptor ce;
        auto l = Nott::Loss::Details::compute(ce, z, in64(labels, {batch}));
        if (loss) *loss = (float)l.item<double>();
        l.backward();
        for (int64_t i = 0; i < count; ++i)
            if (grads_out && grads_out[i]) out(find(names[i])->grad(), grads_out[i]);
        if (block_outs)
            for (size_t j = 0; j < outs.size(); ++j) out(outs[j], block_outs[j]);
        Nott::Optimizer::Details::AdamWOptions o;
        o.learning_rate = lr;
        o.weight_decay = weight_decay;
        Nott::Optimizer::Details::AdamW opt(net.owner.parameters(), Nott::Optimizer::Details::to_torch_options(o));
        opt.step();
        opt.zero_grad(false);
        for (int64_t i = 0; i < count; ++i)
            if (after_out && after_out[i]) out(*find(names[i]), after_out[i]);
    });
}

// Loads a parameters.binary archive into the reference's ResNet-18 and runs
// its training-mode forward on x[batch,3,224,224]; logits [batch,1000].
int ref_resnet18_forward_archive(const char* path, int64_t batch, const float* x, float* logits) {
    return guarded([&] {
        ResNet18Ref net;
        torch::serialize::InputArchive ar;
        ar.load_from(std::string(path));
        net.owner.load(ar);
        net.owner.train();
        torch::NoGradGuard ng;
        out(net.forward(in(x, {batch, 3, 224, 224})), logits);
    });
}

// Writes parameters.binary (torch::nn::Module::save, the archive
// Model::save stores, core.hpp:2131-2135) of the reference's configs[0]
// (model 0) or configs[4] (model 1) model: weights as its layer factories
// initialise them from torch's CPU generator seeded with `seed`, then one
// training-mode forward on uniform inputs so that the BatchNorm running
// statistics and batch counters are not at their initial values.
int ref_save_archive(int model, uint64_t seed, int64_t batch, const char* path) {
    return guarded([&] {
        torch::manual_seed(seed);
        torch::serialize::OutputArchive ar;
        if (model == 0) {
            SmallCnnRef net;
            torch::NoGradGuard ng;
            net.c.owner.train();
            (void)net.forward(torch::rand({batch, 1, 28, 28}));
            net.c.owner.save(ar);
        } else if (model == 1) {
            ResNet18Ref net;
            torch::NoGradGuard ng;
            net.owner.train();
            (void)net.forward(torch::rand({batch, 3, 224, 224}));
            net.owner.save(ar);
        } else {
            throw std::invalid_argument("model must be 0 (small CNN) or 1 (ResNet-18)");
        }
        ar.save_to(std::string(path));
    });
}

// The initial parameters of the reference's configs[0] (model 0) or
// configs[4] (model 1) model when torch's CPU generator is seeded with
// `seed` right before the model is built: each layer factory constructs its
// torch::nn module (whose constructor draws its default initialisation) and
// then applies the descriptor's HeUniform (initialization/apply.hpp:45-51).
// For each of the `count` registration keys, outs[i] receives that parameter.
int ref_init_params(int model, uint64_t seed, int64_t count, const char* const* names, float* const* outs) {
    return guarded([&] {
        torch::manual_seed(seed);
        auto copy_out = [&](torch::nn::Module& m) {
            auto params = m.named_parameters(true);
            for (int64_t i = 0; i < count; ++i) {
                auto* p = params.find(names[i]);
                if (!p) throw std::runtime_error(std::string("no parameter ") + names[i]);
                out(*p, outs[i]);
            }
        };
        if (model == 0) {
            SmallCnnRef net;
            copy_out(net.c.owner);
        } else if (model == 1) {
            ResNet18Ref net;
            copy_out(net.owner);
        } else {
            throw std::invalid_argument("model must be 0 (small CNN) or 1 (ResNet-18)");
        }
    });
}

// Times full fp32 training steps on the CPU (forward, CE mean,
// backward, Adam (model 0, configs[0]) or AdamW (model 1, configs[4]) step,
// zero_grad) at the given batch; median seconds per step in *sec.  Inputs
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
