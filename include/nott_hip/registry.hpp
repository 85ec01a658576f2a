// Nott's layer factory bound to the HIP modules.
//
// Nott builds every layer through Nott::Layer::Details::build_registered_layer
// (src/layer/registry.hpp:186-200): one function template per descriptor,
// generic in the owner that registers the module (Model::add, core.hpp:
// 516-523; Sequential and Residual blocks, block/details/blocks/
// sequential.hpp:26, residual.hpp:53-62).  This header adds, in the same
// namespace, overloads for the descriptors on the training hot path
//
//   Conv2dDescriptor       (reference conv.hpp:140-191)
//   FCDescriptor           (fc.hpp:32-49)
//   BatchNorm2dDescriptor  (batchnorm.hpp:38-59)
//   PoolingDescriptor      (pooling.hpp:81-200: MaxPool2d, AdaptiveAvgPool2d to 1×1)
//   FlattenDescriptor      (flatten.hpp:59-70)
//
// that register the Nott::HIP modules of host.hpp instead of torch::nn's and
// return the reference's own RegisteredLayer.  They are constrained
// templates with the reference's signatures, so for an owner that opts in
// (Nott::HIP::enable_layers<Owner>) overload resolution prefers them, and
// for every other owner nothing changes.  Every other descriptor keeps the
// reference's factory.
//
// What stays the same as the reference's factory:
//  * the registration key (`conv2d_<i>`, `fc_<i>`, `batchnorm2d_<i>`,
//    `maxpool2d_<i>`, `adaptive_avgpool2d_<i>`, `flatten_<i>`) and the
//    parameter and buffer names under it, so checkpoints line up;
//  * the initial values: the torch::nn module the reference would build is
//    constructed (its constructor draws its default initialisation from the
//    default generator), its tensors are copied into the HIP module, and then
//    the reference's own apply_module_initialization runs on the HIP module,
//    so after torch::manual_seed(s) both factories produce the same weights;
//  * the option checks and their exception type (std::invalid_argument).
//
// What differs: a ReLU activation is fused into the layer's HIP forward
// (the RegisteredLayer then reports Identity, so Model::forward's
// Activation::Details::apply is a no-op); other activations are left to the
// caller as the reference leaves them.  Options the HIP kernels do not
// implement (grouped convolution, non-zero padding modes, BatchNorm without
// affine parameters or running statistics, other pooling kinds) throw
// std::invalid_argument at build time rather than running elsewhere.
//
// Use: compile with Nott's `src/` directory on the include path, include
// this header after Nott's layer headers and before core.hpp (Model::add
// names the factory with a qualified call, which sees only the overloads
// declared before it), and opt the owner in:
//
//   namespace Nott { class Model; }
//   template <> struct Nott::HIP::enable_layers<Nott::Model> : std::true_type {};
#ifndef NOTT_HIP_REGISTRY_HPP
#define NOTT_HIP_REGISTRY_HPP

#include <algorithm>
#include <array>
#include <cctype>
#include <stdexcept>
#include <string>
#include <type_traits>
#include <variant>
#include <vector>

#include "activation/activation.hpp"
#include "initialization/apply.hpp"
#include "initialization/initialization.hpp"
#include "layer/details/batchnorm.hpp"
#include "layer/details/conv.hpp"
#include "layer/details/fc.hpp"
#include "layer/details/flatten.hpp"
#include "layer/details/pooling.hpp"
#include "layer/registry.hpp"

#include "nott_hip/host.hpp"

namespace Nott::HIP {

// Owners whose layers are built on the HIP modules.  Specialise to
// std::true_type for the owner type (Nott::Model, a block module, or one's
// own torch::nn::Module with register_module).
template <class Owner>
struct enable_layers : std::false_type {};

template <class Owner>
concept LayerOwner = enable_layers<std::remove_cv_t<Owner>>::value;

namespace factory {

inline bool is_relu(const ::Nott::Activation::Descriptor& a) { return a.type == ::Nott::Activation::Type::ReLU; }

inline void copy_values(Tensor& dst, const Tensor& src) {
    torch::NoGradGuard ng;
    dst.copy_(src);
}

// Forward functors for RegisteredLayer::bind_inline_forward (trivially
// copyable, one pointer): the layer with its ReLU fused.
struct ConvRelu {
    Conv2dImpl* m;
    Tensor operator()(Tensor x) const { return m->forward_relu(x); }
};
struct LinearRelu {
    LinearImpl* m;
    Tensor operator()(Tensor x) const { return m->forward_relu(x); }
};
struct BatchNormRelu {
    BatchNorm2dImpl* m;
    Tensor operator()(Tensor x) const { return m->forward_relu(x); }
};

}  // namespace factory
}  // namespace Nott::HIP

namespace Nott::Layer::Details {

template <class Owner>
    requires ::Nott::HIP::LayerOwner<Owner>
RegisteredLayer build_registered_layer(Owner& owner, const Conv2dDescriptor& descriptor, std::size_t index) {
    namespace F = ::Nott::HIP::factory;
    const auto& o = descriptor.options;
    if (o.in_channels <= 0 || o.out_channels <= 0)
        throw std::invalid_argument("Conv2d layers require positive channel counts.");
    if (o.groups != 1) throw std::invalid_argument("Nott::HIP::Conv2d: grouped convolution is not supported.");
    std::string mode = o.padding_mode;
    std::transform(mode.begin(), mode.end(), mode.begin(), [](unsigned char ch) { return (char)std::tolower(ch); });
    if (mode == "reflect" || mode == "replicate" || mode == "circular")
        throw std::invalid_argument("Nott::HIP::Conv2d: padding mode '" + o.padding_mode + "' is not supported.");
    if (!mode.empty() && mode != "zeros")
        throw std::invalid_argument("Unsupported padding mode provided to Conv2d descriptor: " + o.padding_mode);

    // The module the reference builds, from the same options in the same
    // order (torch checks the sizes as it does for the reference), for its
    // geometry and its constructor's default initialisation (and the
    // generator draws that makes).
    auto torch_options = torch::nn::Conv2dOptions(o.in_channels, o.out_channels, o.kernel_size);
    if (!o.stride.empty()) torch_options.stride(o.stride);
    if (!o.padding.empty()) torch_options.padding(o.padding);
    if (!o.dilation.empty()) torch_options.dilation(o.dilation);
    torch_options.bias(o.bias);
    torch::nn::Conv2d defaults(torch_options);
    const auto& to = defaults->options;
    if (!std::holds_alternative<torch::ExpandingArray<2>>(to.padding()))
        throw std::invalid_argument("Nott::HIP::Conv2d: only explicit padding is supported.");
    const auto& pad = std::get<torch::ExpandingArray<2>>(to.padding());

    ::Nott::HIP::Conv2dOptions hip_options;
    hip_options.in_channels = o.in_channels;
    hip_options.out_channels = o.out_channels;
    hip_options.kernel_size = {(*to.kernel_size())[0], (*to.kernel_size())[1]};
    hip_options.stride = {(*to.stride())[0], (*to.stride())[1]};
    hip_options.padding = {(*pad)[0], (*pad)[1]};
    hip_options.dilation = {(*to.dilation())[0], (*to.dilation())[1]};
    hip_options.bias = o.bias;
    auto module = owner.register_module("conv2d_" + std::to_string(index), ::Nott::HIP::Conv2d(hip_options));
    F::copy_values(module->weight, defaults->weight);
    if (o.bias) F::copy_values(module->bias, defaults->bias);
    ::Nott::Initialization::Details::apply_module_initialization(module, descriptor);

    RegisteredLayer registered_layer{};
    registered_layer.module = to_shared_module_ptr(module);
    registered_layer.local = descriptor.local;
    if (F::is_relu(descriptor.activation)) {
        registered_layer.activation = ::Nott::Activation::Type::Identity;
        registered_layer.bind_inline_forward(F::ConvRelu{module.get()});
    } else {
        registered_layer.activation = descriptor.activation.type;
        registered_layer.bind_module_forward(module.get());
    }
    return registered_layer;
}

template <class Owner>
    requires ::Nott::HIP::LayerOwner<Owner>
RegisteredLayer build_registered_layer(Owner& owner, const FCDescriptor& descriptor, std::size_t index) {
    namespace F = ::Nott::HIP::factory;
    const auto& o = descriptor.options;
    if (o.in_features <= 0 || o.out_features <= 0)
        throw std::invalid_argument("Fully connected layers require positive in/out features.");
    torch::nn::Linear defaults(torch::nn::LinearOptions(o.in_features, o.out_features).bias(o.bias));
    auto module = owner.register_module("fc_" + std::to_string(index),
                                        ::Nott::HIP::Linear(o.in_features, o.out_features, o.bias));
    F::copy_values(module->weight, defaults->weight);
    if (o.bias) F::copy_values(module->bias, defaults->bias);
    ::Nott::Initialization::Details::apply_module_initialization(module, descriptor);

    RegisteredLayer registered_layer{};
    registered_layer.module = to_shared_module_ptr(module);
    registered_layer.local = descriptor.local;
    if (F::is_relu(descriptor.activation)) {
        registered_layer.activation = ::Nott::Activation::Type::Identity;
        registered_layer.bind_inline_forward(F::LinearRelu{module.get()});
    } else {
        registered_layer.activation = descriptor.activation.type;
        registered_layer.bind_module_forward(module.get());
    }
    return registered_layer;
}

template <class Owner>
    requires ::Nott::HIP::LayerOwner<Owner>
RegisteredLayer build_registered_layer(Owner& owner, const BatchNorm2dDescriptor& descriptor, std::size_t index) {
    namespace F = ::Nott::HIP::factory;
    const auto& o = descriptor.options;
    if (o.num_features <= 0) throw std::invalid_argument("BatchNorm2d requires a positive number of features.");
    if (!o.affine || !o.track_running_stats)
        throw std::invalid_argument(
            "Nott::HIP::BatchNorm2d: only affine=true with running statistics is supported.");
    auto module = owner.register_module("batchnorm2d_" + std::to_string(index),
                                        ::Nott::HIP::BatchNorm2d(o.num_features, o.eps, o.momentum));
    ::Nott::Initialization::Details::apply_module_initialization(module, descriptor);

    RegisteredLayer registered_layer{};
    registered_layer.module = to_shared_module_ptr(module);
    registered_layer.local = descriptor.local;
    if (F::is_relu(descriptor.activation)) {
        registered_layer.activation = ::Nott::Activation::Type::Identity;
        registered_layer.bind_inline_forward(F::BatchNormRelu{module.get()});
    } else {
        registered_layer.activation = descriptor.activation.type;
        registered_layer.bind_module_forward(module.get());
    }
    return registered_layer;
}

template <class Owner>
    requires ::Nott::HIP::LayerOwner<Owner>
RegisteredLayer build_registered_layer(Owner& owner, const PoolingDescriptor& descriptor, std::size_t index) {
    namespace F = ::Nott::HIP::factory;
    RegisteredLayer registered_layer{};
    registered_layer.activation = descriptor.activation.type;
    registered_layer.local = descriptor.local;
    std::visit(
        [&](const auto& options) {
            using OptionType = std::decay_t<decltype(options)>;
            if constexpr (std::is_same_v<OptionType, MaxPool2dOptions>) {
                // The reference's torch options, built the same way (stride
                // defaults to the window).
                auto to = torch::nn::MaxPool2dOptions(options.kernel_size).ceil_mode(options.ceil_mode);
                if (!options.stride.empty()) to.stride(options.stride);
                if (!options.padding.empty()) to.padding(options.padding);
                if (!options.dilation.empty()) to.dilation(options.dilation);
                using A2 = std::array<int64_t, 2>;
                const auto pair = [](const torch::ExpandingArray<2>& a) { return A2{(*a)[0], (*a)[1]}; };
                auto module = owner.register_module(
                    "maxpool2d_" + std::to_string(index),
                    ::Nott::HIP::MaxPool2d(pair(to.kernel_size()), pair(to.stride()), pair(to.padding()),
                                           pair(to.dilation()), to.ceil_mode()));
                registered_layer.module = to_shared_module_ptr(module);
                registered_layer.bind_module_forward(module.get());
            } else if constexpr (std::is_same_v<OptionType, AdaptiveAvgPool2dOptions>) {
                const auto to = torch::nn::AdaptiveAvgPool2dOptions(options.output_size);
                const auto& out = *to.output_size();
                if (!out[0].has_value() || !out[1].has_value() || *out[0] != 1 || *out[1] != 1)
                    throw std::invalid_argument("Nott::HIP::AdaptiveAvgPool2d: only a 1x1 output is supported.");
                auto module = owner.register_module("adaptive_avgpool2d_" + std::to_string(index),
                                                    ::Nott::HIP::AdaptiveAvgPool2d());
                registered_layer.module = to_shared_module_ptr(module);
                registered_layer.bind_module_forward(module.get());
            } else {
                throw std::invalid_argument(
                    "Nott::HIP: only MaxPool2d and AdaptiveAvgPool2d (1x1) pooling layers are supported.");
            }
        },
        descriptor.options);
    return registered_layer;
}

template <class Owner>
    requires ::Nott::HIP::LayerOwner<Owner>
RegisteredLayer build_registered_layer(Owner& owner, const FlattenDescriptor& descriptor, std::size_t index) {
    auto module = owner.register_module(
        "flatten_" + std::to_string(index),
        ::Nott::HIP::Flatten(descriptor.options.start_dim, descriptor.options.end_dim));
    RegisteredLayer registered_layer{};
    registered_layer.activation = descriptor.activation.type;
    registered_layer.module = to_shared_module_ptr(module);
    registered_layer.local = descriptor.local;
    registered_layer.bind_module_forward(module.get());
    return registered_layer;
}

}  // namespace Nott::Layer::Details

#endif  // NOTT_HIP_REGISTRY_HPP
