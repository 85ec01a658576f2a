// Test module: Nott's own layer descriptors and factory, built on the HIP
// modules through include/nott_hip/registry.hpp.
//
// Compiled (tests/factory/Makefile) against the reference's headers under
// /root/reference/src: the descriptors and their option structs
// (src/layer/details/*.hpp), the dispatching build_registered_layer over a
// std::variant of descriptors (src/layer/registry.hpp:193-200),
// RegisteredLayer, the initialisation (src/initialization/apply.hpp) and the
// activation dispatch (src/activation/apply.hpp) are the reference's,
// unchanged.  The umbrella src/layer/layer.hpp (the Nott::Layer::Conv2d, FC,
// ... factory functions and the full Descriptor variant) is not included: it
// pulls in layer/details/recurrent.hpp, which includes the CUDA-only
// <ATen/cuda/CUDAContext.h>.  The descriptors are therefore written as
// aggregates, which is all those functions do (layer.hpp:107-233), and the
// variant lists the descriptor kinds used here.  The owner below
// does what Model::add and Model::forward do with them (core.hpp:516-523,
// 1926-1936); the optimizer is Nott::HIP::FusedAdam held as Nott holds one
// (std::unique_ptr<torch::optim::Optimizer>, core.hpp:170-181) and stepped as
// run_training_step steps it (step, then zero_grad(false); core.hpp:
// 3819-3823).
#include <torch/extension.h>

#include "activation/apply.hpp"
#include "layer/details/dropout.hpp"
#include "nott_hip/registry.hpp"

#include <memory>
#include <string>
#include <vector>

namespace NH = Nott::HIP;
namespace NL = Nott::Layer::Details;
using torch::Tensor;
using Nott::Activation::Identity;
using Nott::Activation::ReLU;
using Nott::Initialization::HeUniform;

namespace {
struct FactoryModelImpl;
}
template <>
struct Nott::HIP::enable_layers<FactoryModelImpl> : std::true_type {};

namespace {

// The layer kinds of Nott::Layer::Descriptor (layer.hpp:88-104) used here.
using Descriptor = std::variant<NL::FCDescriptor, NL::Conv2dDescriptor, NL::BatchNorm2dDescriptor,
                                NL::PoolingDescriptor, NL::HardDropoutDescriptor, NL::FlattenDescriptor>;

struct FactoryModelImpl : torch::nn::Module {
    std::vector<NL::RegisteredLayer> layers;
    // Model::add for a layer descriptor: the reference's variant dispatch,
    // the next module index, the layer kept in order.
    void add(const Descriptor& d) { layers.push_back(NL::build_registered_layer(*this, d, layers.size())); }
    // Model::forward without compiled routing: each layer, then its activation.
    Tensor forward(Tensor x) {
        for (auto& l : layers) x = Nott::Activation::Details::apply(l.activation, l.forward(std::move(x)));
        return x;
    }
};

// What a registered module is: the HIP module class, or the torch one.
std::string kind_of(const torch::nn::Module& m) {
    if (m.as<NH::Conv2dImpl>()) return "hip.Conv2d";
    if (m.as<NH::LinearImpl>()) return "hip.Linear";
    if (m.as<NH::BatchNorm2dImpl>()) return "hip.BatchNorm2d";
    if (m.as<NH::MaxPool2dImpl>()) return "hip.MaxPool2d";
    if (m.as<NH::AdaptiveAvgPool2dImpl>()) return "hip.AdaptiveAvgPool2d";
    if (m.as<NH::FlattenImpl>()) return "hip.Flatten";
    return "other:" + m.name();
}

// configs[0] as a Nott user writes it: 1×28×28 → Conv(32, 3×3, pad 1) ReLU →
// MaxPool 2 → Conv(64) ReLU → MaxPool 2 → Flatten → FC 3136→128 ReLU →
// FC 128→10, HeUniform weights.
std::vector<Descriptor> small_cnn() {
    NL::PoolingDescriptor pool;
    pool.options = NL::MaxPool2dOptions{{2, 2}, {2, 2}};
    return {
        NL::Conv2dDescriptor{{1, 32, {3, 3}, {1, 1}, {1, 1}, {1, 1}, 1, true, "zeros"}, ReLU, HeUniform},
        pool,
        NL::Conv2dDescriptor{{32, 64, {3, 3}, {1, 1}, {1, 1}, {1, 1}, 1, true, "zeros"}, ReLU, HeUniform},
        pool,
        NL::FlattenDescriptor{},
        NL::FCDescriptor{{3136, 128, true}, ReLU, HeUniform},
        NL::FCDescriptor{{128, 10, true}, Identity, HeUniform},
    };
}

struct Session {
    std::shared_ptr<FactoryModelImpl> model = std::make_shared<FactoryModelImpl>();
    std::unique_ptr<torch::optim::Optimizer> opt;

    explicit Session(uint64_t seed) {
        torch::manual_seed(seed);
        for (const auto& d : small_cnn()) model->add(d);
    }
    std::vector<std::pair<std::string, std::string>> modules() const {
        std::vector<std::pair<std::string, std::string>> out;
        for (const auto& c : model->named_children()) out.emplace_back(c.key(), kind_of(*c.value()));
        return out;
    }
    std::vector<std::string> activations() const {
        std::vector<std::string> out;
        for (const auto& l : model->layers)
            out.push_back(l.activation == Nott::Activation::Type::Identity ? "identity" : "other");
        return out;
    }
    std::map<std::string, Tensor> params() const {
        std::map<std::string, Tensor> out;
        for (const auto& p : model->named_parameters()) out[p.key()] = p.value().detach();
        return out;
    }
    std::map<std::string, Tensor> grads() const {
        std::map<std::string, Tensor> out;
        for (const auto& p : model->named_parameters()) out[p.key()] = p.value().grad();
        return out;
    }
    void to_device(int device, double lr) {
        model->to(torch::Device(torch::kCUDA, device));
        model->train();
        std::vector<Tensor> ps;
        for (auto& p : model->parameters()) ps.push_back(p);
        opt = std::make_unique<NH::FusedAdam>(ps, torch::optim::AdamOptions(lr));
    }
    Tensor forward_backward(const Tensor& x, const Tensor& y) {
        Tensor logits = model->forward(x);
        Tensor loss = NH::cross_entropy(logits, y);
        loss.backward();
        return loss.detach();
    }
    void optimizer_step() {
        opt->step();
        opt->zero_grad(false);
    }
};

// One layer built through the factory in a fresh owner, for the option
// checks (exceptions propagate: std::invalid_argument is ValueError in
// Python, c10::Error RuntimeError).
NL::PoolingDescriptor pooling(NL::PoolingOptions o) {
    NL::PoolingDescriptor d;
    d.options = std::move(o);
    return d;
}

std::string build_one(const std::string& which) {
    auto owner = std::make_shared<FactoryModelImpl>();
    NL::Conv2dOptions conv{4, 8, {3, 3}, {1, 1}, {1, 1}, {1, 1}, 1, true, "zeros"};
    auto add_conv = [&] { owner->add(NL::Conv2dDescriptor{conv}); };
    if (which == "conv") {
        add_conv();
    } else if (which == "conv_groups") {
        conv.groups = 2;
        add_conv();
    } else if (which == "conv_reflect") {
        conv.padding_mode = "reflect";
        add_conv();
    } else if (which == "conv_bad_mode") {
        conv.padding_mode = "mirror";
        add_conv();
    } else if (which == "conv_zero_channels") {
        conv.out_channels = 0;
        add_conv();
    } else if (which == "conv_strided_rect") {
        conv.kernel_size = {1, 3};
        conv.stride = {2, 1};
        conv.padding = {0, 1};
        conv.bias = false;
        add_conv();
    } else if (which == "conv_three_kernel_values") {
        conv.kernel_size = {3, 3, 3};
        add_conv();
    } else if (which == "fc_zero") {
        owner->add(NL::FCDescriptor{{0, 4, true}});
    } else if (which == "bn") {
        owner->add(NL::BatchNorm2dDescriptor{{8, 1e-5, 0.1, true, true}, ReLU});
    } else if (which == "bn_no_affine") {
        owner->add(NL::BatchNorm2dDescriptor{{8, 1e-5, 0.1, false, true}});
    } else if (which == "bn_no_stats") {
        owner->add(NL::BatchNorm2dDescriptor{{8, 1e-5, 0.1, true, false}});
    } else if (which == "maxpool_3s2p1") {
        owner->add(pooling(NL::MaxPool2dOptions{{3, 3}, {2, 2}, {1, 1}}));
    } else if (which == "maxpool_default_stride") {
        owner->add(pooling(NL::MaxPool2dOptions{{3, 3}, {}, {1, 1}, {1, 1}, true}));
    } else if (which == "avgpool2d") {
        owner->add(pooling(NL::AvgPool2dOptions{{2, 2}, {2, 2}}));
    } else if (which == "adaptive_avg_1x1") {
        owner->add(pooling(NL::AdaptiveAvgPool2dOptions{{1, 1}}));
    } else if (which == "adaptive_avg_2x2") {
        owner->add(pooling(NL::AdaptiveAvgPool2dOptions{{2, 2}}));
    } else if (which == "adaptive_max") {
        owner->add(pooling(NL::AdaptiveMaxPool2dOptions{{1, 1}}));
    } else if (which == "flatten") {
        owner->add(NL::FlattenDescriptor{});
    } else if (which == "dropout") {
        // Not on the HIP path: the reference's own factory builds it.
        owner->add(NL::HardDropoutDescriptor{{0.5}});
    } else {
        throw std::invalid_argument("unknown case " + which);
    }
    // "<key> <kind>[ <geometry>]": the registration key, the module class and,
    // for the HIP convolution and max-pool, the geometry the module holds.
    const auto children = owner->named_children();
    if (children.is_empty()) return std::string();
    const auto& m = *children[0].value();
    std::string out = children[0].key() + " " + kind_of(m);
    const std::vector<int64_t>* g = nullptr;
    if (auto* c = m.as<NH::Conv2dImpl>()) g = &c->geometry();
    if (auto* p = m.as<NH::MaxPool2dImpl>()) g = &p->geometry();
    if (g)
        for (int64_t v : *g) out += " " + std::to_string(v);
    return out;
}
}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    namespace py = pybind11;
    py::class_<Session>(m, "SmallCnnFactory")
        .def(py::init<uint64_t>(), py::arg("seed"))
        .def("modules", &Session::modules)
        .def("activations", &Session::activations)
        .def("params", &Session::params)
        .def("grads", &Session::grads)
        .def("to_device", &Session::to_device, py::arg("device"), py::arg("lr"))
        .def("forward_backward", &Session::forward_backward, py::call_guard<py::gil_scoped_release>())
        .def("optimizer_step", &Session::optimizer_step, py::call_guard<py::gil_scoped_release>());
    m.def("build_one", &build_one);
}
