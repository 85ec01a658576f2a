// Python binding of the C++ host layer (include/nott_hip/host.hpp): the
// training steps of BASELINE configs[0] (small CNN + Adam) and configs[4]
// (ResNet-18 + AdamW, fp32 or bf16 mixed precision), assembled the way a
// Nott user builds them — each layer followed by its activation
// (reference core.hpp:1926-1936), residual blocks summing branch and skip
// before the block's final activation (block/details/blocks/residual.hpp:
// 87-141) — and stepped as Model::run_training_step does (core.hpp:3735-3827):
// forward, mean cross-entropy, loss.backward(), optimizer step, zero_grad.
#include <torch/extension.h>

#include "nott_hip/host.hpp"

#include <ATen/hip/HIPGraph.h>
#include <c10/hip/HIPGuard.h>

namespace NH = Nott::HIP;
using torch::Tensor;

namespace {

// ------------------------------------------------------------- configs[0]
struct SmallCNNImpl : torch::nn::Module {
    NH::Conv2d conv0{nullptr}, conv1{nullptr};
    NH::MaxPool2d pool0{nullptr}, pool1{nullptr};
    NH::Flatten flat{nullptr};
    NH::Linear fc0{nullptr}, fc1{nullptr};
    SmallCNNImpl() {
        // every layer under its Nott registration key (<kind>_<index>)
        conv0 = register_module("conv2d_0", NH::Conv2d(NH::Conv2dOptions{1, 32, {3, 3}, {1, 1}, {1, 1}}));
        pool0 = register_module("maxpool2d_1", NH::MaxPool2d(2, 2));
        conv1 = register_module("conv2d_2", NH::Conv2d(NH::Conv2dOptions{32, 64, {3, 3}, {1, 1}, {1, 1}}));
        pool1 = register_module("maxpool2d_3", NH::MaxPool2d(2, 2));
        flat = register_module("flatten_4", NH::Flatten());
        fc0 = register_module("fc_5", NH::Linear(3136, 128));
        fc1 = register_module("fc_6", NH::Linear(128, 10));
    }
    Tensor forward(Tensor x) {
        x = pool0(conv0->forward_relu(x));   // Conv + ReLU (fused), MaxPool2
        x = pool1(conv1->forward_relu(x));
        x = flat(x);                     // Flatten (a view)
        x = NH::relu(fc0(x));
        return fc1(x);
    }
};
TORCH_MODULE(SmallCNN);

// ------------------------------------------------------------- configs[4]
struct BasicBlockImpl : torch::nn::Module {
    NH::Conv2d c1{nullptr}, c2{nullptr}, proj{nullptr};
    NH::BatchNorm2d b1{nullptr}, b2{nullptr};
    BasicBlockImpl(int64_t in, int64_t out, int64_t stride) {
        c1 = register_module("conv0", NH::Conv2d(NH::Conv2dOptions{in, out, {3, 3}, {stride, stride}, {1, 1}, {1, 1}, false}));
        b1 = register_module("bn0", NH::BatchNorm2d(out));
        c2 = register_module("conv1", NH::Conv2d(NH::Conv2dOptions{out, out, {3, 3}, {1, 1}, {1, 1}, {1, 1}, false}));
        b2 = register_module("bn1", NH::BatchNorm2d(out));
        // Projection shortcut: a single 1×1 stride-2 conv, no BN (residual.hpp:18-20, 99-104).
        if (stride != 1 || in != out)
            proj = register_module("proj", NH::Conv2d(NH::Conv2dOptions{in, out, {1, 1}, {stride, stride}, {0, 0}, {1, 1}, false}));
    }
    Tensor forward(const Tensor& x) {
        auto f = NH::ForkFn::apply(x);     // x feeds the branch and the skip
        if (!keep) {
            // BN + ReLU and BN + skip + ReLU fused (same values; the probe
            // below keeps every intermediate as its own tensor).
            Tensor h = b1->forward_relu(c1(f[0]));
            Tensor skip = proj ? proj(f[1]) : f[1];
            return b2->forward_add_relu(c2(h), skip);
        }
        Tensor c0 = c1(f[0]);
        Tensor h = NH::relu(b1(c0));
        Tensor c1o = c2(h);
        Tensor h2 = b2(c1o);
        Tensor skip = proj ? proj(f[1]) : f[1];
        Tensor sum = NH::AddFn::apply(h2, skip);
        if (keep) {
            for (auto* t : {&c0, &h, &c1o, &h2, &sum, &f[0], &f[1]}) t->retain_grad();
            kept = {{"c0", c0}, {"h", h}, {"c1", c1o}, {"h2", h2}, {"sum", sum}, {"f0", f[0]}, {"f1", f[1]}};
        }
        return NH::relu(sum);
    }
    bool keep = false;
    std::vector<std::pair<std::string, Tensor>> kept;
};
TORCH_MODULE(BasicBlock);

struct ResNet18Impl : torch::nn::Module {
    NH::Conv2d stem{nullptr};
    NH::BatchNorm2d stem_bn{nullptr};
    std::vector<BasicBlock> blocks;
    NH::Linear fc{nullptr};
    explicit ResNet18Impl(int64_t classes) {
        stem = register_module("stem", NH::Conv2d(NH::Conv2dOptions{3, 64, {7, 7}, {2, 2}, {3, 3}, {1, 1}, false}));
        stem_bn = register_module("stem_bn", NH::BatchNorm2d(64));
        const int64_t widths[4] = {64, 128, 256, 512};
        int64_t in = 64;
        for (int s = 0; s < 4; ++s)
            for (int b = 0; b < 2; ++b) {
                const int64_t stride = (s > 0 && b == 0) ? 2 : 1;
                blocks.push_back(register_module("block" + std::to_string(s) + "_" + std::to_string(b),
                                                 BasicBlock(in, widths[s], stride)));
                in = widths[s];
            }
        fc = register_module("fc", NH::Linear(512, classes));
    }
    Tensor forward(Tensor x) {
        x = NH::max_pool2d(keep_grads ? NH::relu(stem_bn(stem(x))) : stem_bn->forward_relu(stem(x)), 3, 2, 1);
        if (keep_grads) mark(x, "stem_out");
        for (size_t i = 0; i < blocks.size(); ++i) {
            x = blocks[i](x);
            if (keep_grads) mark(x, "block_out" + std::to_string(i));
        }
        x = NH::AvgPoolGlobalFn::apply(x).flatten(1);
        return fc(x);
    }
    // Intermediate activations whose gradients are kept (tests of the wiring).
    bool keep_grads = false;
    std::vector<std::pair<std::string, Tensor>> marked;
    void mark(Tensor& t, const std::string& name) {
        t.retain_grad();
        marked.emplace_back(name, t);
    }
};
TORCH_MODULE(ResNet18);

// Conv / Linear weights of a module tree (the tensors that get bf16 copies).
void collect_weights(torch::nn::Module& m, std::vector<Tensor*>& copies, std::vector<Tensor>& masters) {
    for (auto& child : m.modules(/*include_self=*/true)) {
        if (auto* c = child->as<NH::Conv2dImpl>()) {
            copies.push_back(&c->weight_compute);
            masters.push_back(c->weight);
        } else if (auto* l = child->as<NH::LinearImpl>()) {
            copies.push_back(&l->weight_compute);
            masters.push_back(l->weight);
        }
    }
}

// A model + fused optimizer on one device; the Python side drives it.
template <class Model>
struct Trainer {
    Model model;
    std::unique_ptr<NH::FusedAdam> opt;
    bool bf16;
    Trainer(Model m, bool bf16_, NH::FusedAdam::Options o, int device, uint64_t seed) : model(std::move(m)), bf16(bf16_) {
        torch::NoGradGuard ng;
        auto gen = at::detail::createCPUGenerator(seed);
        torch::Generator g(gen);
        for (auto& kv : model->named_parameters()) {
            Tensor p = kv.value();
            const auto& name = kv.key();
            if (name.size() >= 6 && name.compare(name.size() - 6, 6, "weight") == 0 && p.dim() >= 2) NH::he_uniform_(p, g);
        }
        if (device >= 0) model->to(torch::Device(torch::kCUDA, device));   // device < 0: host only (tests of the wiring)
        model->train();
        std::vector<Tensor*> copies;
        std::vector<Tensor> masters;
        if (bf16) collect_weights(*model, copies, masters);
        std::vector<Tensor> params;
        for (auto& p : model->parameters()) params.push_back(p);
        opt = std::make_unique<NH::FusedAdam>(params, o, copies, masters);
    }
    Tensor input(const Tensor& x) { return bf16 ? x.to(torch::kBFloat16) : x; }
    // forward + loss + backward (grads land in the flat gradient arena)
    Tensor forward_backward(const Tensor& x, const Tensor& y) {
        Tensor logits = model->forward(input(x));
        Tensor loss = NH::cross_entropy(logits, y);
        loss.backward();
        return loss.detach();
    }
    Tensor step(const Tensor& x, const Tensor& y) {
        Tensor loss = forward_backward(x, y);
        opt->step();   // fused AdamW + zero_grad (+ bf16 copies)
        return loss;
    }

    // Step orchestration on device (the reference's CUDA-graph step path,
    // src/core.hpp:3829-3945): forward + loss + backward are captured once
    // into a HIP graph over static input buffers, so a step is two input
    // copies, one graph launch and the fused AdamW launch.  The optimizer
    // step stays outside the graph because its step count and bias
    // corrections change every step.  `warmup` forward/backward passes run
    // first on the capture stream (workspace, library plans and allocator
    // pools reach their steady state; their gradients are zeroed again).
    std::unique_ptr<at::cuda::CUDAGraph> graph;
    Tensor gx, gy, gloss;
    void warmup(const Tensor& x, const Tensor& y, int passes) {
        for (int i = 0; i < passes; ++i) forward_backward(x, y);
        opt->zero_grad();
    }
    void capture(const Tensor& x, const Tensor& y, int passes) {
        gx = x.clone();
        gy = y.clone();
        if (hipDeviceSynchronize() != hipSuccess) throw std::runtime_error("capture: device synchronize failed");
        auto s = c10::hip::getStreamFromPool();
        {
            c10::hip::HIPStreamGuard guard(s);
            warmup(gx, gy, passes);
            if (hipStreamSynchronize(s.stream()) != hipSuccess) throw std::runtime_error("capture: stream sync failed");
            auto g = std::make_unique<at::cuda::CUDAGraph>();
            g->capture_begin();
            gloss = forward_backward(gx, gy);
            g->capture_end();
            graph = std::move(g);
        }
        if (hipDeviceSynchronize() != hipSuccess) throw std::runtime_error("capture: device synchronize failed");
    }
    // parameters.binary in Nott's archive layout (src/core.hpp:2131-2135).
    void save(const std::string& path) { NH::save_parameters(*model, path); }
    Tensor step_graph(const Tensor& x, const Tensor& y) {
        if (!graph) throw std::logic_error("step_graph: call capture() first");
        gx.copy_(x);
        gy.copy_(y);
        graph->replay();
        opt->step();
        return gloss.clone();
    }
    Tensor forward(const Tensor& x) {
        torch::NoGradGuard ng;
        return model->forward(input(x));
    }
    std::map<std::string, Tensor> params() {
        std::map<std::string, Tensor> out;
        for (auto& kv : model->named_parameters()) out[kv.key()] = kv.value().detach();
        return out;
    }
    std::map<std::string, Tensor> grads() {
        std::map<std::string, Tensor> out;
        for (auto& kv : model->named_parameters()) out[kv.key()] = kv.value().grad();
        return out;
    }
    std::map<std::string, Tensor> buffers() {
        std::map<std::string, Tensor> out;
        for (auto& kv : model->named_buffers()) out[kv.key()] = kv.value();
        return out;
    }
    // Copies values into named parameters (then refreshes bf16 copies).
    void load(const std::map<std::string, Tensor>& values) {
        torch::NoGradGuard ng;
        auto named = model->named_parameters();
        for (auto& kv : values) {
            auto* p = named.find(kv.first);
            if (!p) throw std::invalid_argument("no parameter " + kv.first);
            p->copy_(kv.second);
        }
        opt->refresh();
    }
    int64_t num_params() {
        int64_t n = 0;
        for (auto& p : model->parameters()) n += p.numel();
        return n;
    }
};

}  // namespace

PYBIND11_MODULE(_nott_host, m) {
    m.doc() = "C++ host layer (Nott::HIP) over libnott_hip: configs[0] and configs[4] training steps";
    using SmallT = Trainer<SmallCNN>;
    py::class_<SmallT>(m, "SmallCNNTrainer")
        .def(py::init([](int device, uint64_t seed, double lr) {
                 NH::FusedAdam::Options o;
                 o.lr = lr;   // Adam, betas (0.9, 0.999), eps 1e-8, no weight decay
                 return new SmallT(SmallCNN(), false, o, device, seed);
             }),
             py::arg("device") = 0, py::arg("seed") = 0, py::arg("lr") = 1e-3)
        .def("step", &SmallT::step, py::call_guard<py::gil_scoped_release>())
        .def("warmup", &SmallT::warmup, py::arg("x"), py::arg("y"), py::arg("passes") = 2,
             py::call_guard<py::gil_scoped_release>())
        .def("capture", &SmallT::capture, py::arg("x"), py::arg("y"), py::arg("passes") = 2,
             py::call_guard<py::gil_scoped_release>())
        .def("step_graph", &SmallT::step_graph, py::call_guard<py::gil_scoped_release>())
        .def("save", &SmallT::save, py::arg("path"))
        .def("forward_backward", &SmallT::forward_backward, py::call_guard<py::gil_scoped_release>())
        .def("optimizer_step", [](SmallT& t) { t.opt->step(); }, py::call_guard<py::gil_scoped_release>())
        .def("forward", &SmallT::forward, py::call_guard<py::gil_scoped_release>())
        .def("params", &SmallT::params)
        .def("grads", &SmallT::grads)
        .def("load", &SmallT::load)
        .def("num_params", &SmallT::num_params);
    using ResT = Trainer<ResNet18>;
    py::class_<ResT>(m, "ResNet18Trainer")
        .def(py::init([](int device, uint64_t seed, bool bf16, double lr, double wd, int64_t classes) {
                 NH::FusedAdam::Options o;
                 o.lr = lr;
                 o.weight_decay = wd;
                 o.decoupled = true;   // AdamW
                 return new ResT(ResNet18(classes), bf16, o, device, seed);
             }),
             py::arg("device") = 0, py::arg("seed") = 0, py::arg("bf16") = false, py::arg("lr") = 1e-3,
             py::arg("weight_decay") = 1e-2, py::arg("classes") = 1000)
        .def("step", &ResT::step, py::call_guard<py::gil_scoped_release>())
        .def("warmup", &ResT::warmup, py::arg("x"), py::arg("y"), py::arg("passes") = 2,
             py::call_guard<py::gil_scoped_release>())
        .def("capture", &ResT::capture, py::arg("x"), py::arg("y"), py::arg("passes") = 2,
             py::call_guard<py::gil_scoped_release>())
        .def("step_graph", &ResT::step_graph, py::call_guard<py::gil_scoped_release>())
        .def("save", &ResT::save, py::arg("path"))
        .def("forward_backward", &ResT::forward_backward, py::call_guard<py::gil_scoped_release>())
        .def("optimizer_step", [](ResT& t) { t.opt->step(); }, py::call_guard<py::gil_scoped_release>())
        .def("forward", &ResT::forward, py::call_guard<py::gil_scoped_release>())
        .def("params", &ResT::params)
        .def("grads", &ResT::grads)
        .def("buffers", &ResT::buffers)
        .def("activation_grads",
             [](ResT& t, const Tensor& x, const Tensor& y) {
                 t.model->keep_grads = true;
                 t.model->marked.clear();
                 t.model->blocks[0]->keep = true;
                 {
                     py::gil_scoped_release nogil;
                     t.forward_backward(x, y);
                 }
                 std::map<std::string, Tensor> out;
                 for (auto& kv : t.model->marked) out[kv.first] = kv.second.grad();
                 for (auto& kv : t.model->blocks[0]->kept) out["b0_" + kv.first] = kv.second.grad();
                 t.model->blocks[0]->keep = false;
                 t.model->blocks[0]->kept.clear();
                 t.model->keep_grads = false;
                 t.model->marked.clear();
                 return out;
             })
        .def("load", &ResT::load)
        .def("num_params", &ResT::num_params);
}
