// Python binding of the C++ host layer (include/nott_hip/host.hpp): the
// training steps of BASELINE configs[0] (small CNN + Adam) and configs[4]
// (ResNet-18 + AdamW, fp32 or bf16 mixed precision), assembled the way a
// Nott user builds them — each layer followed by its activation
// (reference core.hpp:1926-1936), residual blocks summing branch and skip
// before the block's final activation (block/details/blocks/residual.hpp:
// 87-141) — and stepped as Model::run_training_step does (core.hpp:3735-3827):
// forward, mean cross-entropy, loss.backward(), optimizer step, zero_grad.
#include <torch/extension.h>

#include "nott_hip/architecture.hpp"
#include "nott_hip/host.hpp"

#include <filesystem>

#include <ATen/hip/HIPGraph.h>
#include <c10/hip/HIPGuard.h>

namespace NH = Nott::HIP;
namespace NA = Nott::HIP::arch;
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
    // The descriptor list a Nott model of this architecture records, in
    // add() order (core.hpp:490-817): the layer factories' descriptors with
    // ReLU on both convolutions and the first FC, Kaiming-uniform weights.
    static std::vector<NA::Node> descriptors() {
        return {NA::module("layer", NA::conv2d(1, 32, 3, 1, 1, true, "relu", "he_uniform")),
                NA::module("layer", NA::max_pool2d(2, 2, 0)),
                NA::module("layer", NA::conv2d(32, 64, 3, 1, 1, true, "relu", "he_uniform")),
                NA::module("layer", NA::max_pool2d(2, 2, 0)),
                NA::module("layer", NA::flatten()),
                NA::module("layer", NA::fc(3136, 128, true, "relu", "he_uniform")),
                NA::module("layer", NA::fc(128, 10, true, "identity", "he_uniform"))};
    }
    Tensor forward(Tensor x) {
        // Conv + ReLU (fused), MaxPool2; the ReLU's backward runs in the
        // pool's backward pass
        x = pool0->forward_relu_input(conv0->forward_relu(x, true));
        x = pool1->forward_relu_input(conv1->forward_relu(x, true));
        x = flat(x);                     // Flatten (a view)
        // FC + ReLU in the GEMM's epilogue; the ReLU's backward runs in
        // fc1's dx epilogue
        x = fc0->forward_relu(x, true);
        return fc1->forward_relu_input(x);
    }
};
TORCH_MODULE(SmallCNN);

// ------------------------------------------------------------- configs[4]
// ResNet-18 as a Nott model registers it (core.hpp:516-523, 576-592): the
// stem Conv2d (identity activation), BatchNorm2d with ReLU and MaxPool2d,
// eight Residual blocks (residual_block_<i>, each down-sampling block its
// own descriptor with a 1×1 stride-2 projection; residual.hpp:18-20, 99-104),
// AdaptiveAvgPool2d, Flatten and the FC layer, each under its
// `<kind>_<index>` key, so parameter names match the reference's
// (e.g. residual_block_3.conv2d_0.weight, fc_13.bias).
struct ResNet18Impl : torch::nn::Module {
    NH::Conv2d stem{nullptr};
    NH::BatchNorm2d stem_bn{nullptr};
    NH::MaxPool2d pool{nullptr};
    std::vector<NH::ResidualBasicBlock> blocks;
    NH::AdaptiveAvgPool2d gap{nullptr};
    NH::Flatten flat{nullptr};
    NH::Linear fc{nullptr};
    int64_t classes;
    explicit ResNet18Impl(int64_t classes_) : classes(classes_) {
        int64_t index = 0;
        auto key = [&](const char* kind) { return std::string(kind) + "_" + std::to_string(index++); };
        stem = register_module(key("conv2d"), NH::Conv2d(NH::Conv2dOptions{3, 64, {7, 7}, {2, 2}, {3, 3}, {1, 1}, false}));
        stem_bn = register_module(key("batchnorm2d"), NH::BatchNorm2d(64));
        pool = register_module(key("maxpool2d"), NH::MaxPool2d(3, 2, 1));
        const int64_t widths[4] = {64, 128, 256, 512};
        int64_t in = 64;
        for (int s = 0; s < 4; ++s)
            for (int b = 0; b < 2; ++b) {
                const int64_t stride = (s > 0 && b == 0) ? 2 : 1;
                const bool projection = stride != 1 || in != widths[s];
                blocks.push_back(register_module(key("residual_block"),
                                                 NH::ResidualBasicBlock(in, widths[s], stride, projection)));
                in = widths[s];
            }
        gap = register_module(key("adaptive_avgpool2d"), NH::AdaptiveAvgPool2d());
        flat = register_module(key("flatten"), NH::Flatten());
        fc = register_module(key("fc"), NH::Linear(512, classes));
    }
    // The descriptor list a Nott model of this architecture records: stem
    // conv (identity), BatchNorm2d + ReLU, MaxPool2d 3/2/1, eight residual
    // block descriptors ({conv 3×3, BN + ReLU, conv 3×3, BN}, final ReLU, a
    // 1×1 projection conv on the down-sampling ones), AdaptiveAvgPool2d,
    // Flatten, FC; Kaiming-uniform conv and FC weights.
    std::vector<NA::Node> descriptors() const { return descriptors_for(classes); }
    static std::vector<NA::Node> descriptors_for(int64_t classes) {
        std::vector<NA::Node> mods;
        mods.push_back(NA::module("layer", NA::conv2d(3, 64, 7, 2, 3, false, "identity", "he_uniform")));
        mods.push_back(NA::module("layer", NA::batch_norm2d(64, "relu")));
        mods.push_back(NA::module("layer", NA::max_pool2d(3, 2, 1)));
        const int64_t widths[4] = {64, 128, 256, 512};
        int64_t in = 64;
        for (int s = 0; s < 4; ++s)
            for (int b = 0; b < 2; ++b) {
                const int64_t out = widths[s], stride = (s > 0 && b == 0) ? 2 : 1;
                std::vector<NA::Node> layers;
                layers.push_back(NA::conv2d(in, out, 3, stride, 1, false, "identity", "he_uniform"));
                layers.push_back(NA::batch_norm2d(out, "relu"));
                layers.push_back(NA::conv2d(out, out, 3, 1, 1, false, "identity", "he_uniform"));
                layers.push_back(NA::batch_norm2d(out, "identity"));
                const NA::Node proj = NA::conv2d(in, out, 1, stride, 0, false, "identity", "he_uniform");
                const bool projection = stride != 1 || in != out;
                mods.push_back(NA::module("block", NA::residual(std::move(layers), projection ? &proj : nullptr, "relu")));
                in = out;
            }
        mods.push_back(NA::module("layer", NA::adaptive_avg_pool2d(1, 1)));
        mods.push_back(NA::module("layer", NA::flatten()));
        mods.push_back(NA::module("layer", NA::fc(512, classes, true, "identity", "he_uniform")));
        return mods;
    }
    Tensor forward(Tensor x) {
        // BatchNorm + ReLU + max-pool with the BatchNorm's output never stored
        x = stem_bn->forward_relu_maxpool(stem(x), pool->geometry());
        if (record) outputs.push_back(x);
        // consecutive blocks: the final ReLU's backward of block i runs in
        // block i + 1's fork, together with the fork's sum
        for (size_t i = 0; i < blocks.size(); ++i) {
            x = blocks[i]->forward(x, i > 0, i + 1 < blocks.size());
            if (record) outputs.push_back(x);
        }
        x = fc(flat(gap(x)));
        if (record) outputs.push_back(x);
        return x;
    }
    // When set, forward keeps the stem output, every block output (the
    // post-ReLU activations; tests compare their zero patterns) and the logits.
    bool record = false;
    std::vector<Tensor> outputs;
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

// A model and its optimizer on one device; the Python side drives it.  The
// optimizer is held as Nott's OptimizerBinding holds it, a
// std::unique_ptr<torch::optim::Optimizer> (core.hpp:170-181), and stepped
// through the virtual step() (core.hpp:5049-5057).
template <class Model, bool Decoupled>
struct Trainer {
    using Fused = NH::FusedAdamImpl<Decoupled>;
    Model model;
    std::unique_ptr<torch::optim::Optimizer> opt;
    Fused* fused = nullptr;   // the same object, for the flat-arena extras
    bool bf16;
    Trainer(Model m, bool bf16_, const typename Fused::TorchOptions& o, int device, uint64_t seed)
        : model(std::move(m)), bf16(bf16_) {
        torch::NoGradGuard ng;
        auto gen = at::detail::createCPUGenerator(seed);
        torch::Generator g(gen);
        // The weights a Nott model built from the same descriptors draws
        // after torch::manual_seed(seed).
        NH::reference_init_(*model, g);
        model->to(torch::Device(torch::kCUDA, device));
        model->train();
        std::vector<Tensor> params;
        for (auto& p : model->parameters()) params.push_back(p);
        auto f = std::make_unique<Fused>(params, o);
        // Model::run_training_step always follows step() with zero_grad()
        // (core.hpp:3819-3823): clear the gradients in the update pass.
        f->set_fused_zero_grad(true);
        if (bf16) {
            std::vector<Tensor*> copies;
            std::vector<Tensor> masters;
            collect_weights(*model, copies, masters);
            f->attach_bf16_copies(copies, masters);
        }
        fused = f.get();
        opt = std::move(f);
    }
    // The model's input in the compute dtype (bf16: one nott_cast).
    Tensor input(const Tensor& x) {
        if (!bf16) return x;
        Tensor xc = x.contiguous();
        Tensor out = torch::empty(xc.sizes(), xc.options().dtype(torch::kBFloat16));
        nott_ctx c = NH::bind(xc);
        NH::check(nott_cast(c, xc.numel(), xc.data_ptr(), NOTT_F32, out.data_ptr(), NOTT_BF16), c, "input cast");
        return out;
    }
    // forward + loss + backward (grads land in the flat gradient arena)
    // Convolution weight gradients overlap the data-gradient chain on a
    // side stream, joined before anything reads the gradients.
    Tensor forward_backward(const Tensor& x, const Tensor& y) {
        const int dev = x.device().index();
        NH::SideStreamScope side(dev);
        Tensor logits = model->forward(input(x));
        Tensor loss = NH::cross_entropy(logits, y);
        loss.backward();
        NH::join_side_stream(dev);
        return loss.detach();
    }
    // One training step: forward, loss, backward, optimizer step with the
    // gradients cleared in the same pass.
    Tensor step(const Tensor& x, const Tensor& y) {
        Tensor loss = forward_backward(x, y);
        opt->step();
        return loss;
    }
    // Nott's sequence through the base-class interface only:
    // step_optimizers() then zero_grad(false) (core.hpp:3820-3823).
    void optimizer_step() {
        opt->step();
        opt->zero_grad(false);
    }

    // Step orchestration on device (the reference's CUDA-graph step path,
    // src/core.hpp:3829-3945): forward, loss, backward, the fused optimizer
    // step (its step count and bias corrections in device memory, its
    // hyper-parameters read at launch time) and the device-side loss
    // accumulation (core.hpp:4481-4487) are captured once into a HIP graph
    // over static input buffers, so a step is two input copies and one
    // graph launch.  `passes` forward/backward passes run first on the
    // capture stream so the workspace and the allocator pools reach their
    // steady state; their gradients are cleared again and the model's buffers
    // (BatchNorm running statistics) restored, so the warm-up leaves no trace
    // in the model.
    std::unique_ptr<at::cuda::CUDAGraph> graph;
    Tensor gx, gy, gloss;
    Tensor loss_acc;     // float64 device scalar: Σ loss·batch since the last reset
    int64_t batch_rows = 0;
    void warmup(const Tensor& x, const Tensor& y, int passes) {
        std::vector<Tensor> saved;
        for (auto& b : model->buffers()) saved.push_back(b.clone());
        for (int i = 0; i < passes; ++i) forward_backward(x, y);
        fused->zero_flat_grads();
        torch::NoGradGuard ng;
        auto bufs = model->buffers();
        for (size_t i = 0; i < bufs.size(); ++i) bufs[i].copy_(saved[i]);
        for (auto& child : model->modules(/*include_self=*/true))
            if (auto* bn = child->template as<NH::BatchNorm2dImpl>()) bn->uncount(passes);
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
            fused->graph_prepare();
            loss_acc = torch::zeros({1}, gx.options().dtype(torch::kFloat64));
            batch_rows = gx.size(0);
            auto g = std::make_unique<at::cuda::CUDAGraph>();
            g->capture_begin();
            gloss = forward_backward(gx, gy);
            fused->graph_step();
            {
                nott_ctx c = NH::bind(gloss);
                NH::check(nott_loss_accumulate(c, gloss.data_ptr<float>(), (double)batch_rows,
                                               loss_acc.data_ptr<double>()),
                          c, "loss accumulation");
            }
            g->capture_end();
            graph = std::move(g);
            // The captured forward was recorded, not run.
            for (auto& child : model->modules(/*include_self=*/true))
                if (auto* bn = child->template as<NH::BatchNorm2dImpl>()) bn->uncount(1);
        }
        if (hipDeviceSynchronize() != hipSuccess) throw std::runtime_error("capture: device synchronize failed");
    }
    // parameters.binary in Nott's archive layout (src/core.hpp:2131-2135).
    void save(const std::string& path) { NH::save_parameters(*model, path); }
    // Loads a parameters.binary written by Model::save (core.hpp:2188-2236
    // reads the same archive): every parameter and buffer by its
    // registration key, with the reference's checks (a missing key or a
    // shape mismatch throws), copied into this model's tensors (which are
    // views into the optimizer's flat arena) and the bf16 copies refreshed.
    // torch::nn::Module::save nests one archive per child module, so a key
    // a.b.weight is read through the archives a and b.
    static bool read_nested(torch::serialize::InputArchive& ar, const std::string& key, Tensor& t) {
        const auto dot = key.find('.');
        if (dot == std::string::npos) return ar.try_read(key, t);
        torch::serialize::InputArchive sub;
        if (!ar.try_read(key.substr(0, dot), sub)) return false;
        return read_nested(sub, key.substr(dot + 1), t);
    }
    void load_archive(const std::string& path) {
        torch::serialize::InputArchive ar;
        ar.load_from(path);
        std::map<std::string, Tensor> vals;
        auto take = [&](const std::string& key, const Tensor& dst) {
            Tensor t;
            if (!read_nested(ar, key, t)) throw std::runtime_error("checkpoint is missing '" + key + "'");
            if (t.sizes() != dst.sizes()) throw std::runtime_error("checkpoint tensor '" + key + "' has another shape");
            vals[key] = t.to(dst.device(), dst.scalar_type());
        };
        for (auto& kv : model->named_parameters()) take(kv.key(), kv.value());
        for (auto& kv : model->named_buffers()) take(kv.key(), kv.value());
        load(vals);
        for (auto& child : model->modules(/*include_self=*/true))
            if (auto* bn = child->template as<NH::BatchNorm2dImpl>()) bn->reload_counter();
    }
    // Model::model_name (core.hpp:2078-2086): the set name, else the
    // module's own ("Nott::Model" for a model constructed without one).
    std::string model_name_;
    void set_model_name(const std::string& n) { model_name_ = n; }
    std::string model_name() const { return model_name_.empty() ? std::string("Nott::Model") : model_name_; }
    NA::Node architecture() const { return NA::architecture(model_name(), model->descriptors()); }
    std::string architecture_json() const { return NA::to_json(architecture()); }
    // Model::save (core.hpp:2088-2137): <directory>/<model name>/ holding
    // architecture.json and parameters.binary.  The reference asks on stdin
    // whether to overwrite an existing directory and, on an empty or
    // negative answer, picks <name>_<k> with the first free k; this host
    // never reads stdin and always takes that default.  Returns the
    // directory written.
    std::string save_model(const std::string& directory) {
        namespace fs = std::filesystem;
        if (directory.empty()) throw std::invalid_argument("Model::save requires a non-empty directory path.");
        fs::path target = fs::path(directory) / model_name();
        if (fs::exists(target))
            for (int k = 1;; ++k) {
                auto candidate = fs::path(directory) / (model_name() + "_" + std::to_string(k));
                if (!fs::exists(candidate)) { target = candidate; break; }
            }
        fs::create_directories(target);
        const auto arch_path = target / "architecture.json";
        try {
            NA::write_file(arch_path.string(), architecture());
        } catch (const std::exception& e) {
            throw std::runtime_error("Failed to write architecture description to '" + arch_path.string() + "': " +
                                     e.what());
        }
        save((target / "parameters.binary").string());
        return target.string();
    }
    // Model::load (core.hpp:2140-2244) for a model whose layers are fixed:
    // the directory's architecture.json must describe this model's
    // descriptor list (the reference replays add() from it instead), then
    // every parameter and buffer is read from parameters.binary with the
    // key and shape checks of load_archive.  The file's name becomes the
    // model's name.
    void load_model(const std::string& directory) {
        namespace fs = std::filesystem;
        if (directory.empty()) throw std::invalid_argument("Model::load requires a non-empty directory path.");
        const auto arch_path = fs::path(directory) / "architecture.json";
        const auto params_path = fs::path(directory) / "parameters.binary";
        if (!fs::exists(arch_path))
            throw std::runtime_error("Architecture file not found at '" + arch_path.string() + "'.");
        if (!fs::exists(params_path))
            throw std::runtime_error("Parameter archive not found at '" + params_path.string() + "'.");
        NA::Node file;
        try {
            file = NA::read_file(arch_path.string());
        } catch (const std::exception& e) {
            throw std::runtime_error("Failed to read architecture description from '" + arch_path.string() + "': " +
                                     e.what());
        }
        const NA::Node* modules = file.find("modules");
        if (!modules)
            throw std::runtime_error("Architecture description '" + arch_path.string() +
                                     "' is missing the 'modules' entry.");
        NA::Node want;
        for (auto& m : model->descriptors()) want.push_back(std::move(m));
        std::string where;
        if (!NA::matches(want, *modules, where))
            throw std::runtime_error("Architecture description '" + arch_path.string() +
                                     "' describes another model (first difference at modules" + where + ").");
        const NA::Node* name = file.find("name");
        model_name_ = name ? name->data : std::string();
        load_archive(params_path.string());
    }
    // One replayed step: the batch goes into the graph's input buffers, the
    // optimizer's current options into its pinned hyper-parameter block.
    Tensor step_graph(const Tensor& x, const Tensor& y) {
        if (!graph) throw std::logic_error("step_graph: call capture() first");
        gx.copy_(x);
        gy.copy_(y);
        replay();
        return gloss.clone();
    }
    void replay() {
        fused->graph_sync();
        graph->replay();
        fused->graph_after_replay();
        for (auto& child : model->modules(/*include_self=*/true))
            if (auto* bn = child->template as<NH::BatchNorm2dImpl>()) bn->count_batch();
    }
    // Σ loss·batch accumulated on the device by the replayed steps since the
    // last reset (core.hpp:4481-4487), read back (one synchronisation).
    double loss_sum() {
        if (!loss_acc.defined()) throw std::logic_error("loss_sum: call capture() first");
        return loss_acc.item<double>();
    }
    void reset_loss_sum() {
        if (loss_acc.defined()) loss_acc.zero_();
    }
    // One epoch over host tensors as Model::run_epochs stages it
    // (core.hpp:4165-4305, 4481-4487): xs / ys hold whole batches in pinned
    // host memory; batch i+1 is copied to the device on a copy stream into
    // the other of two buffers while step i runs, each step is one graph
    // replay (optimizer and loss accumulation included), and the mean loss
    // of the epoch is read back once at the end.
    double train_epoch(const Tensor& xs, const Tensor& ys) {
        if (!graph) throw std::logic_error("train_epoch: call capture() first");
        if (!xs.is_pinned() || !ys.is_pinned()) throw std::invalid_argument("train_epoch: inputs must be pinned host tensors");
        const int64_t b = batch_rows, n = xs.size(0) / b;
        if (n * b != xs.size(0) || ys.size(0) != xs.size(0))
            throw std::invalid_argument("train_epoch: sample count must be a multiple of the captured batch");
        const auto dev = gx.device();
        const int di = dev.index();
        auto main = c10::hip::getCurrentHIPStream(di);
        auto copy = c10::hip::getStreamFromPool(false, di);
        std::array<Tensor, 2> bx{torch::empty_like(gx), torch::empty_like(gx)};
        std::array<Tensor, 2> by{torch::empty_like(gy), torch::empty_like(gy)};
        struct Events {
            hipEvent_t e[4] = {};
            Events() {
                for (auto& x : e)
                    if (hipEventCreateWithFlags(&x, hipEventDisableTiming) != hipSuccess)
                        throw std::runtime_error("train_epoch: hipEventCreate failed");
            }
            ~Events() {
                for (auto& x : e) (void)hipEventDestroy(x);
            }
        } ev;
        hipEvent_t* landed = ev.e;        // batch in buffer k is on the device
        hipEvent_t* consumed = ev.e + 2;  // buffer k was copied into the graph's inputs
        auto hip_ok = [](hipError_t e, const char* what) {
            if (e != hipSuccess) throw std::runtime_error(std::string("train_epoch: ") + what);
        };
        auto stage = [&](int64_t i) {
            const int k = (int)(i & 1);
            c10::hip::HIPStreamGuard g(copy);
            if (i >= 2) hip_ok(hipStreamWaitEvent(copy.stream(), consumed[k], 0), "wait");
            bx[k].copy_(xs.narrow(0, i * b, b).view(gx.sizes()), /*non_blocking=*/true);
            by[k].copy_(ys.narrow(0, i * b, b).view(gy.sizes()), /*non_blocking=*/true);
            hip_ok(hipEventRecord(landed[k], copy.stream()), "record");
        };
        reset_loss_sum();
        stage(0);
        for (int64_t i = 0; i < n; ++i) {
            const int k = (int)(i & 1);
            if (i + 1 < n) stage(i + 1);
            hip_ok(hipStreamWaitEvent(main.stream(), landed[k], 0), "wait");
            gx.copy_(bx[k], /*non_blocking=*/true);
            gy.copy_(by[k], /*non_blocking=*/true);
            hip_ok(hipEventRecord(consumed[k], main.stream()), "record");
            replay();
        }
        return loss_sum() / (double)(n * b);
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
        for (auto& child : model->modules(/*include_self=*/true))
            if (auto* bn = child->template as<NH::BatchNorm2dImpl>()) bn->sync_counter();
        std::map<std::string, Tensor> out;
        for (auto& kv : model->named_buffers()) out[kv.key()] = kv.value();
        return out;
    }
    // Copies values into named parameters or buffers (then refreshes the
    // bf16 copies).
    void load(const std::map<std::string, Tensor>& values) {
        torch::NoGradGuard ng;
        auto named = model->named_parameters();
        auto bufs = model->named_buffers();
        for (auto& kv : values) {
            if (auto* p = named.find(kv.first)) p->copy_(kv.second);
            else if (auto* b = bufs.find(kv.first)) b->copy_(kv.second);
            else throw std::invalid_argument("no parameter or buffer " + kv.first);
        }
        fused->refresh();
    }
    // Scheduler-style learning-rate write into a param group's options
    // (lrscheduler/details/cosineannealing.hpp:52-63).
    void set_lr(double lr) {
        for (auto& g : opt->param_groups()) g.options().set_lr(lr);
    }
    void set_fused_zero_grad(bool on) { fused->set_fused_zero_grad(on); }
    int64_t num_params() {
        int64_t n = 0;
        for (auto& p : model->parameters()) n += p.numel();
        return n;
    }
};

}  // namespace

// Parameter groups behind the fused optimizer, driven from Python through
// the torch::optim::Optimizer interface only (tests of the drop-in: groups
// with their own options, scheduler-style lr writes, zero_grad modes).
struct OptimizerHandle {
    std::unique_ptr<torch::optim::Optimizer> opt;
    OptimizerHandle(const std::vector<std::vector<Tensor>>& groups, const std::vector<double>& lrs,
                    const std::vector<double>& wds, bool decoupled, double beta1, double beta2, double eps) {
        if (groups.size() != lrs.size() || groups.size() != wds.size())
            throw std::invalid_argument("one lr and weight decay per group");
        auto make = [&](auto defaults, auto tag) {
            using Opts = decltype(defaults);
            std::vector<torch::optim::OptimizerParamGroup> pg;
            for (size_t i = 0; i < groups.size(); ++i) {
                auto o = std::make_unique<Opts>(lrs[i]);
                o->betas(std::make_tuple(beta1, beta2)).eps(eps).weight_decay(wds[i]);
                pg.emplace_back(groups[i], std::move(o));
            }
            defaults.betas(std::make_tuple(beta1, beta2)).eps(eps);
            using F = typename decltype(tag)::type;
            return std::unique_ptr<torch::optim::Optimizer>(new F(pg, defaults));
        };
        struct W { using type = NH::FusedAdamW; };
        struct A { using type = NH::FusedAdam; };
        opt = decoupled ? make(torch::optim::AdamWOptions(1e-3), W{}) : make(torch::optim::AdamOptions(1e-3), A{});
    }
};

PYBIND11_MODULE(_nott_host, m) {
    m.doc() = "C++ host layer (Nott::HIP) over libnott_hip: configs[0] and configs[4] training steps";
    // Workspace held by the device's contexts (one per stream used).
    m.def("workspace_bytes", [](int device) { return NH::device_workspace_bytes(device); }, py::arg("device") = 0);
    // Whether trainers run convolution weight gradients on the side stream
    // (on by default; the switch exists so tests can compare both orders).
    m.def("set_side_stream", [](bool on) { NH::set_side_stream_enabled(on); }, py::arg("on"));
    // architecture.json text of a model (no device needed): "small_cnn" or
    // "resnet18" with `classes` outputs.
    m.def("architecture_json", [](const std::string& model, int64_t classes, const std::string& name) {
        if (model == "small_cnn") return NA::to_json(NA::architecture(name, SmallCNNImpl::descriptors()));
        if (model == "resnet18") return NA::to_json(NA::architecture(name, ResNet18Impl::descriptors_for(classes)));
        throw std::invalid_argument("unknown model '" + model + "'");
    }, py::arg("model"), py::arg("classes") = 1000, py::arg("name") = "Nott::Model");
    // Initial parameters (CPU tensors by registration key) of a model as the
    // trainers initialise it from `seed` (no device needed).
    m.def("initial_parameters", [](const std::string& model, uint64_t seed, int64_t classes) {
        auto gen = at::detail::createCPUGenerator(seed);
        torch::Generator g(gen);
        std::shared_ptr<torch::nn::Module> net;
        if (model == "small_cnn") net = SmallCNN().ptr();
        else if (model == "resnet18") net = ResNet18(classes).ptr();
        else throw std::invalid_argument("unknown model '" + model + "'");
        NH::reference_init_(*net, g);
        std::map<std::string, Tensor> out;
        for (auto& kv : net->named_parameters()) out[kv.key()] = kv.value().detach().clone();
        return out;
    }, py::arg("model"), py::arg("seed"), py::arg("classes") = 1000);
    using SmallT = Trainer<SmallCNN, false>;
    py::class_<SmallT>(m, "SmallCNNTrainer")
        .def(py::init([](int device, uint64_t seed, double lr) {
                 // Adam, betas (0.9, 0.999), eps 1e-8, no weight decay
                 return new SmallT(SmallCNN(), false, torch::optim::AdamOptions(lr), device, seed);
             }),
             py::arg("device") = 0, py::arg("seed") = 0, py::arg("lr") = 1e-3)
        .def("step", &SmallT::step, py::call_guard<py::gil_scoped_release>())
        .def("warmup", &SmallT::warmup, py::arg("x"), py::arg("y"), py::arg("passes") = 2,
             py::call_guard<py::gil_scoped_release>())
        .def("capture", &SmallT::capture, py::arg("x"), py::arg("y"), py::arg("passes") = 2,
             py::call_guard<py::gil_scoped_release>())
        .def("step_graph", &SmallT::step_graph, py::call_guard<py::gil_scoped_release>())
        .def("train_epoch", &SmallT::train_epoch, py::call_guard<py::gil_scoped_release>())
        .def("loss_sum", &SmallT::loss_sum)
        .def("reset_loss_sum", &SmallT::reset_loss_sum)
        .def("save", &SmallT::save, py::arg("path"))
        .def("load_archive", &SmallT::load_archive, py::arg("path"))
        .def("save_model", &SmallT::save_model, py::arg("directory"))
        .def("load_model", &SmallT::load_model, py::arg("directory"))
        .def("architecture_json", &SmallT::architecture_json)
        .def("set_model_name", &SmallT::set_model_name)
        .def("model_name", &SmallT::model_name)
        .def("forward_backward", &SmallT::forward_backward, py::call_guard<py::gil_scoped_release>())
        .def("optimizer_step", &SmallT::optimizer_step, py::call_guard<py::gil_scoped_release>())
        .def("forward", &SmallT::forward, py::call_guard<py::gil_scoped_release>())
        .def("params", &SmallT::params)
        .def("grads", &SmallT::grads)
        .def("buffers", &SmallT::buffers)
        .def("load", &SmallT::load)
        .def("set_lr", &SmallT::set_lr)
        .def("set_fused_zero_grad", &SmallT::set_fused_zero_grad)
        .def("num_params", &SmallT::num_params);
    using ResT = Trainer<ResNet18, true>;
    py::class_<ResT>(m, "ResNet18Trainer")
        .def(py::init([](int device, uint64_t seed, bool bf16, double lr, double wd, int64_t classes) {
                 torch::optim::AdamWOptions o(lr);   // AdamW, betas (0.9, 0.999), eps 1e-8
                 o.weight_decay(wd);
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
        .def("train_epoch", &ResT::train_epoch, py::call_guard<py::gil_scoped_release>())
        .def("loss_sum", &ResT::loss_sum)
        .def("reset_loss_sum", &ResT::reset_loss_sum)
        .def("save", &ResT::save, py::arg("path"))
        .def("load_archive", &ResT::load_archive, py::arg("path"))
        .def("save_model", &ResT::save_model, py::arg("directory"))
        .def("load_model", &ResT::load_model, py::arg("directory"))
        .def("architecture_json", &ResT::architecture_json)
        .def("set_model_name", &ResT::set_model_name)
        .def("model_name", &ResT::model_name)
        .def("forward_backward", &ResT::forward_backward, py::call_guard<py::gil_scoped_release>())
        .def("optimizer_step", &ResT::optimizer_step, py::call_guard<py::gil_scoped_release>())
        .def("forward", &ResT::forward, py::call_guard<py::gil_scoped_release>())
        .def("params", &ResT::params)
        .def("grads", &ResT::grads)
        .def("buffers", &ResT::buffers)
        .def("load", &ResT::load)
        .def("set_lr", &ResT::set_lr)
        .def("set_fused_zero_grad", &ResT::set_fused_zero_grad)
        .def("forward_backward_recording",
             [](ResT& t, const Tensor& x, const Tensor& y) {
                 // forward + loss + backward, keeping the stem and block outputs
                 t.model->record = true;
                 t.model->outputs.clear();
                 Tensor loss;
                 {
                     py::gil_scoped_release nogil;
                     loss = t.forward_backward(x, y);
                 }
                 std::vector<Tensor> outs;
                 for (auto& o : t.model->outputs) outs.push_back(o.detach());
                 t.model->record = false;
                 t.model->outputs.clear();
                 return std::make_pair(loss, outs);
             })
        .def("num_params", &ResT::num_params);
    py::class_<OptimizerHandle>(m, "FusedOptimizer")
        .def(py::init<const std::vector<std::vector<Tensor>>&, const std::vector<double>&,
                      const std::vector<double>&, bool, double, double, double>(),
             py::arg("groups"), py::arg("lrs"), py::arg("weight_decays"), py::arg("decoupled"),
             py::arg("beta1") = 0.9, py::arg("beta2") = 0.999, py::arg("eps") = 1e-8)
        .def("step", [](OptimizerHandle& h) { h.opt->step(); }, py::call_guard<py::gil_scoped_release>())
        .def("zero_grad", [](OptimizerHandle& h, bool set_to_none) { h.opt->zero_grad(set_to_none); },
             py::arg("set_to_none") = false)
        .def("set_lr", [](OptimizerHandle& h, size_t group, double lr) {
                 h.opt->param_groups().at(group).options().set_lr(lr);
             })
        .def("num_groups", [](OptimizerHandle& h) { return h.opt->param_groups().size(); })
        .def("state_step", [](OptimizerHandle& h, const Tensor& p) {
                 auto it = h.opt->state().find(p.unsafeGetTensorImpl());
                 if (it == h.opt->state().end()) throw std::invalid_argument("no state for this parameter");
                 return dynamic_cast<torch::optim::AdamParamState*>(it->second.get())
                            ? static_cast<torch::optim::AdamParamState&>(*it->second).step()
                            : static_cast<torch::optim::AdamWParamState&>(*it->second).step();
             })
        .def("exp_avg", [](OptimizerHandle& h, const Tensor& p) {
                 auto it = h.opt->state().find(p.unsafeGetTensorImpl());
                 if (it == h.opt->state().end()) throw std::invalid_argument("no state for this parameter");
                 if (auto* a = dynamic_cast<torch::optim::AdamParamState*>(it->second.get())) return a->exp_avg();
                 return static_cast<torch::optim::AdamWParamState&>(*it->second).exp_avg();
             });
}
