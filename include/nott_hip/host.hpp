// nott_hip/host.hpp — C++ host layer of the MI355X backward path, behind
// Nott's layer / loss / optimizer interfaces.
//
// The reference builds each layer as a torch::nn module and lets libtorch
// autograd run the backward (reference src/layer/details/conv.hpp:177,
// fc.hpp:40, pooling.hpp:144,164, batchnorm.hpp:50, flatten.hpp:34,
// activation/details/relu.hpp:13, loss/details/ce.hpp:36,
// attention/details/kernel.hpp:20-96, optimizer/details/adam.hpp:63,159).
// Here every such node is a torch::autograd::Function whose forward and
// backward call libnott_hip through the C ABI (include/nott_hip.h) on the
// caller's current HIP stream; libtorch keeps only the graph walk, tensor
// storage and the caching allocator.
//
// Parameter gradients are written straight into `param.grad()` with the
// ABI's accumulate flag (AccumulateGrad semantics on a zero_grad'ed grad),
// and the function returns no gradient for the parameter, so libtorch never
// runs an accumulation kernel.  Gradient fan-out (a tensor read by two
// consumers, e.g. the residual skip) goes through Fork, whose backward sums
// the two gradients with nott_add.
//
// Errors: a negative ABI status becomes std::invalid_argument (bad shapes or
// options, as the reference's factories throw) or std::runtime_error
// (launch / allocation failures).
#pragma once

#include <torch/torch.h>
#include <c10/hip/HIPStream.h>

#include <array>
#include <cstring>
#include <atomic>
#include <map>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

#include "nott_hip.h"

namespace Nott {
namespace HIP {

using torch::Tensor;
using torch::autograd::AutogradContext;
using torch::autograd::variable_list;

// ------------------------------------------------------------------ runtime
// One context per (device, stream): a context's workspace is used only by
// launches on the stream it is bound to, so work that runs on different
// streams at the same time never shares a workspace.
namespace detail {
inline std::mutex& ctx_mutex() {
    static std::mutex mu;
    return mu;
}
inline std::map<std::pair<int, hipStream_t>, nott_ctx>& ctx_map() {
    static std::map<std::pair<int, hipStream_t>, nott_ctx> m;
    return m;
}
}  // namespace detail

inline nott_ctx stream_context(int device, hipStream_t stream) {
    if (device < 0 || device >= 64) throw std::invalid_argument("Nott::HIP: bad device index");
    std::lock_guard<std::mutex> g(detail::ctx_mutex());
    auto& m = detail::ctx_map();
    auto it = m.find({device, stream});
    if (it != m.end()) return it->second;
    nott_ctx c = nullptr;
    const int st = nott_create(device, &c);
    if (st != NOTT_OK) throw std::runtime_error(std::string("nott_create: ") + nott_status_string(st));
    nott_set_stream(c, (void*)stream);
    m.emplace(std::make_pair(device, stream), c);
    return c;
}

// Workspace held by all contexts of `device`.
inline int64_t device_workspace_bytes(int device) {
    std::lock_guard<std::mutex> g(detail::ctx_mutex());
    int64_t total = 0;
    for (auto& kv : detail::ctx_map()) {
        if (kv.first.first != device) continue;
        int64_t b = 0;
        if (nott_workspace_bytes(kv.second, &b) == NOTT_OK) total += b;
    }
    return total;
}

// The context of t's device and that device's current HIP stream.
inline nott_ctx bind(const Tensor& t) {
    if (!t.is_cuda()) throw std::invalid_argument("Nott::HIP: tensor must live on a HIP device");
    const int dev = t.device().index();
    return stream_context(dev, c10::hip::getCurrentHIPStream((c10::DeviceIndex)dev).stream());
}

// A HIP stream as the c10::Stream record_stream takes: tensors on these
// devices report device type CUDA, so the stream goes under that type (same
// stream id).
inline c10::Stream as_tensor_stream(const c10::hip::HIPStream& s, int dev) {
    return c10::Stream(c10::Stream::UNSAFE, c10::Device(c10::DeviceType::CUDA, (c10::DeviceIndex)dev), s.id());
}

inline void check(int st, nott_ctx c, const char* what) {
    if (st == NOTT_OK) return;
    const std::string msg = std::string(what) + ": " + nott_last_error(c);
    if (st == NOTT_ERR_INVALID_ARG || st == NOTT_ERR_UNSUPPORTED) throw std::invalid_argument(msg);
    throw std::runtime_error(msg);
}

// ------------------------------------------------------------- side stream
// A convolution's weight gradient reads only the saved input and the
// incoming gradient, and nothing reads it before the optimizer.  While a
// SideStreamScope is alive for a device (the trainers hold one around
// forward, loss and backward), weight gradients run on a second stream of
// that device (from the stream pool, default priority), after an event on
// the current stream, with a context of their own (so their workspace is
// not the data gradients'); the tensors they read are recorded on that
// stream for the caching allocator.  join_side_stream() makes the current
// stream wait for everything issued there; the scope's holder joins before
// anything reads the gradients.  Graph capture follows the fork and the
// join like any other cross-stream dependency.
namespace detail {
struct Side {
    nott_ctx ctx = nullptr;
    hipStream_t stream = nullptr;
    c10::Stream c10_stream{c10::Stream::DEFAULT, c10::Device(c10::DeviceType::CUDA, 0)};
    hipEvent_t fork = nullptr, join = nullptr;
    int depth = 0;          // live scopes
    bool pending = false;   // work issued since the last join
};
inline Side& side(int dev) {
    static std::array<Side, 64> s;
    return s.at((size_t)dev);
}
// Process-wide switch (on by default); off, scopes leave everything on the
// current stream.
inline std::atomic<bool>& side_allowed() {
    static std::atomic<bool> on{true};
    return on;
}
inline void hip_ok(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}
}  // namespace detail

class SideStreamScope {
  public:
    explicit SideStreamScope(int dev) : dev_(dev), active_(detail::side_allowed().load()) {
        if (!active_) return;
        detail::Side& s = detail::side(dev);
        if (!s.ctx) {
            auto hs = c10::hip::getStreamFromPool(false, (c10::DeviceIndex)dev);
            s.stream = hs.stream();
            s.c10_stream = as_tensor_stream(hs, dev);
            for (hipEvent_t* e : {&s.fork, &s.join})
                detail::hip_ok(hipEventCreateWithFlags(e, hipEventDisableTiming), "side stream event");
            s.ctx = stream_context(dev, s.stream);
        }
        ++s.depth;
    }
    // The outermost scope joins whatever is still forked (its holder joins
    // explicitly on the normal path; this covers a backward left by an
    // exception, so no side-stream work stays unjoined, under capture or not).
    ~SideStreamScope() {
        if (!active_) return;
        detail::Side& s = detail::side(dev_);
        if (--s.depth == 0 && s.pending) {
            hipStream_t cur = c10::hip::getCurrentHIPStream((c10::DeviceIndex)dev_).stream();
            if (hipEventRecord(s.join, s.stream) == hipSuccess) (void)hipStreamWaitEvent(cur, s.join, 0);
            s.pending = false;
        }
    }
    SideStreamScope(const SideStreamScope&) = delete;
    SideStreamScope& operator=(const SideStreamScope&) = delete;

  private:
    int dev_;
    bool active_;
};

inline void set_side_stream_enabled(bool on) { detail::side_allowed().store(on); }

// The context a weight gradient of `flops` on dy's device launches with: the
// side stream's (ordered after the current stream's work so far, `reads`
// recorded on it) while a scope is alive and the gradient is large enough to
// pay for the fork and join (measured: the small CNN's convolutions, under
// half a GFLOP, lost 8% of the step; ResNet-18's 0.8-GFLOP 1×1 shortcuts
// gain a little), else the ordinary one.
constexpr double kSideMinFlops = 6e8;
inline nott_ctx wgrad_context(const Tensor& dy, std::initializer_list<Tensor> reads, double flops) {
    nott_ctx c = bind(dy);
    const int dev = dy.device().index();
    detail::Side& s = detail::side(dev);
    if (s.depth == 0 || flops < kSideMinFlops) return c;
    hipStream_t cur = c10::hip::getCurrentHIPStream((c10::DeviceIndex)dev).stream();
    detail::hip_ok(hipEventRecord(s.fork, cur), "side stream fork");
    detail::hip_ok(hipStreamWaitEvent(s.stream, s.fork, 0), "side stream fork");
    for (const Tensor& t : reads)
        if (t.defined() && t.numel() > 0) const_cast<Tensor&>(t).record_stream(s.c10_stream);
    s.pending = true;
    return s.ctx;
}

// The current stream of `dev` waits for the side stream's work.
inline void join_side_stream(int dev) {
    detail::Side& s = detail::side(dev);
    if (!s.pending) return;
    hipStream_t cur = c10::hip::getCurrentHIPStream((c10::DeviceIndex)dev).stream();
    detail::hip_ok(hipEventRecord(s.join, s.stream), "side stream join");
    detail::hip_ok(hipStreamWaitEvent(cur, s.join, 0), "side stream join");
    s.pending = false;
}

inline nott_dtype dtype_of(const Tensor& t) {
    if (t.scalar_type() == torch::kFloat32) return NOTT_F32;
    if (t.scalar_type() == torch::kBFloat16) return NOTT_BF16;
    throw std::invalid_argument("Nott::HIP: tensors must be float32 or bfloat16");
}

// A defined, zero-element tensor stands for "absent" (e.g. no bias):
// autograd::Function::apply records the device of every tensor argument, so
// arguments must always be defined tensors.
inline bool present(const Tensor& t) { return t.defined() && t.numel() > 0; }
inline Tensor absent(const Tensor& like) { return torch::empty({0}, like.options().dtype(torch::kFloat32)); }
inline Tensor or_absent(const Tensor& t, const Tensor& like) { return t.defined() ? t : absent(like); }

inline void* ptr(const Tensor& t) { return present(t) ? t.data_ptr() : nullptr; }
inline float* fptr(const Tensor& t) { return present(t) ? t.data_ptr<float>() : nullptr; }

inline Tensor contig(const Tensor& t) { return t.is_contiguous() ? t : t.contiguous(); }

// Gradient buffers a fused optimizer keeps in its flat arena, by parameter.
// A parameter whose .grad() was reset to none (Optimizer::zero_grad(true))
// gets its arena slice back, zeroed, the next time a backward writes it, so
// one fused launch still sees every gradient.
namespace detail {
inline std::mutex& arena_mutex() {
    static std::mutex mu;
    return mu;
}
inline std::unordered_map<const c10::TensorImpl*, Tensor>& arena_grads() {
    static std::unordered_map<const c10::TensorImpl*, Tensor> m;
    return m;
}
inline Tensor arena_grad(const Tensor& p) {
    std::lock_guard<std::mutex> g(arena_mutex());
    auto it = arena_grads().find(p.unsafeGetTensorImpl());
    return it == arena_grads().end() ? Tensor() : it->second;
}
// A tensor over `arena`'s storage at element offset `off` with the given
// shape (contiguous).  It shares memory with the arena but is not an
// autograd view, so libtorch's Optimizer::zero_grad may detach_ it.
inline Tensor alias(const Tensor& arena, int64_t off, at::IntArrayRef sizes) {
    torch::NoGradGuard ng;
    std::vector<int64_t> strides(sizes.size(), 1);
    for (int64_t i = (int64_t)sizes.size() - 2; i >= 0; --i) strides[i] = strides[i + 1] * sizes[i + 1];
    Tensor t = torch::empty({0}, arena.options());
    t.set_(arena.storage(), arena.storage_offset() + off, sizes, strides);
    return t;
}
}  // namespace detail

// Ensures p.grad() exists (zeros) so that backward can accumulate into it.
inline Tensor grad_buffer(const Tensor& p) {
    if (!present(p) || !p.requires_grad()) return Tensor();
    if (!p.grad().defined()) {
        torch::NoGradGuard ng;
        Tensor g = detail::arena_grad(p);
        if (g.defined()) {
            nott_ctx c = bind(g);
            check(nott_zero(c, g.numel() * (int64_t)g.element_size(), g.data_ptr()), c, "gradient re-attach");
        } else {
            g = torch::zeros_like(p);
        }
        const_cast<Tensor&>(p).mutable_grad() = g;
    }
    return p.grad();
}

// --------------------------------------------------------------- Conv2d
// geometry = {stride_h, stride_w, pad_h, pad_w, dil_h, dil_w}
// 2·N·P·Q·K·C·R·S of a convolution whose output (or output gradient) is y.
inline double conv_flops(const nott_conv2d_desc& d, const Tensor& y) {
    return 2.0 * (double)y.numel() * (double)d.c * (double)d.r * (double)d.s;
}

// When x needs a gradient and the layer takes the 3×3 stride-1 kernels, the
// forward runs through nott_conv2d_fwd_prep, whose single weight-prep launch
// also writes the data gradient's weight layout into the returned tensor
// (saved for the backward, which then launches no prep); undefined
// otherwise, and the caller runs its ordinary forward.
inline Tensor prep_dgrad_weights(nott_ctx c, const nott_conv2d_desc& d, const Tensor& x, const Tensor& wc,
                                 const Tensor& b, int relu, Tensor& y) {
    int64_t bytes = 0;
    if (!x.requires_grad() || nott_conv2d_dgrad_prep_bytes(&d, dtype_of(x), &bytes) != NOTT_OK || bytes == 0)
        return Tensor();
    Tensor wd = torch::empty({bytes}, x.options().dtype(torch::kUInt8));
    check(nott_conv2d_fwd_prep(c, &d, dtype_of(x), ptr(x), ptr(wc), fptr(b), relu, ptr(y), wd.data_ptr()), c,
          "conv2d forward");
    return wd;
}
inline void dgrad_with(nott_ctx c, const nott_conv2d_desc& d, const Tensor& dy, const Tensor& wc, const Tensor& wd,
                       Tensor& dx) {
    if (wd.defined())
        check(nott_conv2d_bwd_data_prepped(c, &d, dtype_of(dy), ptr(dy), wd.data_ptr(), ptr(dx)), c, "conv2d dgrad");
    else
        check(nott_conv2d_bwd_data(c, &d, dtype_of(dy), ptr(dy), ptr(wc), ptr(dx)), c, "conv2d dgrad");
}

struct Conv2dFn : torch::autograd::Function<Conv2dFn> {
    static nott_conv2d_desc desc(const Tensor& x, const Tensor& w, const std::vector<int64_t>& g) {
        nott_conv2d_desc d{};
        d.n = x.size(0); d.c = x.size(1); d.h = x.size(2); d.w = x.size(3);
        d.k = w.size(0); d.r = w.size(2); d.s = w.size(3);
        d.stride_h = g[0]; d.stride_w = g[1]; d.pad_h = g[2]; d.pad_w = g[3]; d.dil_h = g[4]; d.dil_w = g[5];
        d.groups = 1; d.layout = NOTT_NCHW;
        return d;
    }
    // x: input; w: master weight (fp32, receives the gradient); wc: weight in
    // the compute dtype (== w for fp32); b: fp32 bias or undefined.
    static Tensor forward(AutogradContext* ctx, Tensor x, Tensor w, Tensor wc, Tensor b, std::vector<int64_t> geom) {
        x = contig(x);
        const nott_conv2d_desc d = desc(x, wc, geom);
        const int64_t p = (d.h + 2 * d.pad_h - d.dil_h * (d.r - 1) - 1) / d.stride_h + 1;
        const int64_t q = (d.w + 2 * d.pad_w - d.dil_w * (d.s - 1) - 1) / d.stride_w + 1;
        Tensor y = torch::empty({d.n, d.k, p, q}, x.options());
        nott_ctx c = bind(x);
        Tensor wd = prep_dgrad_weights(c, d, x, wc, b, 0, y);
        if (!wd.defined()) check(nott_conv2d_fwd(c, &d, dtype_of(x), ptr(x), ptr(wc), fptr(b), ptr(y)), c, "conv2d forward");
        ctx->save_for_backward({x, w, wc, b, wd});
        ctx->saved_data["geom"] = geom;
        ctx->saved_data["needs_dx"] = x.requires_grad();
        return y;
    }
    static variable_list backward(AutogradContext* ctx, variable_list grads) {
        auto s = ctx->get_saved_variables();
        Tensor x = s[0], w = s[1], wc = s[2], b = s[3], wd = s[4];
        Tensor dy = contig(grads[0]);
        const auto geom = ctx->saved_data["geom"].toIntVector();
        const nott_conv2d_desc d = desc(x, wc, geom);
        nott_ctx c = bind(dy);
        Tensor dx;
        if (ctx->saved_data["needs_dx"].toBool()) {
            dx = torch::empty_like(x);
            dgrad_with(c, d, dy, wc, wd, dx);
        }
        Tensor gw = grad_buffer(w), gb = grad_buffer(b);
        if (gw.defined() || gb.defined()) {
            // the side stream only where a data gradient runs beside it: the
            // first layer's weight gradient (no dx) ends backward, and queued
            // behind the side stream's backlog it would only delay the join
            // (ResNet-18 bf16 step 3.099 -> 3.077 ms)
            nott_ctx cw = dx.defined() ? wgrad_context(dy, {x, dy}, conv_flops(d, dy)) : c;
            check(nott_conv2d_bwd_weight(cw, &d, dtype_of(dy), ptr(x), ptr(dy), fptr(gw), fptr(gb), 1), cw,
                  "conv2d wgrad");
        }
        return {dx, Tensor(), Tensor(), Tensor(), Tensor()};
    }
};

// Conv2d followed by ReLU, the activation fused into the convolution's
// forward (nott_conv2d_fwd_act); backward = ReLU mask from the saved output,
// then the convolution's gradients.  consumer_masks: the output's only
// consumer applies the ReLU's backward itself (a max-pool taking it with
// forward_relu_input), so the gradient arrives masked.
struct Conv2dReluFn : torch::autograd::Function<Conv2dReluFn> {
    static Tensor forward(AutogradContext* ctx, Tensor x, Tensor w, Tensor wc, Tensor b, std::vector<int64_t> geom,
                          bool consumer_masks) {
        x = contig(x);
        const nott_conv2d_desc d = Conv2dFn::desc(x, wc, geom);
        const int64_t p = (d.h + 2 * d.pad_h - d.dil_h * (d.r - 1) - 1) / d.stride_h + 1;
        const int64_t q = (d.w + 2 * d.pad_w - d.dil_w * (d.s - 1) - 1) / d.stride_w + 1;
        Tensor y = torch::empty({d.n, d.k, p, q}, x.options());
        nott_ctx c = bind(x);
        Tensor wd = prep_dgrad_weights(c, d, x, wc, b, 1, y);
        if (!wd.defined())
            check(nott_conv2d_fwd_act(c, &d, dtype_of(x), ptr(x), ptr(wc), fptr(b), 1, ptr(y)), c, "conv2d+relu forward");
        ctx->save_for_backward({x, w, wc, b, y, wd});
        ctx->saved_data["geom"] = geom;
        ctx->saved_data["needs_dx"] = x.requires_grad();
        ctx->saved_data["consumer_masks"] = consumer_masks;
        return y;
    }
    static variable_list backward(AutogradContext* ctx, variable_list grads) {
        auto s = ctx->get_saved_variables();
        Tensor x = s[0], w = s[1], wc = s[2], b = s[3], y = s[4], wd = s[5];
        Tensor dy = contig(grads[0]);
        const auto geom = ctx->saved_data["geom"].toIntVector();
        const nott_conv2d_desc d = Conv2dFn::desc(x, wc, geom);
        nott_ctx c = bind(dy);
        Tensor dz = dy;
        if (!ctx->saved_data["consumer_masks"].toBool()) {
            dz = torch::empty_like(dy);
            check(nott_relu_bwd(c, dtype_of(dy), dy.numel(), ptr(y), ptr(dy), ptr(dz)), c, "relu backward");
        }
        Tensor dx;
        if (ctx->saved_data["needs_dx"].toBool()) {
            dx = torch::empty_like(x);
            dgrad_with(c, d, dz, wc, wd, dx);
        }
        Tensor gw = grad_buffer(w), gb = grad_buffer(b);
        if (gw.defined() || gb.defined()) {
            nott_ctx cw = dx.defined() ? wgrad_context(dz, {x, dz}, conv_flops(d, dz)) : c;
            check(nott_conv2d_bwd_weight(cw, &d, dtype_of(dz), ptr(x), ptr(dz), fptr(gw), fptr(gb), 1), cw,
                  "conv2d wgrad");
        }
        return {dx, Tensor(), Tensor(), Tensor(), Tensor(), Tensor()};
    }
};

// --------------------------------------------------------------- Linear
// flags: kLinRelu, the layer's ReLU fused into the forward GEMM (backward:
// the ReLU mask from the saved output, unless kLinConsumerMasks says the
// output's only consumer applies it); kLinReluInput, x is the previous
// layer's ReLU output and dx takes that ReLU's backward (its producer then
// skips it).
constexpr int64_t kLinRelu = 1, kLinConsumerMasks = 2, kLinReluInput = 4;
struct LinearFn : torch::autograd::Function<LinearFn> {
    static Tensor forward(AutogradContext* ctx, Tensor x, Tensor w, Tensor wc, Tensor b, int64_t flags) {
        x = contig(x);
        const int64_t kin = x.size(-1), m = x.numel() / kin, nout = wc.size(0);
        auto shape = x.sizes().vec();
        shape.back() = nout;
        Tensor y = torch::empty(shape, x.options());
        nott_ctx c = bind(x);
        const bool relu = (flags & kLinRelu) != 0;
        check(nott_linear_fwd_act(c, dtype_of(x), m, kin, nout, ptr(x), ptr(wc), fptr(b), relu ? 1 : 0, ptr(y)), c,
              "linear forward");
        ctx->save_for_backward({x, w, wc, b, relu && !(flags & kLinConsumerMasks) ? y : Tensor()});
        ctx->saved_data["needs_dx"] = x.requires_grad();
        ctx->saved_data["flags"] = flags;
        return y;
    }
    static variable_list backward(AutogradContext* ctx, variable_list grads) {
        auto s = ctx->get_saved_variables();
        Tensor x = s[0], w = s[1], wc = s[2], b = s[3], y = s[4];
        Tensor dy = contig(grads[0]);
        const int64_t kin = x.size(-1), m = x.numel() / kin, nout = wc.size(0);
        const int64_t flags = ctx->saved_data["flags"].toInt();
        nott_ctx c = bind(dy);
        Tensor dz = dy;
        if (y.defined()) {
            dz = torch::empty_like(dy);
            check(nott_relu_bwd(c, dtype_of(dy), dy.numel(), ptr(y), ptr(dy), ptr(dz)), c, "relu backward");
        }
        Tensor dx = ctx->saved_data["needs_dx"].toBool() ? torch::empty_like(x) : Tensor();
        Tensor gw = grad_buffer(w), gb = grad_buffer(b);
        check(nott_linear_bwd_act(c, dtype_of(dz), m, kin, nout, ptr(dz), ptr(x), ptr(wc), ptr(dx), fptr(gw), fptr(gb),
                                  1, (flags & kLinReluInput) ? 1 : 0),
              c, "linear backward");
        return {dx, Tensor(), Tensor(), Tensor(), Tensor()};
    }
};

// ----------------------------------------------------------------- ReLU
struct ReluFn : torch::autograd::Function<ReluFn> {
    static Tensor forward(AutogradContext* ctx, Tensor x) {
        x = contig(x);
        Tensor y = torch::empty_like(x);
        nott_ctx c = bind(x);
        check(nott_relu_fwd(c, dtype_of(x), x.numel(), ptr(x), ptr(y)), c, "relu forward");
        ctx->save_for_backward({y});
        return y;
    }
    static variable_list backward(AutogradContext* ctx, variable_list grads) {
        Tensor y = ctx->get_saved_variables()[0];
        Tensor dy = contig(grads[0]);
        Tensor dx = torch::empty_like(dy);
        nott_ctx c = bind(dy);
        check(nott_relu_bwd(c, dtype_of(dy), dy.numel(), ptr(y), ptr(dy), ptr(dx)), c, "relu backward");
        return {dx};
    }
};

// ------------------------------------------------------------ MaxPool2d
// geometry = {kh, kw, stride_h, stride_w, pad_h, pad_w, dil_h, dil_w, ceil_mode}
// relu_input: x is the output of a ReLU whose backward this layer's backward
// applies (nott_maxpool2d_bwd_tap_relu), its producer skipping it.
struct MaxPool2dFn : torch::autograd::Function<MaxPool2dFn> {
    static nott_pool2d_desc desc(const Tensor& x, const std::vector<int64_t>& g) {
        nott_pool2d_desc d{};
        d.n = x.size(0); d.c = x.size(1); d.h = x.size(2); d.w = x.size(3);
        d.kh = g[0]; d.kw = g[1]; d.stride_h = g[2]; d.stride_w = g[3]; d.pad_h = g[4]; d.pad_w = g[5];
        d.dil_h = g[6]; d.dil_w = g[7]; d.ceil_mode = (int32_t)g[8]; d.layout = NOTT_NCHW;
        return d;
    }
    static int64_t out(int64_t in, int64_t k, int64_t s, int64_t p, int64_t dl, bool ceil) {
        int64_t num = in + 2 * p - dl * (k - 1) - 1 + (ceil ? s - 1 : 0);
        int64_t o = num / s + 1;
        if (ceil && (o - 1) * s >= in + p) --o;
        return o;
    }
    static Tensor forward(AutogradContext* ctx, Tensor x, std::vector<int64_t> geom, bool relu_input) {
        x = contig(x);
        const nott_pool2d_desc d = desc(x, geom);
        const int64_t oh = out(d.h, d.kh, d.stride_h, d.pad_h, d.dil_h, d.ceil_mode),
                      ow = out(d.w, d.kw, d.stride_w, d.pad_w, d.dil_w, d.ceil_mode);
        Tensor y = torch::empty({d.n, d.c, oh, ow}, x.options());
        nott_ctx c = bind(x);
        // The indices stay inside the layer, so windows of up to 256 taps keep
        // them as one-byte window taps rather than ATen's int64 flat indices
        // (the same routing, 1/8 of the index traffic).
        Tensor idx;
        if (d.kh * d.kw <= 256) {
            idx = torch::empty({d.n, d.c, oh, ow}, x.options().dtype(torch::kUInt8));
            check(nott_maxpool2d_fwd_tap(c, &d, dtype_of(x), ptr(x), ptr(y), idx.data_ptr<uint8_t>()), c,
                  "maxpool forward");
        } else {
            idx = torch::empty({d.n, d.c, oh, ow}, x.options().dtype(torch::kInt64));
            check(nott_maxpool2d_fwd(c, &d, dtype_of(x), ptr(x), ptr(y), idx.data_ptr<int64_t>()), c,
                  "maxpool forward");
        }
        ctx->save_for_backward({idx, relu_input ? x : Tensor()});
        ctx->saved_data["geom"] = geom;
        ctx->saved_data["xshape"] = x.sizes().vec();
        ctx->mark_non_differentiable({idx});
        return y;
    }
    static variable_list backward(AutogradContext* ctx, variable_list grads) {
        auto s = ctx->get_saved_variables();
        Tensor idx = s[0], rx = s[1];
        Tensor dy = contig(grads[0]);
        const auto xs = ctx->saved_data["xshape"].toIntVector();
        Tensor dx = torch::empty(xs, dy.options());
        const nott_pool2d_desc d = desc(dx, ctx->saved_data["geom"].toIntVector());
        nott_ctx c = bind(dy);
        if (idx.scalar_type() == torch::kUInt8 && rx.defined())
            check(nott_maxpool2d_bwd_tap_relu(c, &d, dtype_of(dy), idx.data_ptr<uint8_t>(), ptr(dy), ptr(rx), ptr(dx)),
                  c, "maxpool+relu backward");
        else if (idx.scalar_type() == torch::kUInt8)
            check(nott_maxpool2d_bwd_tap(c, &d, dtype_of(dy), idx.data_ptr<uint8_t>(), ptr(dy), ptr(dx)), c,
                  "maxpool backward");
        else
            check(nott_maxpool2d_bwd(c, &d, dtype_of(dy), idx.data_ptr<int64_t>(), ptr(dy), ptr(dx)), c,
                  "maxpool backward");
        if (rx.defined() && idx.scalar_type() != torch::kUInt8)
            check(nott_relu_bwd(c, dtype_of(dx), dx.numel(), ptr(rx), ptr(dx), ptr(dx)), c, "relu backward");
        return {dx, Tensor(), Tensor()};
    }
};

// ------------------------------------------- AdaptiveAvgPool2d({1, 1})
struct AvgPoolGlobalFn : torch::autograd::Function<AvgPoolGlobalFn> {
    static Tensor forward(AutogradContext* ctx, Tensor x) {
        x = contig(x);
        Tensor y = torch::empty({x.size(0), x.size(1), 1, 1}, x.options());
        nott_ctx c = bind(x);
        check(nott_avgpool_global_fwd(c, dtype_of(x), x.size(0) * x.size(1), x.size(2) * x.size(3), ptr(x), ptr(y)), c,
              "avgpool forward");
        ctx->saved_data["xshape"] = x.sizes().vec();
        return y;
    }
    static variable_list backward(AutogradContext* ctx, variable_list grads) {
        Tensor dy = contig(grads[0]);
        const auto xs = ctx->saved_data["xshape"].toIntVector();
        Tensor dx = torch::empty(xs, dy.options());
        nott_ctx c = bind(dy);
        check(nott_avgpool_global_bwd(c, dtype_of(dy), xs[0] * xs[1], xs[2] * xs[3], ptr(dy), ptr(dx)), c,
              "avgpool backward");
        return {dx};
    }
};

// ---------------------------------------------------------- BatchNorm2d
// Training mode (batch statistics; running stats updated in forward).
struct BatchNorm2dFn : torch::autograd::Function<BatchNorm2dFn> {
    static Tensor forward(AutogradContext* ctx, Tensor x, Tensor gamma, Tensor beta, Tensor running_mean,
                          Tensor running_var, double eps, double momentum) {
        x = contig(x);
        const int64_t n = x.size(0), ch = x.size(1), hw = x.size(2) * x.size(3);
        Tensor y = torch::empty_like(x);
        auto fo = x.options().dtype(torch::kFloat32);
        Tensor mean = torch::empty({ch}, fo), rstd = torch::empty({ch}, fo);
        nott_ctx c = bind(x);
        check(nott_batchnorm2d_fwd(c, dtype_of(x), n, ch, hw, ptr(x), fptr(gamma), fptr(beta), eps, momentum,
                                   fptr(running_mean), fptr(running_var), ptr(y), fptr(mean), fptr(rstd)),
              c, "batchnorm forward");
        ctx->save_for_backward({x, gamma, beta, mean, rstd});
        ctx->saved_data["needs_dx"] = x.requires_grad();
        return y;
    }
    static variable_list backward(AutogradContext* ctx, variable_list grads) {
        auto s = ctx->get_saved_variables();
        Tensor x = s[0], gamma = s[1], beta = s[2], mean = s[3], rstd = s[4];
        Tensor dy = contig(grads[0]);
        const int64_t n = x.size(0), ch = x.size(1), hw = x.size(2) * x.size(3);
        Tensor dx = ctx->saved_data["needs_dx"].toBool() ? torch::empty_like(x) : Tensor();
        Tensor gg = grad_buffer(gamma), gbt = grad_buffer(beta);
        nott_ctx c = bind(dy);
        check(nott_batchnorm2d_bwd(c, dtype_of(dy), n, ch, hw, ptr(x), ptr(dy), fptr(mean), fptr(rstd), fptr(gamma),
                                   ptr(dx), fptr(gg), fptr(gbt), 1),
              c, "batchnorm backward");
        return {dx, Tensor(), Tensor(), Tensor(), Tensor(), Tensor(), Tensor()};
    }
};

// BatchNorm2d followed by the layer's ReLU (block/details/blocks/residual.hpp:
// 94-96: the layer, then Activation::Details::apply): one apply pass forward;
// the backward recomputes the ReLU mask from x inside the BN backward.
struct BatchNorm2dReluFn : torch::autograd::Function<BatchNorm2dReluFn> {
    static Tensor forward(AutogradContext* ctx, Tensor x, Tensor gamma, Tensor beta, Tensor running_mean,
                          Tensor running_var, double eps, double momentum) {
        x = contig(x);
        const int64_t n = x.size(0), ch = x.size(1), hw = x.size(2) * x.size(3);
        Tensor y = torch::empty_like(x);
        auto fo = x.options().dtype(torch::kFloat32);
        Tensor mean = torch::empty({ch}, fo), rstd = torch::empty({ch}, fo);
        nott_ctx c = bind(x);
        check(nott_batchnorm2d_fwd_act(c, dtype_of(x), n, ch, hw, ptr(x), fptr(gamma), fptr(beta), eps, momentum,
                                       fptr(running_mean), fptr(running_var), nullptr, 1, ptr(y), fptr(mean),
                                       fptr(rstd)),
              c, "batchnorm+relu forward");
        ctx->save_for_backward({x, gamma, beta, mean, rstd});
        ctx->saved_data["needs_dx"] = x.requires_grad();
        return y;
    }
    static variable_list backward(AutogradContext* ctx, variable_list grads) {
        auto s = ctx->get_saved_variables();
        Tensor x = s[0], gamma = s[1], beta = s[2], mean = s[3], rstd = s[4];
        Tensor dy = contig(grads[0]);
        const int64_t n = x.size(0), ch = x.size(1), hw = x.size(2) * x.size(3);
        Tensor dx = ctx->saved_data["needs_dx"].toBool() ? torch::empty_like(x) : Tensor();
        Tensor gg = grad_buffer(gamma), gbt = grad_buffer(beta);
        nott_ctx c = bind(dy);
        check(nott_batchnorm2d_bwd_act(c, dtype_of(dy), n, ch, hw, ptr(x), ptr(dy), fptr(mean), fptr(rstd),
                                       fptr(gamma), fptr(beta), 1, ptr(dx), fptr(gg), fptr(gbt), 1),
              c, "batchnorm+relu backward");
        return {dx, Tensor(), Tensor(), Tensor(), Tensor(), Tensor(), Tensor()};
    }
};

// BatchNorm2d + ReLU followed by a max-pool (ResNet-18's stem: batchnorm.hpp:50
// with its ReLU, then pooling.hpp:144) without the BatchNorm's output in
// memory: the statistics pass, then the pool forms relu(a·x + c) from x as
// it stages its rows (nott_batchnorm2d_fwd_coef, nott_maxpool2d_fwd_tap_bnrelu).
// Backward: the pool's routing into a [n, c, h, w] gradient, then the
// BatchNorm + ReLU backward (mask recomputed from x), as the two layers do.
struct BatchNorm2dReluMaxPool2dFn : torch::autograd::Function<BatchNorm2dReluMaxPool2dFn> {
    static Tensor forward(AutogradContext* ctx, Tensor x, Tensor gamma, Tensor beta, Tensor running_mean,
                          Tensor running_var, double eps, double momentum, std::vector<int64_t> pool_geom) {
        x = contig(x);
        const int64_t n = x.size(0), ch = x.size(1), hw = x.size(2) * x.size(3);
        auto fo = x.options().dtype(torch::kFloat32);
        Tensor mean = torch::empty({ch}, fo), rstd = torch::empty({ch}, fo), coef = torch::empty({2 * ch}, fo);
        nott_ctx c = bind(x);
        check(nott_batchnorm2d_fwd_coef(c, dtype_of(x), n, ch, hw, ptr(x), fptr(gamma), fptr(beta), eps, momentum,
                                        fptr(running_mean), fptr(running_var), fptr(mean), fptr(rstd), fptr(coef)),
              c, "batchnorm statistics");
        const nott_pool2d_desc d = MaxPool2dFn::desc(x, pool_geom);
        const int64_t oh = MaxPool2dFn::out(d.h, d.kh, d.stride_h, d.pad_h, d.dil_h, d.ceil_mode),
                      ow = MaxPool2dFn::out(d.w, d.kw, d.stride_w, d.pad_w, d.dil_w, d.ceil_mode);
        Tensor y = torch::empty({n, ch, oh, ow}, x.options());
        Tensor tap = torch::empty({n, ch, oh, ow}, x.options().dtype(torch::kUInt8));
        check(nott_maxpool2d_fwd_tap_bnrelu(c, &d, dtype_of(x), ptr(x), fptr(coef), ptr(y), tap.data_ptr<uint8_t>()),
              c, "batchnorm+relu+maxpool forward");
        ctx->save_for_backward({x, gamma, beta, mean, rstd, tap});
        ctx->saved_data["geom"] = pool_geom;
        ctx->saved_data["needs_dx"] = x.requires_grad();
        ctx->mark_non_differentiable({tap});
        return y;
    }
    static variable_list backward(AutogradContext* ctx, variable_list grads) {
        auto s = ctx->get_saved_variables();
        Tensor x = s[0], gamma = s[1], beta = s[2], mean = s[3], rstd = s[4], tap = s[5];
        Tensor dy = contig(grads[0]);
        nott_ctx c = bind(dy);
        const nott_pool2d_desc d = MaxPool2dFn::desc(x, ctx->saved_data["geom"].toIntVector());
        Tensor dx = ctx->saved_data["needs_dx"].toBool() ? torch::empty_like(x) : Tensor();
        Tensor gg = grad_buffer(gamma), gbt = grad_buffer(beta);
        check(nott_batchnorm2d_relu_maxpool2d_bwd(c, &d, dtype_of(dy), ptr(x), tap.data_ptr<uint8_t>(), ptr(dy),
                                                  fptr(mean), fptr(rstd), fptr(gamma), fptr(beta), ptr(dx), fptr(gg),
                                                  fptr(gbt), 1),
              c, "batchnorm+relu+maxpool backward");
        return {dx, Tensor(), Tensor(), Tensor(), Tensor(), Tensor(), Tensor(), Tensor()};
    }
};

// The second BatchNorm2d of a residual branch with the skip addition and the
// block's final ReLU (residual.hpp:130-132): y = relu(BN(x) + skip) in one
// apply pass.  Backward: dz = dy·[y > 0] feeds both the BN backward and the
// skip; consumer_masks: y's only consumer is the next block's fork, which
// applies the ReLU's backward itself (dz = dy then).
struct BatchNorm2dAddReluFn : torch::autograd::Function<BatchNorm2dAddReluFn> {
    static Tensor forward(AutogradContext* ctx, Tensor x, Tensor skip, Tensor gamma, Tensor beta,
                          Tensor running_mean, Tensor running_var, double eps, double momentum, bool consumer_masks) {
        x = contig(x);
        skip = contig(skip);
        const int64_t n = x.size(0), ch = x.size(1), hw = x.size(2) * x.size(3);
        Tensor y = torch::empty_like(x);
        auto fo = x.options().dtype(torch::kFloat32);
        Tensor mean = torch::empty({ch}, fo), rstd = torch::empty({ch}, fo);
        nott_ctx c = bind(x);
        check(nott_batchnorm2d_fwd_act(c, dtype_of(x), n, ch, hw, ptr(x), fptr(gamma), fptr(beta), eps, momentum,
                                       fptr(running_mean), fptr(running_var), ptr(skip), 1, ptr(y), fptr(mean),
                                       fptr(rstd)),
              c, "batchnorm+add+relu forward");
        ctx->save_for_backward({x, gamma, beta, mean, rstd, consumer_masks ? Tensor() : y});
        ctx->saved_data["needs_dx"] = x.requires_grad();
        return y;
    }
    static variable_list backward(AutogradContext* ctx, variable_list grads) {
        auto s = ctx->get_saved_variables();
        Tensor x = s[0], gamma = s[1], beta = s[2], mean = s[3], rstd = s[4], y = s[5];
        Tensor dy = contig(grads[0]);
        const int64_t n = x.size(0), ch = x.size(1), hw = x.size(2) * x.size(3);
        nott_ctx c = bind(dy);
        Tensor dz = dy;
        if (y.defined()) {
            dz = torch::empty_like(dy);
            check(nott_relu_bwd(c, dtype_of(dy), dy.numel(), ptr(y), ptr(dy), ptr(dz)), c, "block relu backward");
        }
        Tensor dx = ctx->saved_data["needs_dx"].toBool() ? torch::empty_like(x) : Tensor();
        Tensor gg = grad_buffer(gamma), gbt = grad_buffer(beta);
        check(nott_batchnorm2d_bwd(c, dtype_of(dz), n, ch, hw, ptr(x), ptr(dz), fptr(mean), fptr(rstd), fptr(gamma),
                                   ptr(dx), fptr(gg), fptr(gbt), 1),
              c, "batchnorm backward");
        return {dx, dz, Tensor(), Tensor(), Tensor(), Tensor(), Tensor(), Tensor(), Tensor()};
    }
};

// ------------------------------------------------------------ LayerNorm
struct LayerNormFn : torch::autograd::Function<LayerNormFn> {
    static Tensor forward(AutogradContext* ctx, Tensor x, Tensor gamma, Tensor beta, Tensor gamma_c, Tensor beta_c,
                          double eps) {
        x = contig(x);
        const int64_t d = x.size(-1), rows = x.numel() / d;
        Tensor y = torch::empty_like(x);
        auto fo = x.options().dtype(torch::kFloat32);
        Tensor mean = torch::empty({rows}, fo), rstd = torch::empty({rows}, fo);
        nott_ctx c = bind(x);
        check(nott_layernorm_fwd(c, dtype_of(x), rows, d, ptr(x), ptr(gamma_c), ptr(beta_c), eps, ptr(y), fptr(mean),
                                 fptr(rstd)),
              c, "layernorm forward");
        ctx->save_for_backward({x, gamma, beta, gamma_c, mean, rstd});
        ctx->saved_data["needs_dx"] = x.requires_grad();
        return y;
    }
    static variable_list backward(AutogradContext* ctx, variable_list grads) {
        auto s = ctx->get_saved_variables();
        Tensor x = s[0], gamma = s[1], beta = s[2], gamma_c = s[3], mean = s[4], rstd = s[5];
        Tensor dy = contig(grads[0]);
        const int64_t d = x.size(-1), rows = x.numel() / d;
        Tensor dx = torch::empty_like(x);
        Tensor gg = grad_buffer(gamma), gbt = grad_buffer(beta);
        nott_ctx c = bind(dy);
        check(nott_layernorm_bwd(c, dtype_of(dy), rows, d, ptr(x), ptr(dy), fptr(mean), fptr(rstd), ptr(gamma_c),
                                 ptr(dx), fptr(gg), fptr(gbt), 1),
              c, "layernorm backward");
        return {ctx->saved_data["needs_dx"].toBool() ? dx : Tensor(), Tensor(), Tensor(), Tensor(), Tensor(),
                Tensor()};
    }
};

// ------------------------------------------ scaled dot-product attention
struct AttentionFn : torch::autograd::Function<AttentionFn> {
    static nott_attn_desc desc(const Tensor& q, const Tensor& k, bool causal, double scale) {
        nott_attn_desc d{};
        d.b = q.size(0); d.h = q.size(1); d.t = q.size(2); d.s = k.size(2); d.dh = q.size(3);
        d.causal = causal; d.scale = scale;
        return d;
    }
    static Tensor forward(AutogradContext* ctx, Tensor q, Tensor k, Tensor v, bool causal, double scale) {
        q = contig(q); k = contig(k); v = contig(v);
        const nott_attn_desc d = desc(q, k, causal, scale);
        Tensor o = torch::empty_like(q);
        Tensor lse = torch::empty({d.b, d.h, d.t}, q.options().dtype(torch::kFloat32));
        nott_ctx c = bind(q);
        check(nott_attention_fwd(c, &d, dtype_of(q), ptr(q), ptr(k), ptr(v), ptr(o), fptr(lse)), c,
              "attention forward");
        ctx->save_for_backward({q, k, v, o, lse});
        ctx->saved_data["causal"] = causal;
        ctx->saved_data["scale"] = scale;
        return o;
    }
    static variable_list backward(AutogradContext* ctx, variable_list grads) {
        auto s = ctx->get_saved_variables();
        Tensor q = s[0], k = s[1], v = s[2], o = s[3], lse = s[4];
        Tensor dO = contig(grads[0]);
        const nott_attn_desc d = desc(q, k, ctx->saved_data["causal"].toBool(), ctx->saved_data["scale"].toDouble());
        Tensor dq = torch::empty_like(q), dk = torch::empty_like(k), dv = torch::empty_like(v);
        nott_ctx c = bind(q);
        check(nott_attention_bwd(c, &d, dtype_of(q), ptr(q), ptr(k), ptr(v), ptr(o), ptr(dO), fptr(lse), ptr(dq),
                                 ptr(dk), ptr(dv)),
              c, "attention backward");
        return {dq, dk, dv, Tensor(), Tensor()};
    }
};

// ---------------------------------------------------------------- Fork
// Two uses of one tensor (residual skip): backward sums the two gradients.
// relu_input: x is the previous block's output, a ReLU output whose backward
// is applied here (nott_add_relu_bwd), its producer skipping it.
struct ForkFn : torch::autograd::Function<ForkFn> {
    static variable_list forward(AutogradContext* ctx, Tensor x, bool relu_input) {
        ctx->save_for_backward({relu_input ? x : Tensor()});
        return {x.view(x.sizes()), x.view(x.sizes())};
    }
    static variable_list backward(AutogradContext* ctx, variable_list grads) {
        Tensor y = ctx->get_saved_variables()[0];
        if (!grads[0].defined() || !grads[1].defined()) {
            Tensor g = contig(grads[0].defined() ? grads[0] : grads[1]);
            if (!y.defined() || !g.defined()) return {g, Tensor()};
            Tensor out = torch::empty_like(g);
            nott_ctx c = bind(g);
            check(nott_relu_bwd(c, dtype_of(g), g.numel(), ptr(y), ptr(g), ptr(out)), c, "fork relu backward");
            return {out, Tensor()};
        }
        Tensor a = contig(grads[0]), b = contig(grads[1]);
        Tensor out = torch::empty_like(a);
        nott_ctx c = bind(a);
        if (y.defined())
            check(nott_add_relu_bwd(c, dtype_of(a), a.numel(), ptr(a), ptr(b), ptr(y), ptr(out)), c,
                  "fork add+relu backward");
        else
            check(nott_add(c, dtype_of(a), a.numel(), ptr(a), ptr(b), ptr(out)), c, "fork backward");
        return {out, Tensor()};
    }
};

// Residual join y = a + b (block/details/blocks/residual.hpp:131).
struct AddFn : torch::autograd::Function<AddFn> {
    static Tensor forward(AutogradContext*, Tensor a, Tensor b) {
        a = contig(a); b = contig(b);
        Tensor y = torch::empty_like(a);
        nott_ctx c = bind(a);
        check(nott_add(c, dtype_of(a), a.numel(), ptr(a), ptr(b), ptr(y)), c, "add forward");
        return y;
    }
    static variable_list backward(AutogradContext*, variable_list grads) { return {grads[0], grads[0]}; }
};

// -------------------------------------------------- softmax cross-entropy
// Mean reduction, ignore_index -100, label smoothing (loss/details/ce.hpp:21-37).
// One fused pass computes the loss and dlogits; backward scales dlogits by
// the upstream gradient of the scalar loss.
struct CrossEntropyFn : torch::autograd::Function<CrossEntropyFn> {
    static Tensor forward(AutogradContext* ctx, Tensor logits, Tensor labels, double smoothing) {
        logits = contig(logits);
        labels = contig(labels);
        Tensor dl = torch::empty_like(logits);
        Tensor loss = torch::empty({}, logits.options().dtype(torch::kFloat32));
        nott_ctx c = bind(logits);
        check(nott_softmax_xent_bwd(c, dtype_of(logits), logits.size(0), logits.size(1), ptr(logits),
                                    labels.data_ptr<int64_t>(), smoothing, 1.0, ptr(dl), fptr(loss)),
              c, "cross-entropy");
        ctx->save_for_backward({dl});
        return loss;
    }
    static variable_list backward(AutogradContext* ctx, variable_list grads) {
        Tensor dl = ctx->get_saved_variables()[0];
        Tensor g = grads[0].to(torch::kFloat32).contiguous();
        Tensor out = torch::empty_like(dl);
        nott_ctx c = bind(dl);
        check(nott_scale(c, dtype_of(dl), dl.numel(), ptr(dl), g.data_ptr<float>(), ptr(out)), c, "cross-entropy bwd");
        return {out, Tensor(), Tensor()};
    }
};

// ============================================================== modules
// Options mirror the reference's descriptors (conv.hpp:39-49, fc.hpp:19-30,
// pooling.hpp:41-57, batchnorm.hpp:22-36).  Parameters are fp32 masters; in
// mixed precision (compute_dtype bf16) each weight also has a bf16 working
// copy that the optimizer refreshes after every step.
// Mirrors Nott::Layer::Conv2dOptions (conv.hpp:39-49; bias defaults to true).
struct Conv2dOptions {
    int64_t in_channels = 1, out_channels = 1;
    std::array<int64_t, 2> kernel_size{3, 3}, stride{1, 1}, padding{0, 0}, dilation{1, 1};
    bool bias = true;
};

class Conv2dImpl : public torch::nn::Module {
public:
    explicit Conv2dImpl(const Conv2dOptions& o)
        : geom_{o.stride[0], o.stride[1], o.padding[0], o.padding[1], o.dilation[0], o.dilation[1]} {
        weight = register_parameter(
            "weight", torch::empty({o.out_channels, o.in_channels, o.kernel_size[0], o.kernel_size[1]}));
        if (o.bias) this->bias = register_parameter("bias", torch::zeros({o.out_channels}));
    }
    Tensor forward(const Tensor& x) {
        const Tensor& wc = weight_compute.defined() ? weight_compute : weight;
        return Conv2dFn::apply(x, weight, wc, or_absent(bias, weight), geom_);
    }
    // relu(forward(x)) with the activation fused into the convolution.
    // consumer_masks: the result's only consumer is a MaxPool2d taking it
    // with forward_relu_input, which applies the ReLU's backward.
    Tensor forward_relu(const Tensor& x, bool consumer_masks = false) {
        const Tensor& wc = weight_compute.defined() ? weight_compute : weight;
        return Conv2dReluFn::apply(x, weight, wc, or_absent(bias, weight), geom_, consumer_masks);
    }
    // {stride_h, stride_w, pad_h, pad_w, dil_h, dil_w}
    const std::vector<int64_t>& geometry() const { return geom_; }
    Tensor weight, bias, weight_compute;
private:
    std::vector<int64_t> geom_;
};
TORCH_MODULE(Conv2d);

class LinearImpl : public torch::nn::Module {
public:
    LinearImpl(int64_t in, int64_t out, bool bias = true) {
        weight = register_parameter("weight", torch::empty({out, in}));
        if (bias) this->bias = register_parameter("bias", torch::zeros({out}));
    }
    Tensor forward(const Tensor& x) { return apply(x, 0); }
    // relu(forward(x)) with the activation in the GEMM's epilogue;
    // consumer_masks: the result's only consumer is a Linear taking it with
    // forward_relu_input, which applies the ReLU's backward.
    Tensor forward_relu(const Tensor& x, bool consumer_masks = false) {
        return apply(x, kLinRelu | (consumer_masks ? kLinConsumerMasks : 0));
    }
    // x = the output of Linear::forward_relu(·, true): this layer's dx takes
    // that ReLU's backward.
    Tensor forward_relu_input(const Tensor& x) { return apply(x, kLinReluInput); }
    Tensor weight, bias, weight_compute;
private:
    Tensor apply(const Tensor& x, int64_t flags) {
        const Tensor& wc = weight_compute.defined() ? weight_compute : weight;
        return LinearFn::apply(x, weight, wc, or_absent(bias, weight), flags);
    }
};
TORCH_MODULE(Linear);

class BatchNorm2dImpl : public torch::nn::Module {
public:
    explicit BatchNorm2dImpl(int64_t c, double eps = 1e-5, double momentum = 0.1) : eps_(eps), momentum_(momentum) {
        weight = register_parameter("weight", torch::ones({c}));
        bias = register_parameter("bias", torch::zeros({c}));
        running_mean = register_buffer("running_mean", torch::zeros({c}));
        running_var = register_buffer("running_var", torch::ones({c}));
        // torch::nn::BatchNorm2d's third buffer, kept for the checkpoint
        // layout.  With a fixed momentum it only counts training forwards;
        // the count is kept on the host (count_batch) and written into the
        // buffer by sync_counter() before a save.
        num_batches_tracked = register_buffer("num_batches_tracked", torch::zeros({}, torch::kLong));
    }
    Tensor forward(const Tensor& x) {
        if (!is_training()) throw std::invalid_argument("Nott::HIP::BatchNorm2d: only training mode runs on HIP");
        ++batches_;
        return BatchNorm2dFn::apply(x, weight, bias, running_mean, running_var, eps_, momentum_);
    }
    // relu(BN(x)): the layer with its ReLU activation, fused.
    Tensor forward_relu(const Tensor& x) {
        if (!is_training()) throw std::invalid_argument("Nott::HIP::BatchNorm2d: only training mode runs on HIP");
        ++batches_;
        return BatchNorm2dReluFn::apply(x, weight, bias, running_mean, running_var, eps_, momentum_);
    }
    // maxpool(relu(BN(x))) with the pool geometry of a MaxPool2d
    // (MaxPool2dImpl::geometry()): the BatchNorm's output is never stored.
    Tensor forward_relu_maxpool(const Tensor& x, const std::vector<int64_t>& pool_geom) {
        if (!is_training()) throw std::invalid_argument("Nott::HIP::BatchNorm2d: only training mode runs on HIP");
        if (pool_geom[0] * pool_geom[1] > 256) return MaxPool2dFn::apply(forward_relu(x), pool_geom, false);
        ++batches_;
        return BatchNorm2dReluMaxPool2dFn::apply(x, weight, bias, running_mean, running_var, eps_, momentum_,
                                                 pool_geom);
    }
    // relu(BN(x) + skip): the residual branch's last layer, skip addition and
    // final ReLU, fused.
    // consumer_masks: the result's only consumer is a ResidualBasicBlock
    // taking it with relu_input, whose fork applies the ReLU's backward.
    Tensor forward_add_relu(const Tensor& x, const Tensor& skip, bool consumer_masks = false) {
        if (!is_training()) throw std::invalid_argument("Nott::HIP::BatchNorm2d: only training mode runs on HIP");
        ++batches_;
        return BatchNorm2dAddReluFn::apply(x, skip, weight, bias, running_mean, running_var, eps_, momentum_,
                                           consumer_masks);
    }
    // A forward replayed from a captured graph (no host code ran), or one
    // recorded during capture / undone by a warm-up (not run as a step).
    void count_batch() { ++batches_; }
    void uncount(int64_t n) { batches_ -= n; }
    void sync_counter() {
        torch::NoGradGuard ng;
        num_batches_tracked.fill_(batches_);
    }
    // After the buffer was loaded from a checkpoint: continue counting from it.
    void reload_counter() { batches_ = num_batches_tracked.item<int64_t>(); }
    Tensor weight, bias, running_mean, running_var, num_batches_tracked;
private:
    double eps_, momentum_;
    int64_t batches_ = 0;
};
TORCH_MODULE(BatchNorm2d);

inline Tensor relu(const Tensor& x) { return ReluFn::apply(x); }

// Writes `m` in the archive layout torch::nn::Module::save produces (its own
// parameters, then buffers, then one child archive per submodule), with every
// tensor copied to the host first, so a CPU model built from the reference's
// descriptors loads it directly.  Nott's Model::save writes the same archive
// as parameters.binary (src/core.hpp:2131-2135) and Model::load reads it back
// by the registration keys (`conv2d_0.weight`, `fc_5.bias`, ...,
// src/core.hpp:2188-2236).
inline void save_module_host(const torch::nn::Module& m, torch::serialize::OutputArchive& ar) {
    for (const auto& p : m.named_parameters(/*recurse=*/false)) ar.write(p.key(), p.value().detach().cpu());
    for (const auto& b : m.named_buffers(/*recurse=*/false))
        if (b.value().defined()) ar.write(b.key(), b.value().detach().cpu(), /*is_buffer=*/true);
    for (const auto& c : m.named_children()) {
        torch::serialize::OutputArchive child(ar.compilation_unit());
        save_module_host(*c.value(), child);
        ar.write(c.key(), child);
    }
}
inline void save_parameters(torch::nn::Module& m, const std::string& path) {
    for (auto& child : m.modules(/*include_self=*/true))
        if (auto* bn = child->as<BatchNorm2dImpl>()) bn->sync_counter();
    torch::serialize::OutputArchive ar;
    save_module_host(m, ar);
    ar.save_to(path);
}

inline Tensor max_pool2d(const Tensor& x, int64_t k, int64_t stride, int64_t pad = 0, bool ceil_mode = false) {
    return MaxPool2dFn::apply(x, std::vector<int64_t>{k, k, stride, stride, pad, pad, 1, 1, ceil_mode ? 1 : 0}, false);
}

// Parameter-less layers as modules, so that a model registers every layer of
// its descriptor list under Nott's `<kind>_<index>` key (pooling.hpp:132-149,
// flatten.hpp:19-41) and its checkpoint archive has the same child entries.
class MaxPool2dImpl : public torch::nn::Module {
public:
    // Square window, stride and padding, no dilation.
    MaxPool2dImpl(int64_t k, int64_t stride, int64_t pad = 0, bool ceil_mode = false)
        : geom_{k, k, stride, stride, pad, pad, 1, 1, ceil_mode ? 1 : 0} {}
    // Per-axis window, stride, padding and dilation (torch::nn::MaxPool2dOptions).
    MaxPool2dImpl(std::array<int64_t, 2> k, std::array<int64_t, 2> stride, std::array<int64_t, 2> pad,
                  std::array<int64_t, 2> dilation, bool ceil_mode)
        : geom_{k[0], k[1], stride[0], stride[1], pad[0], pad[1], dilation[0], dilation[1], ceil_mode ? 1 : 0} {}
    Tensor forward(const Tensor& x) { return MaxPool2dFn::apply(x, geom_, false); }
    // x = the output of Conv2d::forward_relu(·, true): the ReLU's backward is
    // applied here, in the pool's backward pass (one pass instead of two).
    Tensor forward_relu_input(const Tensor& x) { return MaxPool2dFn::apply(x, geom_, true); }
    // {kh, kw, stride_h, stride_w, pad_h, pad_w, dil_h, dil_w, ceil_mode}
    const std::vector<int64_t>& geometry() const { return geom_; }
private:
    std::vector<int64_t> geom_;
};
TORCH_MODULE(MaxPool2d);
class FlattenImpl : public torch::nn::Module {
public:
    // Nott's Flatten wraps a torch::nn::Flatten registered as "flatten"
    // (flatten.hpp:34): an empty child entry in the archive.  The result is a
    // view (x.flatten(start_dim, end_dim), as torch::nn::Flatten computes it).
    explicit FlattenImpl(int64_t start_dim = 1, int64_t end_dim = -1) : start_(start_dim), end_(end_dim) {
        register_module("flatten", std::make_shared<torch::nn::Module>());
    }
    Tensor forward(const Tensor& x) { return x.flatten(start_, end_); }
private:
    int64_t start_, end_;
};
TORCH_MODULE(Flatten);
// AdaptiveAvgPool2d({1, 1}) (pooling.hpp:164-167): no parameters or buffers.
class AdaptiveAvgPool2dImpl : public torch::nn::Module {
public:
    Tensor forward(const Tensor& x) { return AvgPoolGlobalFn::apply(x); }
};
TORCH_MODULE(AdaptiveAvgPool2d);

// The residual block Nott builds from
//   Block::Residual({Conv2d(in→out, 3×3, stride s, pad 1, no bias),
//                    BatchNorm2d(out) + ReLU, Conv2d(out→out, 3×3, pad 1, no bias),
//                    BatchNorm2d(out)},
//                   1, {projection: Conv2d(in→out, 1×1, stride s, no bias)},
//                   {final_activation: ReLU})
// (block/details/blocks/residual.hpp:37-141): the layers registered as
// conv2d_0, batchnorm2d_1, conv2d_2, batchnorm2d_3 and the projection as
// conv2d_4 (residual.hpp:49-62), so checkpoint keys match the reference's.
// forward = relu(bn3(conv2(relu(bn1(conv0(x))))) + skip(x)) with skip the
// projection or the identity (residual.hpp:87-132); the layer ReLU and the
// skip addition + final ReLU run fused into the BatchNorm apply passes.
class ResidualBasicBlockImpl : public torch::nn::Module {
public:
    ResidualBasicBlockImpl(int64_t in, int64_t out, int64_t stride, bool projection) {
        conv0 = register_module("conv2d_0", Conv2d(Conv2dOptions{in, out, {3, 3}, {stride, stride}, {1, 1}, {1, 1}, false}));
        bn1 = register_module("batchnorm2d_1", BatchNorm2d(out));
        conv2 = register_module("conv2d_2", Conv2d(Conv2dOptions{out, out, {3, 3}, {1, 1}, {1, 1}, {1, 1}, false}));
        bn3 = register_module("batchnorm2d_3", BatchNorm2d(out));
        if (projection)
            proj = register_module("conv2d_4", Conv2d(Conv2dOptions{in, out, {1, 1}, {stride, stride}, {0, 0}, {1, 1}, false}));
    }
    // relu_input: x is the output of the previous block run with
    // consumer_masks (its final ReLU's backward then runs in this block's
    // fork); consumer_masks: the output's only consumer is the next block,
    // run with relu_input.
    Tensor forward(const Tensor& x, bool relu_input = false, bool consumer_masks = false) {
        auto f = ForkFn::apply(x, relu_input);   // x feeds the branch and the skip
        Tensor h = bn1->forward_relu(conv0(f[0]));
        Tensor skip = proj ? proj(f[1]) : f[1];
        return bn3->forward_add_relu(conv2(h), skip, consumer_masks);
    }
    Conv2d conv0{nullptr}, conv2{nullptr}, proj{nullptr};
    BatchNorm2d bn1{nullptr}, bn3{nullptr};
};
TORCH_MODULE(ResidualBasicBlock);

inline Tensor cross_entropy(const Tensor& logits, const Tensor& labels, double label_smoothing = 0.0) {
    return CrossEntropyFn::apply(logits, labels, label_smoothing);
}

// Kaiming-uniform (HeUniform: torch::nn::init::kaiming_uniform_(w, a = 0,
// fan_in, relu), reference initialization/apply.hpp:45-51) drawn from a
// torch CPU generator given by the caller.  The bound is formed as libtorch
// forms it, sqrt(3) · (gain / sqrt(fan_in)) with gain sqrt(2), which is not
// always the same double as sqrt(6 / fan_in); the draws are then identical.
inline void he_uniform_(Tensor& w, torch::Generator& gen) {
    torch::NoGradGuard ng;
    const int64_t fan_in = w.numel() / w.size(0);
    const double std_ = std::sqrt(2.0) / std::sqrt((double)fan_in);
    const double bound = std::sqrt(3.0) * std_;
    Tensor cpu = torch::empty(w.sizes(), torch::kFloat32).uniform_(-bound, bound, gen);
    w.copy_(cpu);
}

// Draws the initial weights of a model built from Nott descriptors with
// HeUniform initialisation exactly as the reference draws them from a
// generator seeded with the same value: for every Conv2d and Linear in
// registration order (pre-order over the module tree, the order Nott's
// layer factories run), the torch::nn module's constructor first draws its
// default initialisation (weight, then bias: one uniform draw per element;
// conv.hpp:182 / fc.hpp:38 construct torch::nn::Conv2d / Linear), then
// apply_module_initialization redraws the weight with HeUniform and zeroes
// the bias (initialization/apply.hpp:10-17, 45-51).  The default draws'
// values are overwritten, but they advance the generator, so they are made
// with the same shapes and dtype.  BatchNorm2d draws nothing (ones / zeros).
inline void reference_init_(torch::nn::Module& model, torch::Generator& gen) {
    torch::NoGradGuard ng;
    auto layer = [&](Tensor& w, Tensor& b) {
        Tensor scratch = torch::empty(w.sizes(), torch::kFloat32);
        scratch.uniform_(0.0, 1.0, gen);
        if (b.defined()) torch::empty(b.sizes(), torch::kFloat32).uniform_(0.0, 1.0, gen);
        he_uniform_(w, gen);
        if (b.defined()) b.zero_();
    };
    for (auto& child : model.modules(/*include_self=*/true)) {
        if (auto* c = child->as<Conv2dImpl>()) layer(c->weight, c->bias);
        else if (auto* l = child->as<LinearImpl>()) layer(l->weight, l->bias);
    }
}

// ============================================================ optimizer
// Fused Adam / AdamW behind libtorch's optimizer interface: a drop-in for
// Nott::Optimizer::Details::Adam / AdamW (reference optimizer/details/adam.hpp:
// 63-154, 159-250), which Model::set_optimizer holds as a
// std::unique_ptr<torch::optim::Optimizer> (core.hpp:170-181, 1364-1381) and
// Model::step_optimizers steps through the virtual step() (core.hpp:
// 5049-5057).  Same constructors (parameters or parameter groups, the torch
// options, warm-up buckets), same param_groups() whose options() a scheduler
// rewrites with set_lr (lrscheduler/details/cosineannealing.hpp:52-63), and a
// state() with one AdamParamState / AdamWParamState per parameter.
//
// Layout: at construction every parameter and its gradient are moved into
// flat fp32 arenas (P, G, M, V), one contiguous range per param group with
// 256-byte aligned segments.  A parameter keeps its identity (set_data onto
// its arena slice); its .grad() and its state's exp_avg / exp_avg_sq are
// tensors over the arenas' storage, so step() is one nott_adam_step launch
// per group, reading the group's options at call time.  libtorch's own
// Optimizer::zero_grad(false) (what Nott's Model::zero_grad calls, core.hpp:
// 2425-2442) zeroes the arena slices in place; after zero_grad(true) the
// host modules re-attach each parameter's arena slice when a backward next
// writes it (grad_buffer).
//
// set_fused_zero_grad(true) makes step() also clear the gradients in the same
// pass, for callers that always follow step() with zero_grad() as
// Model::run_training_step does (core.hpp:3819-3823).
//
// Mixed precision: bf16 working copies of chosen weights live in a flat bf16
// arena aligned like the masters and are refreshed with one nott_cast after
// each step.  amsgrad is not supported (std::invalid_argument), nor is
// serialising the optimizer state (Nott's checkpoint stores parameters only).
template <bool Decoupled>
class FusedAdamImpl : public torch::optim::Optimizer {
public:
    using TorchOptions = std::conditional_t<Decoupled, torch::optim::AdamWOptions, torch::optim::AdamOptions>;
    using ParamState = std::conditional_t<Decoupled, torch::optim::AdamWParamState, torch::optim::AdamParamState>;

    FusedAdamImpl(std::vector<Tensor> params, const TorchOptions& options,
                  std::vector<std::vector<Tensor>> warmup_buckets = {})
        : torch::optim::Optimizer(std::move(params), std::make_unique<TorchOptions>(options)) {
        (void)warmup_buckets;   // state is created eagerly; the buckets only order warm-up in the reference
        build();
    }
    FusedAdamImpl(const std::vector<torch::optim::OptimizerParamGroup>& groups, const TorchOptions& options,
                  std::vector<std::vector<Tensor>> warmup_buckets = {})
        : torch::optim::Optimizer(groups, std::make_unique<TorchOptions>(options)) {
        (void)warmup_buckets;
        build();
    }
    ~FusedAdamImpl() override {
        if (replayed_) (void)hipEventDestroy(replayed_);
        std::lock_guard<std::mutex> g(detail::arena_mutex());
        for (auto* impl : registered_) detail::arena_grads().erase(impl);
    }

    // Updates every parameter whose gradient is defined, as
    // torch::optim::Adam[W]::step does (a parameter whose .grad() is none is
    // skipped and keeps its step count).  Consecutive parameters with a
    // gradient and the same step count form one segment of the arena, and
    // each segment is one nott_adam_step launch with its group's options at
    // call time: one launch per group in the usual case.  A gradient tensor
    // assigned from outside is copied into the arena first.
    Tensor step(LossClosure closure = nullptr) override {
        Tensor loss;
        if (closure) {
            torch::AutoGradMode enable(true);
            loss = closure();
        }
        if (param_groups_.size() != group_count_)
            throw std::logic_error("FusedAdam: parameter groups were added after construction");
        if (!P_.defined()) return loss;
        torch::NoGradGuard ng;
        nott_ctx c = bind(P_);
        struct Seg { int64_t off, end, step; };
        for (auto& group : param_groups_) {
            const auto& o = static_cast<const TorchOptions&>(group.options());
            std::vector<Seg> segs;
            for (auto& p : group.params()) {
                auto it = offsets_.find(p.unsafeGetTensorImpl());
                if (it == offsets_.end()) continue;   // does not require grad
                const int64_t off = it->second, len = (p.numel() + 63) / 64 * 64;
                Tensor gv = p.grad();
                if (!gv.defined()) continue;
                float* slot = G_.data_ptr<float>() + off;
                if (gv.data_ptr() != (void*)slot) {
                    Tensor a = detail::alias(G_, off, p.sizes());
                    a.copy_(gv);
                    p.mutable_grad() = a;
                }
                auto& st = static_cast<ParamState&>(*state_.at(p.unsafeGetTensorImpl()));
                const int64_t t = st.step() + 1;
                st.step(t);
                device_steps_stale_ = true;
                if (!segs.empty() && segs.back().end == off && segs.back().step == t) segs.back().end = off + len;
                else segs.push_back({off, off + len, t});
            }
            for (const auto& sg : segs)
                check(nott_adam_step(c, Decoupled ? 1 : 0, sg.end - sg.off, P_.data_ptr<float>() + sg.off, NOTT_F32,
                                     G_.data_ptr<float>() + sg.off, NOTT_F32, M_.data_ptr<float>() + sg.off,
                                     V_.data_ptr<float>() + sg.off, o.lr(), std::get<0>(o.betas()),
                                     std::get<1>(o.betas()), o.eps(), o.weight_decay(), sg.step, fuse_zero_ ? 1 : 0),
                      c, "adam step");
        }
        if (Pb_.defined()) refresh();
        return loss;
    }

    // The reference's warm-up hook (adam.hpp:98-150, called through
    // OptimizerBinding::warmup): the state already exists, nothing to do.
    void ensure_state_initialized() {}

    // ---- Graph mode: the optimizer step inside a captured HIP graph
    // (OptimizerBinding::capture_safe, core.hpp:170-181, 3829-3945).
    // graph_prepare() runs before capture: each group gets a device state
    // (nott_adam_device_state: its step count and the launch's scalar
    // block) and a pinned block of hyper-parameters the device reads at
    // launch time.  graph_step() is called while capturing and records one
    // nott_adam_step_graph launch per group (and the bf16 refresh).  Before
    // every replay graph_sync() writes the groups' current options (a
    // scheduler's set_lr included) into the pinned blocks and, if an eager
    // step() ran since, the host step count into the device state; after
    // it, graph_after_replay() advances the per-parameter step counts the
    // device advanced and records an event behind the replay.  A replay
    // still queued reads the pinned block only when its optimizer node runs,
    // so graph_sync() waits for that event before it changes a value (and
    // only then: with unchanged options, replays queue back to back).  Every
    // parameter of a group must have a gradient and the group's step counts
    // must be equal at capture.
    void graph_prepare() {
        if (!P_.defined()) return;
        torch::NoGradGuard ng;
        const int64_t ng_ = (int64_t)param_groups_.size();
        dev_state_ = torch::zeros({ng_, 8}, P_.options().dtype(torch::kInt64));
        hparams_ = torch::empty({ng_, 5}, torch::TensorOptions().dtype(torch::kFloat64)).pin_memory();
        ranges_.assign(param_groups_.size(), {0, 0});
        wd_nonzero_.assign(param_groups_.size(), 0);
        for (size_t gi = 0; gi < param_groups_.size(); ++gi) {
            int64_t lo = -1, hi = -1, t = -1;
            for (auto& p : param_groups_[gi].params()) {
                auto it = offsets_.find(p.unsafeGetTensorImpl());
                if (it == offsets_.end()) continue;
                if (!p.grad().defined() || p.grad().data_ptr() != (void*)(G_.data_ptr<float>() + it->second))
                    throw std::logic_error("FusedAdam graph mode: every parameter needs its arena gradient");
                const int64_t st = static_cast<ParamState&>(*state_.at(p.unsafeGetTensorImpl())).step();
                if (t >= 0 && st != t) throw std::logic_error("FusedAdam graph mode: unequal step counts in a group");
                t = st;
                const int64_t off = it->second, end = off + (p.numel() + 63) / 64 * 64;
                lo = lo < 0 ? off : std::min(lo, off);
                hi = std::max(hi, end);
            }
            if (lo >= 0) ranges_[gi] = {lo, hi};
            const auto& o = static_cast<const TorchOptions&>(param_groups_[gi].options());
            wd_nonzero_[gi] = o.weight_decay() != 0.0;
        }
        device_steps_stale_ = true;
        if (!replayed_ && hipEventCreateWithFlags(&replayed_, hipEventDisableTiming) != hipSuccess)
            throw std::runtime_error("FusedAdam graph mode: hipEventCreate failed");
        replay_pending_ = false;
        graph_sync();
    }
    void graph_step() {
        if (!P_.defined()) return;
        nott_ctx c = bind(P_);
        auto* st = reinterpret_cast<nott_adam_device_state*>(dev_state_.data_ptr<int64_t>());
        const double* hp = hparams_.data_ptr<double>();
        for (size_t gi = 0; gi < ranges_.size(); ++gi) {
            const int64_t lo = ranges_[gi].first, hi = ranges_[gi].second;
            if (hi <= lo) continue;
            check(nott_adam_step_graph(c, Decoupled ? 1 : 0, hi - lo, P_.data_ptr<float>() + lo, NOTT_F32,
                                       G_.data_ptr<float>() + lo, NOTT_F32, M_.data_ptr<float>() + lo,
                                       V_.data_ptr<float>() + lo, hp + 5 * gi, st + gi, wd_nonzero_[gi],
                                       fuse_zero_ ? 1 : 0),
                  c, "adam step (graph)");
        }
        if (Pb_.defined()) refresh();
    }
    void graph_sync() {
        if (!hparams_.defined()) return;
        double* hp = hparams_.data_ptr<double>();
        std::vector<double> want(5 * param_groups_.size());
        for (size_t gi = 0; gi < param_groups_.size(); ++gi) {
            const auto& o = static_cast<const TorchOptions&>(param_groups_[gi].options());
            if ((o.weight_decay() != 0.0) != (wd_nonzero_[gi] != 0))
                throw std::logic_error("FusedAdam graph mode: weight decay switched on or off after capture");
            want[5 * gi + 0] = o.lr();
            want[5 * gi + 1] = std::get<0>(o.betas());
            want[5 * gi + 2] = std::get<1>(o.betas());
            want[5 * gi + 3] = o.eps();
            want[5 * gi + 4] = o.weight_decay();
        }
        if (std::memcmp(want.data(), hp, want.size() * sizeof(double)) != 0) {
            if (replay_pending_) {
                detail::hip_ok(hipEventSynchronize(replayed_), "FusedAdam graph mode: wait for the last replay");
                replay_pending_ = false;
            }
            std::memcpy(hp, want.data(), want.size() * sizeof(double));
        }
        if (device_steps_stale_) {
            Tensor host = torch::zeros({(int64_t)param_groups_.size(), 8}, torch::kInt64);
            for (size_t gi = 0; gi < param_groups_.size(); ++gi)
                for (auto& p : param_groups_[gi].params()) {
                    auto it = state_.find(p.unsafeGetTensorImpl());
                    if (it != state_.end()) host[gi][0] = static_cast<ParamState&>(*it->second).step();
                }
            dev_state_.copy_(host);
            device_steps_stale_ = false;
        }
    }
    void graph_after_replay() {
        if (replayed_) {
            const auto stream = c10::hip::getCurrentHIPStream(P_.device().index());
            detail::hip_ok(hipEventRecord(replayed_, stream.stream()), "FusedAdam graph mode: record the replay");
            replay_pending_ = true;
        }
        for (size_t gi = 0; gi < ranges_.size(); ++gi) {
            if (ranges_[gi].second <= ranges_[gi].first) continue;
            for (auto& p : param_groups_[gi].params()) {
                auto it = state_.find(p.unsafeGetTensorImpl());
                if (it == state_.end()) continue;
                auto& st = static_cast<ParamState&>(*it->second);
                st.step(st.step() + 1);
            }
        }
    }

    void set_fused_zero_grad(bool on) { fuse_zero_ = on; }

    // Clears every gradient with one kernel (what Optimizer::zero_grad(false)
    // does with one fill per parameter).
    void zero_flat_grads() {
        if (!G_.defined()) return;
        nott_ctx c = bind(G_);
        check(nott_zero(c, G_.numel() * 4, G_.data_ptr()), c, "zero_grad");
    }

    // bf16 working copies: *copies[j] becomes a bf16 view of masters[j]'s
    // values, refreshed after every step (and by refresh()).
    void attach_bf16_copies(const std::vector<Tensor*>& copies, const std::vector<Tensor>& masters) {
        if (copies.size() != masters.size()) throw std::invalid_argument("FusedAdam: copy/master mismatch");
        if (copies.empty()) return;
        torch::NoGradGuard ng;
        Pb_ = torch::zeros({P_.numel()}, P_.options().dtype(torch::kBFloat16));
        for (size_t j = 0; j < masters.size(); ++j) {
            auto it = offsets_.find(masters[j].unsafeGetTensorImpl());
            if (it == offsets_.end()) throw std::invalid_argument("FusedAdam: bf16 master not among params");
            *copies[j] = detail::alias(Pb_, it->second, masters[j].sizes());
        }
        refresh();
    }
    // Re-casts the bf16 working copies (after parameters were overwritten).
    void refresh() {
        if (!Pb_.defined()) return;
        nott_ctx c = bind(P_);
        check(nott_cast(c, P_.numel(), P_.data_ptr(), NOTT_F32, Pb_.data_ptr(), NOTT_BF16), c, "bf16 copy");
    }
    // Step count of a parameter's state (0 before its first update).
    int64_t step_count(const Tensor& p) const {
        auto it = state_.find(p.unsafeGetTensorImpl());
        return it == state_.end() ? 0 : static_cast<const ParamState&>(*it->second).step();
    }
    const Tensor& flat_params() const { return P_; }
    const Tensor& flat_grads() const { return G_; }

    void save(torch::serialize::OutputArchive&) const override {
        throw std::logic_error("FusedAdam: optimizer state serialisation is not supported");
    }
    void load(torch::serialize::InputArchive&) override {
        throw std::logic_error("FusedAdam: optimizer state serialisation is not supported");
    }

private:
    void build() {
        torch::NoGradGuard ng;
        int64_t total = 0;
        c10::optional<torch::Device> dev;
        std::vector<std::vector<int64_t>> offs(param_groups_.size());
        for (size_t gi = 0; gi < param_groups_.size(); ++gi) {
            const auto& o = static_cast<const TorchOptions&>(param_groups_[gi].options());
            if (o.amsgrad()) throw std::invalid_argument("FusedAdam: amsgrad is not supported");
            for (const auto& p : param_groups_[gi].params()) {
                offs[gi].push_back(-1);
                if (!p.defined() || !p.requires_grad()) continue;
                if (p.scalar_type() != torch::kFloat32) throw std::invalid_argument("FusedAdam: parameters must be float32");
                if (!p.is_cuda()) throw std::invalid_argument("FusedAdam: parameters must live on a HIP device");
                if (dev && *dev != p.device()) throw std::invalid_argument("FusedAdam: parameters on several devices");
                dev = p.device();
                offs[gi].back() = total;
                total += (p.numel() + 63) / 64 * 64;   // 256-byte aligned segments
            }
        }
        group_count_ = param_groups_.size();
        if (total == 0) return;
        auto fo = torch::TensorOptions().dtype(torch::kFloat32).device(*dev);
        P_ = torch::zeros({total}, fo);
        G_ = torch::zeros({total}, fo);
        M_ = torch::zeros({total}, fo);
        V_ = torch::zeros({total}, fo);
        std::lock_guard<std::mutex> g(detail::arena_mutex());
        for (size_t gi = 0; gi < param_groups_.size(); ++gi) {
            auto& params = param_groups_[gi].params();
            for (size_t k = 0; k < params.size(); ++k) {
                const int64_t off = offs[gi][k];
                if (off < 0) continue;
                auto& p = params[k];
                Tensor pv = detail::alias(P_, off, p.sizes());
                pv.copy_(p.detach());
                p.set_data(pv);
                // A gradient that exists moves into the arena; one that does
                // not is attached (zeroed) by the first backward that writes it.
                Tensor gv = detail::alias(G_, off, p.sizes());
                if (p.grad().defined()) {
                    gv.copy_(p.grad());
                    p.mutable_grad() = gv;
                }
                auto st = std::make_unique<ParamState>();
                st->step(0);
                st->exp_avg(detail::alias(M_, off, p.sizes()));
                st->exp_avg_sq(detail::alias(V_, off, p.sizes()));
                state_[p.unsafeGetTensorImpl()] = std::move(st);
                detail::arena_grads()[p.unsafeGetTensorImpl()] = gv;
                registered_.push_back(p.unsafeGetTensorImpl());
                offsets_[p.unsafeGetTensorImpl()] = off;
            }
        }
    }

    size_t group_count_ = 0;
    // graph mode: per-group device state, pinned hyper-parameters, arena ranges
    Tensor dev_state_, hparams_;
    hipEvent_t replayed_ = nullptr;   // recorded behind the last replay
    bool replay_pending_ = false;
    std::vector<std::pair<int64_t, int64_t>> ranges_;
    std::vector<int> wd_nonzero_;
    bool device_steps_stale_ = true;
    std::vector<const c10::TensorImpl*> registered_;
    std::unordered_map<const c10::TensorImpl*, int64_t> offsets_;
    Tensor P_, G_, M_, V_, Pb_;
    bool fuse_zero_ = false;
};
using FusedAdam = FusedAdamImpl<false>;    // Nott::Optimizer::Details::Adam
using FusedAdamW = FusedAdamImpl<true>;    // Nott::Optimizer::Details::AdamW

}  // namespace HIP
}  // namespace Nott
