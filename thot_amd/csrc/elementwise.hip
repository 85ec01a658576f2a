// Bandwidth-bound elementwise kernels: ReLU forward/backward, residual add,
// casts, zero fill and global average pool forward/backward.
//
// ReLU backward replaces libtorch's threshold_backward for the ReLU that
// Nott applies after every layer (reference activation/apply.hpp:24-57,
// activation/details/relu.hpp:13): dx = (y <= 0) ? 0 : dy.
// Global average pool replaces AdaptiveAvgPool2d({1,1}) (layer/details/pooling.hpp:164-167).
#include "common.hpp"

namespace {

constexpr int kThreads = 256;

struct ReluFwd {
    __device__ __forceinline__ float operator()(float x) const { return (x > 0.f || x != x) ? x : 0.f; }
};

// dx = (y <= 0) ? 0 : dy; a NaN y passes dy through (threshold_backward semantics).
struct ReluBwd {
    __device__ __forceinline__ float operator()(float y, float dy) const { return (y <= 0.f) ? 0.f : dy; }
};

struct Add {
    __device__ __forceinline__ float operator()(float a, float b) const { return a + b; }
};

template <typename T, typename F>
__global__ __launch_bounds__(kThreads) void unary_vec(const T* __restrict__ x, T* __restrict__ y, int64_t n, F f) {
    const int64_t i = ((int64_t)blockIdx.x * kThreads + threadIdx.x) * 4;
    if (i + 4 <= n) {
        f32x4 a = Vec4<T>::ld(x + i);
        a.x = f(a.x); a.y = f(a.y); a.z = f(a.z); a.w = f(a.w);
        Vec4<T>::st(y + i, a);
    } else {
        for (int64_t j = i; j < n; ++j) Io<T>::st(y, j, f(Io<T>::ld(x, j)));
    }
}

template <typename T, typename F>
__global__ __launch_bounds__(kThreads) void binary_vec(const T* __restrict__ a, const T* __restrict__ b,
                                                       T* __restrict__ y, int64_t n, F f) {
    const int64_t i = ((int64_t)blockIdx.x * kThreads + threadIdx.x) * 4;
    if (i + 4 <= n) {
        f32x4 u = Vec4<T>::ld(a + i), v = Vec4<T>::ld(b + i);
        u.x = f(u.x, v.x); u.y = f(u.y, v.y); u.z = f(u.z, v.z); u.w = f(u.w, v.w);
        Vec4<T>::st(y + i, u);
    } else {
        for (int64_t j = i; j < n; ++j) Io<T>::st(y, j, f(Io<T>::ld(a, j), Io<T>::ld(b, j)));
    }
}

template <typename T, typename F>
__global__ __launch_bounds__(kThreads) void unary_scalar(const T* __restrict__ x, T* __restrict__ y, int64_t n, F f) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i < n) Io<T>::st(y, i, f(Io<T>::ld(x, i)));
}

template <typename T, typename F>
__global__ __launch_bounds__(kThreads) void binary_scalar(const T* __restrict__ a, const T* __restrict__ b,
                                                          T* __restrict__ y, int64_t n, F f) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i < n) Io<T>::st(y, i, f(Io<T>::ld(a, i), Io<T>::ld(b, i)));
}

template <typename T>
bool aligned4(const void* p) {
    return ((uintptr_t)p % (4 * sizeof(T))) == 0;
}

template <typename T, typename F>
int run_unary(nott_ctx ctx, int64_t n, const void* x, void* y, F f, const char* name) {
    if (n == 0) return NOTT_OK;
    if (aligned4<T>(x) && aligned4<T>(y)) {
        const int64_t blocks = nott::ceil_div(nott::ceil_div(n, 4), kThreads);
        hipLaunchKernelGGL((unary_vec<T, F>), dim3((unsigned)blocks), dim3(kThreads), 0, ctx->stream,
                           static_cast<const T*>(x), static_cast<T*>(y), n, f);
    } else {
        const int64_t blocks = nott::ceil_div(n, kThreads);
        hipLaunchKernelGGL((unary_scalar<T, F>), dim3((unsigned)blocks), dim3(kThreads), 0, ctx->stream,
                           static_cast<const T*>(x), static_cast<T*>(y), n, f);
    }
    return nott::launch_status(ctx, name);
}

template <typename T, typename F>
int run_binary(nott_ctx ctx, int64_t n, const void* a, const void* b, void* y, F f, const char* name) {
    if (n == 0) return NOTT_OK;
    if (aligned4<T>(a) && aligned4<T>(b) && aligned4<T>(y)) {
        const int64_t blocks = nott::ceil_div(nott::ceil_div(n, 4), kThreads);
        hipLaunchKernelGGL((binary_vec<T, F>), dim3((unsigned)blocks), dim3(kThreads), 0, ctx->stream,
                           static_cast<const T*>(a), static_cast<const T*>(b), static_cast<T*>(y), n, f);
    } else {
        const int64_t blocks = nott::ceil_div(n, kThreads);
        hipLaunchKernelGGL((binary_scalar<T, F>), dim3((unsigned)blocks), dim3(kThreads), 0, ctx->stream,
                           static_cast<const T*>(a), static_cast<const T*>(b), static_cast<T*>(y), n, f);
    }
    return nott::launch_status(ctx, name);
}

template <typename TS, typename TD>
__global__ __launch_bounds__(kThreads) void cast_kernel(const TS* __restrict__ s, TD* __restrict__ d, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i < n) Io<TD>::st(d, i, Io<TS>::ld(s, i));
}

// fp32 → bf16 over 8-element groups (two 16-byte loads, one 16-byte store per
// thread), rounded as the element kernel rounds; both buffers 16-byte aligned.
__global__ __launch_bounds__(kThreads) void cast_f32_bf16_vec_kernel(const float* __restrict__ s, bf16_t* __restrict__ d,
                                                                    int64_t ngroups) {
    const int64_t q = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (q >= ngroups) return;
    const f32x4 lo = *reinterpret_cast<const f32x4*>(s + 8 * q), hi = *reinterpret_cast<const f32x4*>(s + 8 * q + 4);
    *reinterpret_cast<u32x4*>(d + 8 * q) =
        u32x4{pack_bf16x2(lo.x, lo.y), pack_bf16x2(lo.z, lo.w), pack_bf16x2(hi.x, hi.y), pack_bf16x2(hi.z, hi.w)};
}

__global__ __launch_bounds__(kThreads) void zero_kernel(uint32_t* __restrict__ p, int64_t nwords,
                                                        uint8_t* __restrict__ tail, int64_t ntail) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i < nwords) p[i] = 0u;
    if (i < ntail) tail[i] = 0;
}

template <typename T>
__global__ __launch_bounds__(kThreads) void scale_kernel(const T* __restrict__ x, const float* __restrict__ scale,
                                                         T* __restrict__ y, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i < n) Io<T>::st(y, i, Io<T>::ld(x, i) * scale[0]);
}

// One wave per (n, c) plane: mean over hw.
template <typename T>
__global__ __launch_bounds__(kThreads) void avgpool_fwd_kernel(const T* __restrict__ x, T* __restrict__ y,
                                                               int64_t nc, int64_t hw) {
    const int64_t plane = (int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (plane >= nc) return;
    const T* xp = x + plane * hw;
    float acc = 0.f;
    for (int64_t i = lane; i < hw; i += 64) acc += Io<T>::ld(xp, i);
    acc = wave_sum(acc);
    if (lane == 0) Io<T>::st(y, plane, acc / (float)hw);
}

template <typename T>
__global__ __launch_bounds__(kThreads) void avgpool_bwd_kernel(const T* __restrict__ dy, T* __restrict__ dx,
                                                               int64_t nc, int64_t hw) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= nc * hw) return;
    Io<T>::st(dx, i, Io<T>::ld(dy, i / hw) / (float)hw);
}

// dz = (y <= 0) ? 0 : a + b over 16-byte groups (8 bf16 / 4 fp32), the
// sum rounded once as nott_add rounds it.
template <typename T>
__global__ __launch_bounds__(kThreads) void add_relu_bwd_kernel(const T* __restrict__ a, const T* __restrict__ b,
                                                                const T* __restrict__ y, T* __restrict__ dz,
                                                                int64_t n) {
    constexpr int V = 16 / (int)sizeof(T);
    const int64_t i = ((int64_t)blockIdx.x * kThreads + threadIdx.x) * V;
    if (i + V <= n) {
        if constexpr (sizeof(T) == 2) {
            const u32x4 ua = *reinterpret_cast<const u32x4*>(a + i), ub = *reinterpret_cast<const u32x4*>(b + i),
                        uy = *reinterpret_cast<const u32x4*>(y + i);
            u32x4 out;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                float r[2];
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const uint32_t sh = 16 * h;
                    const float fa = __builtin_bit_cast(float, ((ua[k] >> sh) & 0xffffu) << 16);
                    const float fb = __builtin_bit_cast(float, ((ub[k] >> sh) & 0xffffu) << 16);
                    const float fy = __builtin_bit_cast(float, ((uy[k] >> sh) & 0xffffu) << 16);
                    r[h] = (fy <= 0.f) ? 0.f : fa + fb;
                }
                out[k] = pack_bf16x2(r[0], r[1]);
            }
            *reinterpret_cast<u32x4*>(dz + i) = out;
        } else {
            // float vectors loaded as such (element bit-casts of an integer
            // vector are what the compiler has mistranslated)
            const f32x4 fa = *reinterpret_cast<const f32x4*>(a + i), fb = *reinterpret_cast<const f32x4*>(b + i),
                        fy = *reinterpret_cast<const f32x4*>(y + i);
            f32x4 out;
#pragma unroll
            for (int k = 0; k < 4; ++k) out[k] = (fy[k] <= 0.f) ? 0.f : fa[k] + fb[k];
            *reinterpret_cast<f32x4*>(dz + i) = out;
        }
    } else {
        for (int64_t j = i; j < n; ++j) {
            const float fy = Io<T>::ld(y, j);
            Io<T>::st(dz, j, (fy <= 0.f) ? 0.f : Io<T>::ld(a, j) + Io<T>::ld(b, j));
        }
    }
}

}  // namespace

extern "C" {

int nott_relu_fwd(nott_ctx ctx, nott_dtype dtype, int64_t n, const void* x, void* y) {
    NOTT_CHECK_CTX(ctx);
    NOTT_REQUIRE(ctx, nott::valid_dtype(dtype) && n >= 0, "nott_relu_fwd: bad dtype or size");
    NOTT_REQUIRE(ctx, n == 0 || (x && y), "nott_relu_fwd: null buffer");
    nott::DeviceScope scope(ctx->device);
    return dtype == NOTT_F32 ? run_unary<float>(ctx, n, x, y, ReluFwd{}, "relu_fwd")
                             : run_unary<bf16_t>(ctx, n, x, y, ReluFwd{}, "relu_fwd");
}

int nott_relu_bwd(nott_ctx ctx, nott_dtype dtype, int64_t n, const void* y, const void* dy, void* dx) {
    NOTT_CHECK_CTX(ctx);
    NOTT_REQUIRE(ctx, nott::valid_dtype(dtype) && n >= 0, "nott_relu_bwd: bad dtype or size");
    NOTT_REQUIRE(ctx, n == 0 || (y && dy && dx), "nott_relu_bwd: null buffer");
    nott::DeviceScope scope(ctx->device);
    return dtype == NOTT_F32 ? run_binary<float>(ctx, n, y, dy, dx, ReluBwd{}, "relu_bwd")
                             : run_binary<bf16_t>(ctx, n, y, dy, dx, ReluBwd{}, "relu_bwd");
}

int nott_add(nott_ctx ctx, nott_dtype dtype, int64_t n, const void* a, const void* b, void* dst) {
    NOTT_CHECK_CTX(ctx);
    NOTT_REQUIRE(ctx, nott::valid_dtype(dtype) && n >= 0, "nott_add: bad dtype or size");
    NOTT_REQUIRE(ctx, n == 0 || (a && b && dst), "nott_add: null buffer");
    nott::DeviceScope scope(ctx->device);
    return dtype == NOTT_F32 ? run_binary<float>(ctx, n, a, b, dst, Add{}, "add")
                             : run_binary<bf16_t>(ctx, n, a, b, dst, Add{}, "add");
}

int nott_add_relu_bwd(nott_ctx ctx, nott_dtype dtype, int64_t n, const void* a, const void* b, const void* y,
                      void* dz) {
    NOTT_CHECK_CTX(ctx);
    NOTT_REQUIRE(ctx, nott::valid_dtype(dtype) && n >= 0, "nott_add_relu_bwd: bad dtype or size");
    NOTT_REQUIRE(ctx, n == 0 || (a && b && y && dz), "nott_add_relu_bwd: null buffer");
    if (n == 0) return NOTT_OK;
    nott::DeviceScope scope(ctx->device);
    auto go = [&](auto tv) {
        using T = decltype(tv);
        const bool vec = ((uintptr_t)a % 16) == 0 && ((uintptr_t)b % 16) == 0 && ((uintptr_t)y % 16) == 0 &&
                         ((uintptr_t)dz % 16) == 0;
        if (vec) {
            constexpr int V = 16 / (int)sizeof(T);
            const int64_t blocks = nott::ceil_div(nott::ceil_div(n, (int64_t)V), (int64_t)kThreads);
            hipLaunchKernelGGL((add_relu_bwd_kernel<T>), dim3((unsigned)blocks), dim3(kThreads), 0, ctx->stream,
                               static_cast<const T*>(a), static_cast<const T*>(b), static_cast<const T*>(y),
                               static_cast<T*>(dz), n);
            return nott::launch_status(ctx, "add_relu_bwd");
        }
        // unaligned: the two passes (the same values)
        const int st = run_binary<T>(ctx, n, a, b, dz, Add{}, "add");
        if (st != NOTT_OK) return st;
        return run_binary<T>(ctx, n, y, dz, dz, ReluBwd{}, "relu_bwd");
    };
    return dtype == NOTT_F32 ? go(float{}) : go(bf16_t{});
}

int nott_cast(nott_ctx ctx, int64_t n, const void* src, nott_dtype st, void* dst, nott_dtype dt) {
    NOTT_CHECK_CTX(ctx);
    NOTT_REQUIRE(ctx, nott::valid_dtype(st) && nott::valid_dtype(dt) && n >= 0, "nott_cast: bad dtype or size");
    NOTT_REQUIRE(ctx, n == 0 || (src && dst), "nott_cast: null buffer");
    if (n == 0) return NOTT_OK;
    nott::DeviceScope scope(ctx->device);
    const dim3 grid((unsigned)nott::ceil_div(n, kThreads));
    if (st == NOTT_F32 && dt == NOTT_BF16 && ((uintptr_t)src & 15) == 0 && ((uintptr_t)dst & 15) == 0 && n >= 8) {
        // whole 8-element groups vectorised, the tail by the element kernel
        const int64_t ng = n / 8, done = 8 * ng;
        hipLaunchKernelGGL(cast_f32_bf16_vec_kernel, dim3((unsigned)nott::ceil_div(ng, kThreads)), dim3(kThreads), 0,
                           ctx->stream, static_cast<const float*>(src), static_cast<bf16_t*>(dst), ng);
        if (done < n)
            hipLaunchKernelGGL((cast_kernel<float, bf16_t>), dim3(1), dim3(kThreads), 0, ctx->stream,
                               static_cast<const float*>(src) + done, static_cast<bf16_t*>(dst) + done, n - done);
    } else if (st == NOTT_F32 && dt == NOTT_BF16)
        hipLaunchKernelGGL((cast_kernel<float, bf16_t>), grid, dim3(kThreads), 0, ctx->stream,
                           static_cast<const float*>(src), static_cast<bf16_t*>(dst), n);
    else if (st == NOTT_BF16 && dt == NOTT_F32)
        hipLaunchKernelGGL((cast_kernel<bf16_t, float>), grid, dim3(kThreads), 0, ctx->stream,
                           static_cast<const bf16_t*>(src), static_cast<float*>(dst), n);
    else if (st == NOTT_F32)
        hipLaunchKernelGGL((cast_kernel<float, float>), grid, dim3(kThreads), 0, ctx->stream,
                           static_cast<const float*>(src), static_cast<float*>(dst), n);
    else
        hipLaunchKernelGGL((cast_kernel<bf16_t, bf16_t>), grid, dim3(kThreads), 0, ctx->stream,
                           static_cast<const bf16_t*>(src), static_cast<bf16_t*>(dst), n);
    return nott::launch_status(ctx, "cast");
}

int nott_zero(nott_ctx ctx, int64_t bytes, void* dst) {
    NOTT_CHECK_CTX(ctx);
    NOTT_REQUIRE(ctx, bytes >= 0, "nott_zero: negative size");
    if (bytes == 0) return NOTT_OK;
    NOTT_REQUIRE(ctx, dst != nullptr, "nott_zero: null buffer");
    NOTT_REQUIRE(ctx, ((uintptr_t)dst % 4) == 0, "nott_zero: buffer must be 4-byte aligned");
    nott::DeviceScope scope(ctx->device);
    const int64_t nwords = bytes / 4, ntail = bytes % 4;
    uint8_t* tail = static_cast<uint8_t*>(dst) + nwords * 4;
    const int64_t work = nwords > ntail ? nwords : ntail;
    hipLaunchKernelGGL(zero_kernel, dim3((unsigned)nott::ceil_div(work, kThreads)), dim3(kThreads), 0, ctx->stream,
                       static_cast<uint32_t*>(dst), nwords, tail, ntail);
    return nott::launch_status(ctx, "zero");
}

int nott_scale(nott_ctx ctx, nott_dtype dtype, int64_t n, const void* x, const float* scale, void* y) {
    NOTT_CHECK_CTX(ctx);
    NOTT_REQUIRE(ctx, nott::valid_dtype(dtype) && n >= 0, "nott_scale: bad dtype or size");
    if (n == 0) return NOTT_OK;
    NOTT_REQUIRE(ctx, x && scale && y, "nott_scale: null buffer");
    nott::DeviceScope scope(ctx->device);
    const dim3 grid((unsigned)nott::ceil_div(n, kThreads));
    if (dtype == NOTT_F32)
        hipLaunchKernelGGL(scale_kernel<float>, grid, dim3(kThreads), 0, ctx->stream, static_cast<const float*>(x), scale,
                           static_cast<float*>(y), n);
    else
        hipLaunchKernelGGL(scale_kernel<bf16_t>, grid, dim3(kThreads), 0, ctx->stream, static_cast<const bf16_t*>(x),
                           scale, static_cast<bf16_t*>(y), n);
    return nott::launch_status(ctx, "scale");
}

int nott_avgpool_global_fwd(nott_ctx ctx, nott_dtype dtype, int64_t nc, int64_t hw, const void* x, void* y) {
    NOTT_CHECK_CTX(ctx);
    NOTT_REQUIRE(ctx, nott::valid_dtype(dtype) && nc >= 0 && hw > 0, "nott_avgpool_global_fwd: bad arguments");
    if (nc == 0) return NOTT_OK;
    NOTT_REQUIRE(ctx, x && y, "nott_avgpool_global_fwd: null buffer");
    nott::DeviceScope scope(ctx->device);
    const dim3 grid((unsigned)nott::ceil_div(nc, kThreads / 64));
    if (dtype == NOTT_F32)
        hipLaunchKernelGGL(avgpool_fwd_kernel<float>, grid, dim3(kThreads), 0, ctx->stream,
                           static_cast<const float*>(x), static_cast<float*>(y), nc, hw);
    else
        hipLaunchKernelGGL(avgpool_fwd_kernel<bf16_t>, grid, dim3(kThreads), 0, ctx->stream,
                           static_cast<const bf16_t*>(x), static_cast<bf16_t*>(y), nc, hw);
    return nott::launch_status(ctx, "avgpool_fwd");
}

int nott_avgpool_global_bwd(nott_ctx ctx, nott_dtype dtype, int64_t nc, int64_t hw, const void* dy, void* dx) {
    NOTT_CHECK_CTX(ctx);
    NOTT_REQUIRE(ctx, nott::valid_dtype(dtype) && nc >= 0 && hw > 0, "nott_avgpool_global_bwd: bad arguments");
    if (nc == 0) return NOTT_OK;
    NOTT_REQUIRE(ctx, dy && dx, "nott_avgpool_global_bwd: null buffer");
    nott::DeviceScope scope(ctx->device);
    const dim3 grid((unsigned)nott::ceil_div(nc * hw, kThreads));
    if (dtype == NOTT_F32)
        hipLaunchKernelGGL(avgpool_bwd_kernel<float>, grid, dim3(kThreads), 0, ctx->stream,
                           static_cast<const float*>(dy), static_cast<float*>(dx), nc, hw);
    else
        hipLaunchKernelGGL(avgpool_bwd_kernel<bf16_t>, grid, dim3(kThreads), 0, ctx->stream,
                           static_cast<const bf16_t*>(dy), static_cast<bf16_t*>(dx), nc, hw);
    return nott::launch_status(ctx, "avgpool_bwd");
}

}  // extern "C"

namespace {
__global__ void loss_accumulate_kernel(const float* __restrict__ loss, double weight, double* __restrict__ acc) {
    acc[0] += (double)loss[0] * weight;
}
}  // namespace

extern "C" int nott_loss_accumulate(nott_ctx ctx, const float* loss, double weight, double* acc) {
    NOTT_CHECK_CTX(ctx);
    NOTT_REQUIRE(ctx, loss && acc, "nott_loss_accumulate: null buffer");
    nott::DeviceScope scope(ctx->device);
    hipLaunchKernelGGL(loss_accumulate_kernel, dim3(1), dim3(1), 0, ctx->stream, loss, weight, acc);
    return nott::launch_status(ctx, "loss_accumulate");
}
