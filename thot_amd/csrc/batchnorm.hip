// BatchNorm2d (training mode) forward and backward, NCHW.
//
// Replaces torch::nn::BatchNorm2d built by build_registered_layer(Owner&,
// const BatchNorm2dDescriptor&, size_t) (reference layer/details/batchnorm.hpp:38-59;
// eps 1e-5, momentum 0.1, affine, running stats), i.e. ATen native_batch_norm
// and native_batch_norm_backward.
//   forward : μ_c, var_c (biased) over (n, hw); rstd = 1/sqrt(var + eps);
//             y = (x − μ)·rstd·γ + β; running = (1−m)·running + m·stat (unbiased var)
//   backward: dβ = Σdy; dγ = Σdy·x̂; dx = γ·rstd·(dy − Σdy/M − x̂·Σ(dy·x̂)/M)
// Each pass is a per-(channel, slice) partial reduction followed by a tiny
// per-channel finalize and one streaming apply pass.
#include "common.hpp"

#include <initializer_list>
#include <type_traits>

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

template <int NW>
__device__ __forceinline__ void block_sum2(float& a, float& b, float* red) {
    a = wave_sum(a);
    b = wave_sum(b);
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    if (lane == 0) {
        red[wid] = a;
        red[NW + wid] = b;
    }
    __syncthreads();
    float ta = 0.f, tb = 0.f;
#pragma unroll
    for (int i = 0; i < NW; ++i) {
        ta += red[i];
        tb += red[NW + i];
    }
    __syncthreads();
    a = ta;
    b = tb;
}

// A group of V consecutive elements (V = 1, 4, or 8 for bf16) as floats:
// one 4-, 8-, 16- or 16-byte access.
template <typename T, int V>
__device__ __forceinline__ void ld_grp(const T* __restrict__ p, float (&o)[V]) {
    if constexpr (V == 1) {
        o[0] = Io<T>::ld(p, 0);
    } else if constexpr (V == 4) {
        const f32x4 v = Vec4<T>::ld(p);
        o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
    } else {
        static_assert(V == 8 && sizeof(T) == 2, "8-element groups are 16 bytes of bf16");
        const u32x4 u = *reinterpret_cast<const u32x4*>(p);
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            o[2 * k] = __builtin_bit_cast(float, w[k] << 16);
            o[2 * k + 1] = __builtin_bit_cast(float, w[k] & 0xffff0000u);
        }
    }
}
template <typename T, int V>
__device__ __forceinline__ void st_grp(T* __restrict__ p, const float (&o)[V]) {
    if constexpr (V == 1) {
        Io<T>::st(p, 0, o[0]);
    } else if constexpr (V == 4) {
        Vec4<T>::st(p, f32x4{o[0], o[1], o[2], o[3]});
    } else {
        static_assert(V == 8 && sizeof(T) == 2, "8-element groups are 16 bytes of bf16");
        *reinterpret_cast<u32x4*>(p) = u32x4{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3]),
                                            pack_bf16x2(o[4], o[5]), pack_bf16x2(o[6], o[7])};
    }
}
// A group as loaded, for the reductions that keep several groups in flight:
// bf16 groups of 4 or 8 stay packed (2 per dword) until they are added, which
// halves the registers a batch holds; other groups are floats.
template <typename T, int V>
struct RawGrp {
    static constexpr bool kPacked = sizeof(T) == 2 && V >= 4;
    uint32_t w[kPacked ? V / 2 : 1];
    float f[kPacked ? 1 : V];
};
template <typename T, int V>
__device__ __forceinline__ void ld_raw(const T* __restrict__ p, RawGrp<T, V>& r) {
    if constexpr (RawGrp<T, V>::kPacked) {
        if constexpr (V == 8) {
            const u32x4 u = *reinterpret_cast<const u32x4*>(p);
            r.w[0] = u.x; r.w[1] = u.y; r.w[2] = u.z; r.w[3] = u.w;
        } else {
            const u32x2 u = *reinterpret_cast<const u32x2*>(p);
            r.w[0] = u.x; r.w[1] = u.y;
        }
    } else {
        ld_grp<T, V>(p, r.f);
    }
}
template <typename T, int V>
__device__ __forceinline__ void unpack(const RawGrp<T, V>& r, float (&o)[V]) {
    if constexpr (RawGrp<T, V>::kPacked) {
#pragma unroll
        for (int k = 0; k < V / 2; ++k) {
            o[2 * k] = __builtin_bit_cast(float, r.w[k] << 16);
            o[2 * k + 1] = __builtin_bit_cast(float, r.w[k] & 0xffff0000u);
        }
    } else {
#pragma unroll
        for (int e = 0; e < V; ++e) o[e] = r.f[e];
    }
}

// Σ of a group in a fixed pairwise order.
template <int V>
__device__ __forceinline__ float grp_sum(const float (&o)[V]) {
    if constexpr (V == 1) return o[0];
    else if constexpr (V == 4) return (o[0] + o[1]) + (o[2] + o[3]);
    else return ((o[0] + o[1]) + (o[2] + o[3])) + ((o[4] + o[5]) + (o[6] + o[7]));
}

// Items of the per-channel partial reductions: item k of a split is group
// k % hwg of image n0 + k / hwg.  A thread takes items t, t + kThreads, ...,
// kUnroll of them loaded before they are added (in item order), so the
// summation order is fixed and several loads are in flight per thread.
constexpr int kUnroll = 4;
constexpr int kUnrollB = 2;   // the backward's two tensors: half the items

// Partial sums of (x − pivot) and (x − pivot)² over planes [n0, n1) of
// channel blockIdx.x.  pivot = x[0, c, 0] keeps the variance well conditioned.
// Splits of at least kThreads groups (V pixels each) are walked as items
// (above); smaller ones give a thread one group per image: its loads for up
// to kAhead images are issued before the adds, which run in the same order.
constexpr int kAhead = 8;
constexpr int kAheadB = 2;   // the backward's two tensors: half the images
template <typename T, int V>
__global__ __launch_bounds__(kThreads) void bn_stats_kernel(const T* __restrict__ x, int64_t n, int64_t c, int64_t hw,
                                                            int64_t per_split, FastDiv fd_hwg,
                                                            float* __restrict__ partial) {
    __shared__ float red[2 * kWaves];
    const int64_t ch = blockIdx.x;
    const int64_t n0 = (int64_t)blockIdx.y * per_split;
    const int64_t n1 = std::min<int64_t>(n, n0 + per_split);
    const float pivot = Io<T>::ld(x, ch * hw);
    const int64_t hwg = hw / V;
    float s1 = 0.f, s2 = 0.f;
    auto add = [&](float (&v)[V]) {
#pragma unroll
        for (int e = 0; e < V; ++e) v[e] -= pivot;
        float sq[V];
#pragma unroll
        for (int e = 0; e < V; ++e) sq[e] = v[e] * v[e];
        s1 += grp_sum<V>(v);
        s2 += grp_sum<V>(sq);
    };
    if ((n1 - n0) * hwg >= kThreads) {
        const uint32_t items = (uint32_t)((n1 - n0) * hwg);
        auto at = [&](uint32_t k) {
            uint32_t i, j;
            fd_hwg.divmod(k, i, j);
            return x + ((n0 + i) * c + ch) * hw + (int64_t)j * V;
        };
        uint32_t k = threadIdx.x;
        for (; k + (kUnroll - 1) * kThreads < items; k += kUnroll * kThreads) {
            RawGrp<T, V> rv[kUnroll];
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) ld_raw<T, V>(at(k + u * kThreads), rv[u]);
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                float v[V];
                unpack<T, V>(rv[u], v);
                add(v);
            }
        }
        for (; k < items; k += kThreads) {
            float v[V];
            ld_grp<T, V>(at(k), v);
            add(v);
        }
    } else if ((int64_t)threadIdx.x < hwg) {
        const int64_t step = c * hw;
        int64_t e = (n0 * c + ch) * hw + (int64_t)threadIdx.x * V, i = n0;
        for (; i + kAhead <= n1; i += kAhead, e += kAhead * step) {
            RawGrp<T, V> rv[kAhead];
#pragma unroll
            for (int u = 0; u < kAhead; ++u) ld_raw<T, V>(x + e + u * step, rv[u]);
#pragma unroll
            for (int u = 0; u < kAhead; ++u) {
                float v[V];
                unpack<T, V>(rv[u], v);
                add(v);
            }
        }
        for (; i < n1; ++i, e += step) {
            float v[V];
            ld_grp<T, V>(x + e, v);
            add(v);
        }
    }
    block_sum2<kWaves>(s1, s2, red);
    if (threadIdx.x == 0) {
        partial[(ch * gridDim.y + blockIdx.y) * 2 + 0] = s1;
        partial[(ch * gridDim.y + blockIdx.y) * 2 + 1] = s2;
    }
}

// Per channel: mean, rstd, running stats and the affine coefficients
// Per-channel affine form of the normalisation, z = a·x + c, shared by the
// forward apply and by the backward's recomputation of the ReLU mask, so both
// see the same z bit for bit.
__device__ __forceinline__ void bn_coef(float g, float b, float mu, float rs, float& a, float& c) {
#pragma clang fp contract(off)
    a = g * rs;
    c = b - mu * a;
}
__device__ __forceinline__ float bn_z(float x, float a, float c) { return __builtin_fmaf(x, a, c); }
// ReLU forward (a NaN passes) and its gradient mask (zero where y <= 0).
__device__ __forceinline__ float relu_f(float v) { return (v > 0.f || v != v) ? v : 0.f; }

// Backward through a fused ReLU: the incoming gradient is w.r.t.
// relu(a·x + c); the mask is recomputed from x, γ, β, μ and rstd.
struct BnAct {
    int relu;
    const float* gamma;
    const float* beta;
    const float* rstd;
};

// Sum of channel ch's split partials (pairs) by one thread, in split order
// (double accumulation; the channel's pairs are contiguous, read as
// 16-byte pieces when aligned).
__device__ __forceinline__ void sum_partials(const float* __restrict__ partial, int64_t ch, int64_t splits,
                                             double& s1, double& s2) {
    const float* q = partial + ch * splits * 2;
    s1 = 0.0;
    s2 = 0.0;
    int64_t s = 0;
    if (((uintptr_t)q & 15) == 0) {
        for (; s + 8 <= splits; s += 8) {
            f32x4 v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) v[u] = *reinterpret_cast<const f32x4*>(q + 2 * s + 4 * u);
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                s1 += v[u].x;
                s2 += v[u].y;
                s1 += v[u].z;
                s2 += v[u].w;
            }
        }
    }
    for (; s < splits; ++s) {
        s1 += q[2 * s];
        s2 += q[2 * s + 1];
    }
}

// Per channel: mean, rstd, running stats and the coefficients (a, c) of
// y = a·x + c used by the apply pass.  One thread per channel; every load
// the channel needs is issued before its partials are summed.
template <typename T>
__global__ __launch_bounds__(64) void bn_fwd_finalize(const T* __restrict__ x, const float* __restrict__ partial, int64_t c,
                                                      int64_t splits, int64_t hw, int64_t m,
                                                      const float* __restrict__ gamma, const float* __restrict__ beta,
                                                      float eps, float momentum, float* __restrict__ running_mean,
                                                      float* __restrict__ running_var, float* __restrict__ mean,
                                                      float* __restrict__ rstd, float* __restrict__ coef) {
    const int64_t ch = (int64_t)blockIdx.x * 64 + threadIdx.x;
    if (ch >= c) return;
    const float pivot = Io<T>::ld(x, ch * hw);
    const float g = gamma ? gamma[ch] : 1.f, b = beta ? beta[ch] : 0.f;
    const float rm0 = running_mean ? running_mean[ch] : 0.f, rv0 = running_mean ? running_var[ch] : 0.f;
    double s1, s2;
    sum_partials(partial, ch, splits, s1, s2);
    const double md = s1 / (double)m;
    double var = s2 / (double)m - md * md;
    if (var < 0.0) var = 0.0;
    const float mu = (float)(md + pivot);
    const float rs = (float)(1.0 / sqrt(var + (double)eps));
    mean[ch] = mu;
    rstd[ch] = rs;
    bn_coef(g, b, mu, rs, coef[2 * ch + 0], coef[2 * ch + 1]);
    if (running_mean) {
        const double unbiased = m > 1 ? var * (double)m / (double)(m - 1) : var;
        running_mean[ch] = (1.f - momentum) * rm0 + momentum * mu;
        running_var[ch] = (1.f - momentum) * rv0 + momentum * (float)unbiased;
    }
}

// y = act(a_c·x + c_c [+ res]) over the whole tensor (act = ReLU or identity).
// One thread per group of V elements of a flat grid: a group lies in one
// (n, c) plane, found with two multiply-high divisions.
template <typename T, int V>
__global__ __launch_bounds__(kThreads) void bn_affine_kernel(const T* __restrict__ x, T* __restrict__ y, uint32_t ngroups,
                                                             FastDiv fd_hwg, FastDiv fd_c, const float* __restrict__ coef,
                                                             const T* __restrict__ res, int relu) {
    const uint32_t q = blockIdx.x * kThreads + threadIdx.x;
    if (q >= ngroups) return;
    uint32_t plane, j, img, ch;
    fd_hwg.divmod(q, plane, j);
    fd_c.divmod(plane, img, ch);
    const int64_t i = (int64_t)q * V;
    const float a = coef[2 * ch], b = coef[2 * ch + 1];
    float v[V];
    ld_grp<T, V>(x + i, v);
#pragma unroll
    for (int e = 0; e < V; ++e) v[e] = bn_z(v[e], a, b);
    if (res) {
        float r[V];
        ld_grp<T, V>(res + i, r);
#pragma unroll
        for (int e = 0; e < V; ++e) v[e] += r[e];
    }
    if (relu) {
#pragma unroll
        for (int e = 0; e < V; ++e) v[e] = relu_f(v[e]);
    }
    st_grp<T, V>(y + i, v);
}

// Backward partial sums of dy and dy·(x − μ), in the order of bn_stats_kernel.
template <typename T, int V>
__global__ __launch_bounds__(kThreads) void bn_bwd_reduce_kernel(const T* __restrict__ x, const T* __restrict__ dy,
                                                                 const float* __restrict__ mean, int64_t n, int64_t c,
                                                                 int64_t hw, int64_t per_split, FastDiv fd_hwg,
                                                                 float* __restrict__ partial, BnAct act) {
    __shared__ float red[2 * kWaves];
    const int64_t ch = blockIdx.x;
    const int64_t n0 = (int64_t)blockIdx.y * per_split;
    const int64_t n1 = std::min<int64_t>(n, n0 + per_split);
    const float mu = mean[ch];
    float za = 0.f, zc = 0.f;   // z = za·x + zc when the gradient comes through a ReLU
    if (act.relu) bn_coef(act.gamma ? act.gamma[ch] : 1.f, act.beta ? act.beta[ch] : 0.f, mu, act.rstd[ch], za, zc);
    float s1 = 0.f, s2 = 0.f;
    const int64_t hwg = hw / V;
    auto add = [&](float (&g)[V], const float (&v)[V]) {
        if (act.relu) {
#pragma unroll
            for (int e = 0; e < V; ++e)
                if (bn_z(v[e], za, zc) <= 0.f) g[e] = 0.f;
        }
        float gx[V];
#pragma unroll
        for (int e = 0; e < V; ++e) gx[e] = g[e] * (v[e] - mu);
        s1 += grp_sum<V>(g);
        s2 += grp_sum<V>(gx);
    };
    if ((n1 - n0) * hwg >= kThreads) {
        const uint32_t items = (uint32_t)((n1 - n0) * hwg);
        auto off = [&](uint32_t k) {
            uint32_t i, j;
            fd_hwg.divmod(k, i, j);
            return ((n0 + i) * c + ch) * hw + (int64_t)j * V;
        };
        uint32_t k = threadIdx.x;
        for (; k + (kUnrollB - 1) * kThreads < items; k += kUnrollB * kThreads) {
            RawGrp<T, V> rg[kUnrollB], rv[kUnrollB];
#pragma unroll
            for (int u = 0; u < kUnrollB; ++u) {
                const int64_t e = off(k + u * kThreads);
                ld_raw<T, V>(dy + e, rg[u]);
                ld_raw<T, V>(x + e, rv[u]);
            }
#pragma unroll
            for (int u = 0; u < kUnrollB; ++u) {
                float g[V], v[V];
                unpack<T, V>(rg[u], g);
                unpack<T, V>(rv[u], v);
                add(g, v);
            }
        }
        for (; k < items; k += kThreads) {
            float g[V], v[V];
            const int64_t e = off(k);
            ld_grp<T, V>(dy + e, g);
            ld_grp<T, V>(x + e, v);
            add(g, v);
        }
    } else if ((int64_t)threadIdx.x < hwg) {
        const int64_t step = c * hw;
        int64_t e = (n0 * c + ch) * hw + (int64_t)threadIdx.x * V, i = n0;
        for (; i + kAheadB <= n1; i += kAheadB, e += kAheadB * step) {
            RawGrp<T, V> rg[kAheadB], rv[kAheadB];
#pragma unroll
            for (int u = 0; u < kAheadB; ++u) {
                ld_raw<T, V>(dy + e + u * step, rg[u]);
                ld_raw<T, V>(x + e + u * step, rv[u]);
            }
#pragma unroll
            for (int u = 0; u < kAheadB; ++u) {
                float g[V], v[V];
                unpack<T, V>(rg[u], g);
                unpack<T, V>(rv[u], v);
                add(g, v);
            }
        }
        for (; i < n1; ++i, e += step) {
            float g[V], v[V];
            ld_grp<T, V>(dy + e, g);
            ld_grp<T, V>(x + e, v);
            add(g, v);
        }
    }
    block_sum2<kWaves>(s1, s2, red);
    if (threadIdx.x == 0) {
        partial[(ch * gridDim.y + blockIdx.y) * 2 + 0] = s1;
        partial[(ch * gridDim.y + blockIdx.y) * 2 + 1] = s2;
    }
}

// dγ, dβ and the coefficients of dx = A·dy + B·x + C.  One thread per
// channel, its loads issued before the partials are summed.
__global__ __launch_bounds__(64) void bn_bwd_finalize(const float* __restrict__ partial, int64_t c, int64_t splits,
                                                      int64_t m, const float* __restrict__ mean,
                                                      const float* __restrict__ rstd, const float* __restrict__ gamma,
                                                      float* __restrict__ dgamma, float* __restrict__ dbeta,
                                                      int accumulate, float* __restrict__ coef) {
    const int64_t ch = (int64_t)blockIdx.x * 64 + threadIdx.x;
    if (ch >= c) return;
    const double rs = rstd[ch], mu = mean[ch];
    const double g = gamma ? gamma[ch] : 1.0;
    const float dg0 = (dgamma && accumulate) ? dgamma[ch] : 0.f, db0 = (dbeta && accumulate) ? dbeta[ch] : 0.f;
    double sdy, sdyxc;
    sum_partials(partial, ch, splits, sdy, sdyxc);
    const double sdyx = sdyxc * rs;  // Σ dy·x̂
    if (dgamma) dgamma[ch] = accumulate ? dg0 + (float)sdyx : (float)sdyx;
    if (dbeta) dbeta[ch] = accumulate ? db0 + (float)sdy : (float)sdy;
    const double A = g * rs;
    const double B = -g * rs * rs * sdyx / (double)m;
    const double C = -g * rs * sdy / (double)m - B * mu;
    coef[3 * ch + 0] = (float)A;
    coef[3 * ch + 1] = (float)B;
    coef[3 * ch + 2] = (float)C;
}

template <typename T, int V>
__global__ __launch_bounds__(kThreads) void bn_bwd_apply_kernel(const T* __restrict__ x, const T* __restrict__ dy,
                                                                T* __restrict__ dx, uint32_t ngroups, FastDiv fd_hwg,
                                                                FastDiv fd_c, const float* __restrict__ coef,
                                                                const float* __restrict__ mean, BnAct act) {
    const uint32_t q = blockIdx.x * kThreads + threadIdx.x;
    if (q >= ngroups) return;
    uint32_t plane, j, img, ch;
    fd_hwg.divmod(q, plane, j);
    fd_c.divmod(plane, img, ch);
    const int64_t i = (int64_t)q * V;
    const float A = coef[3 * ch], B = coef[3 * ch + 1], C = coef[3 * ch + 2];
    float za = 0.f, zc = 0.f;
    if (act.relu)
        bn_coef(act.gamma ? act.gamma[ch] : 1.f, act.beta ? act.beta[ch] : 0.f, mean[ch], act.rstd[ch], za, zc);
    float g[V], v[V];
    ld_grp<T, V>(dy + i, g);
    ld_grp<T, V>(x + i, v);
    if (act.relu) {
#pragma unroll
        for (int e = 0; e < V; ++e)
            if (bn_z(v[e], za, zc) <= 0.f) g[e] = 0.f;
    }
    float r[V];
#pragma unroll
    for (int e = 0; e < V; ++e) r[e] = A * g[e] + B * v[e] + C;
    st_grp<T, V>(dx + i, r);
}

// Elements per group of the streaming passes: 16-byte groups (8 bf16 / 4
// fp32) when the planes are whole groups and every tensor is 16-byte
// aligned, 4 elements at 8-byte alignment, else single elements.
template <typename T>
int group_width(int64_t hw, std::initializer_list<const void*> ptrs) {
    auto aligned = [&](size_t a) {
        for (const void* q : ptrs)
            if (((uintptr_t)q % a) != 0) return false;
        return true;
    };
    if (sizeof(T) == 2 && hw % 8 == 0 && aligned(16)) return 8;
    if (hw % 4 == 0 && aligned(4 * sizeof(T))) return 4;
    return 1;
}

int64_t pick_splits(int64_t n, int64_t c) {
    int64_t s = nott::ceil_div(2048, c);
    return std::max<int64_t>(1, std::min<int64_t>(s, n));
}

// coef_out (nullable): the per-channel affine coefficients (a, c) of
// y = a·x + c go there instead of the workspace; yv null: no apply pass.
template <typename T>
int fwd(nott_ctx ctx, int64_t n, int64_t c, int64_t hw, const void* xv, const float* gamma, const float* beta,
        float eps, float momentum, float* rm, float* rv, void* yv, float* mean, float* rstd, const void* resv, int relu,
        float* coef_out = nullptr) {
    const T* x = static_cast<const T*>(xv);
    const T* res = static_cast<const T*>(resv);
    T* y = static_cast<T*>(yv);
    const int64_t splits0 = pick_splits(n, c);
    const int64_t per = nott::ceil_div(n, splits0);
    const int64_t splits = nott::ceil_div(n, per);
    float* ws = static_cast<float*>(nott::workspace(ctx, sizeof(float) * (size_t)(2 * c * splits + 2 * c)));
    if (!ws) return NOTT_ERR_ALLOC;
    float* partial = ws;
    float* coef = coef_out ? coef_out : ws + 2 * c * splits;
    const int v = group_width<T>(hw, {xv, yv, resv});
    const dim3 g1((unsigned)c, (unsigned)splits);
    const FastDiv fd_hwg((uint32_t)(hw / v)), fd_c((uint32_t)c);
    const uint32_t ngroups = (uint32_t)(n * c * (hw / v));
    const dim3 ga((unsigned)nott::ceil_div(ngroups, kThreads));
    auto go = [&](auto vt) {
        constexpr int V = decltype(vt)::value;
        hipLaunchKernelGGL((bn_stats_kernel<T, V>), g1, dim3(kThreads), 0, ctx->stream, x, n, c, hw, per, fd_hwg,
                           partial);
        hipLaunchKernelGGL(bn_fwd_finalize<T>, dim3((unsigned)nott::ceil_div(c, 64)), dim3(64), 0, ctx->stream, x,
                           partial, c, splits, hw,
                           n * hw, gamma, beta, eps, momentum, rm, rv, mean, rstd, coef);
        if (y)
            hipLaunchKernelGGL((bn_affine_kernel<T, V>), ga, dim3(kThreads), 0, ctx->stream, x, y, ngroups, fd_hwg,
                               fd_c, coef, res, relu);
    };
    if constexpr (sizeof(T) == 2) {
        if (v == 8) go(std::integral_constant<int, 8>{});
    }
    if (v == 4) go(std::integral_constant<int, 4>{});
    else if (v == 1) go(std::integral_constant<int, 1>{});
    return nott::launch_status(ctx, "batchnorm_fwd");
}

template <typename T>
// ws_ext (nullable): (2·c·splits + 3·c) floats to use instead of the context
// workspace.
int bwd(nott_ctx ctx, int64_t n, int64_t c, int64_t hw, const void* xv, const void* dyv, const float* mean,
        const float* rstd, const float* gamma, void* dxv, float* dgamma, float* dbeta, int accumulate, BnAct act,
        float* ws_ext = nullptr) {
    const T* x = static_cast<const T*>(xv);
    const T* dy = static_cast<const T*>(dyv);
    T* dx = static_cast<T*>(dxv);
    const int64_t splits0 = pick_splits(n, c);
    const int64_t per = nott::ceil_div(n, splits0);
    const int64_t splits = nott::ceil_div(n, per);
    float* ws = ws_ext ? ws_ext
                       : static_cast<float*>(nott::workspace(ctx, sizeof(float) * (size_t)(2 * c * splits + 3 * c)));
    if (!ws) return NOTT_ERR_ALLOC;
    float* partial = ws;
    float* coef = ws + 2 * c * splits;
    const int v = group_width<T>(hw, {xv, dyv, dxv});
    const dim3 g1((unsigned)c, (unsigned)splits);
    const FastDiv fd_hwg((uint32_t)(hw / v)), fd_c((uint32_t)c);
    const uint32_t ngroups = (uint32_t)(n * c * (hw / v));
    const dim3 ga((unsigned)nott::ceil_div(ngroups, kThreads));
    auto go = [&](auto vt) {
        constexpr int V = decltype(vt)::value;
        hipLaunchKernelGGL((bn_bwd_reduce_kernel<T, V>), g1, dim3(kThreads), 0, ctx->stream, x, dy, mean, n, c, hw,
                           per, fd_hwg, partial, act);
        hipLaunchKernelGGL(bn_bwd_finalize, dim3((unsigned)nott::ceil_div(c, 64)), dim3(64), 0, ctx->stream, partial, c,
                           splits, n * hw,
                           mean, rstd, gamma, dgamma, dbeta, accumulate, coef);
        if (dx)
            hipLaunchKernelGGL((bn_bwd_apply_kernel<T, V>), ga, dim3(kThreads), 0, ctx->stream, x, dy, dx, ngroups,
                               fd_hwg, fd_c, coef, mean, act);
    };
    if constexpr (sizeof(T) == 2) {
        if (v == 8) go(std::integral_constant<int, 8>{});
    }
    if (v == 4) go(std::integral_constant<int, 4>{});
    else if (v == 1) go(std::integral_constant<int, 1>{});
    return nott::launch_status(ctx, "batchnorm_bwd");
}

}  // namespace

namespace nott {
bool maxpool_bnrelu_bwd_applies(const nott_pool2d_desc* d, nott_dtype dtype, const uint8_t* tap, const void* dy,
                                const void* x, const void* dx);
int maxpool_bwd_tap_bnrelu_reduce(nott_ctx ctx, const nott_pool2d_desc* d, nott_dtype dtype, const uint8_t* tap,
                                  const void* dy, const void* x, const float* gamma, const float* beta,
                                  const float* mean, const float* rstd, int32_t per_split, int32_t splits,
                                  float* partial);
int maxpool_bwd_tap_bnrelu_apply(nott_ctx ctx, const nott_pool2d_desc* d, nott_dtype dtype, const uint8_t* tap,
                                 const void* dy, const void* x, const float* abc, const float* gamma,
                                 const float* beta, const float* mean, const float* rstd, void* dx);
}  // namespace nott

extern "C" int nott_batchnorm2d_fwd_act(nott_ctx ctx, nott_dtype dtype, int64_t n, int64_t c, int64_t hw,
                                        const void* x, const float* gamma, const float* beta, double eps,
                                        double momentum, float* running_mean, float* running_var,
                                        const void* residual, int relu, void* y, float* mean, float* rstd) {
    NOTT_CHECK_CTX(ctx);
    NOTT_REQUIRE(ctx, nott::valid_dtype(dtype) && n > 0 && c > 0 && hw > 0, "nott_batchnorm2d_fwd: bad shape");
    NOTT_REQUIRE(ctx, (running_mean == nullptr) == (running_var == nullptr),
                 "nott_batchnorm2d_fwd: running_mean and running_var go together");
    NOTT_REQUIRE(ctx, x && y && mean && rstd, "nott_batchnorm2d_fwd: null buffer");
    NOTT_REQUIRE(ctx, c <= 65535 && n * c * hw <= 0xffffffffll, "nott_batchnorm2d_fwd: tensor too large");
    nott::DeviceScope scope(ctx->device);
    return dtype == NOTT_F32 ? fwd<float>(ctx, n, c, hw, x, gamma, beta, (float)eps, (float)momentum, running_mean,
                                          running_var, y, mean, rstd, residual, relu != 0)
                             : fwd<bf16_t>(ctx, n, c, hw, x, gamma, beta, (float)eps, (float)momentum, running_mean,
                                           running_var, y, mean, rstd, residual, relu != 0);
}

extern "C" int nott_batchnorm2d_fwd_coef(nott_ctx ctx, nott_dtype dtype, int64_t n, int64_t c, int64_t hw,
                                         const void* x, const float* gamma, const float* beta, double eps,
                                         double momentum, float* running_mean, float* running_var, float* mean,
                                         float* rstd, float* coef) {
    NOTT_CHECK_CTX(ctx);
    NOTT_REQUIRE(ctx, nott::valid_dtype(dtype) && n > 0 && c > 0 && hw > 0, "nott_batchnorm2d_fwd_coef: bad shape");
    NOTT_REQUIRE(ctx, (running_mean == nullptr) == (running_var == nullptr),
                 "nott_batchnorm2d_fwd_coef: running_mean and running_var go together");
    NOTT_REQUIRE(ctx, x && mean && rstd && coef, "nott_batchnorm2d_fwd_coef: null buffer");
    NOTT_REQUIRE(ctx, c <= 65535 && n * c * hw <= 0xffffffffll, "nott_batchnorm2d_fwd_coef: tensor too large");
    nott::DeviceScope scope(ctx->device);
    return dtype == NOTT_F32 ? fwd<float>(ctx, n, c, hw, x, gamma, beta, (float)eps, (float)momentum, running_mean,
                                          running_var, nullptr, mean, rstd, nullptr, 0, coef)
                             : fwd<bf16_t>(ctx, n, c, hw, x, gamma, beta, (float)eps, (float)momentum, running_mean,
                                           running_var, nullptr, mean, rstd, nullptr, 0, coef);
}

extern "C" int nott_batchnorm2d_fwd(nott_ctx ctx, nott_dtype dtype, int64_t n, int64_t c, int64_t hw, const void* x,
                                    const float* gamma, const float* beta, double eps, double momentum,
                                    float* running_mean, float* running_var, void* y, float* mean, float* rstd) {
    return nott_batchnorm2d_fwd_act(ctx, dtype, n, c, hw, x, gamma, beta, eps, momentum, running_mean, running_var,
                                    nullptr, 0, y, mean, rstd);
}

extern "C" int nott_batchnorm2d_bwd_act(nott_ctx ctx, nott_dtype dtype, int64_t n, int64_t c, int64_t hw,
                                        const void* x, const void* dy, const float* mean, const float* rstd,
                                        const float* gamma, const float* beta, int relu, void* dx, float* dgamma,
                                        float* dbeta, int accumulate) {
    NOTT_CHECK_CTX(ctx);
    NOTT_REQUIRE(ctx, nott::valid_dtype(dtype) && n > 0 && c > 0 && hw > 0, "nott_batchnorm2d_bwd: bad shape");
    NOTT_REQUIRE(ctx, x && dy && mean && rstd, "nott_batchnorm2d_bwd: null buffer");
    NOTT_REQUIRE(ctx, c <= 65535 && n * c * hw <= 0xffffffffll, "nott_batchnorm2d_bwd: tensor too large");
    nott::DeviceScope scope(ctx->device);
    const BnAct act{relu != 0, gamma, beta, rstd};
    return dtype == NOTT_F32 ? bwd<float>(ctx, n, c, hw, x, dy, mean, rstd, gamma, dx, dgamma, dbeta, accumulate, act)
                             : bwd<bf16_t>(ctx, n, c, hw, x, dy, mean, rstd, gamma, dx, dgamma, dbeta, accumulate, act);
}

extern "C" int nott_batchnorm2d_bwd(nott_ctx ctx, nott_dtype dtype, int64_t n, int64_t c, int64_t hw, const void* x,
                                    const void* dy, const float* mean, const float* rstd, const float* gamma, void* dx,
                                    float* dgamma, float* dbeta, int accumulate) {
    return nott_batchnorm2d_bwd_act(ctx, dtype, n, c, hw, x, dy, mean, rstd, gamma, nullptr, 0, dx, dgamma, dbeta,
                                    accumulate);
}

extern "C" int nott_batchnorm2d_relu_maxpool2d_bwd(nott_ctx ctx, const nott_pool2d_desc* d, nott_dtype dtype,
                                                   const void* x, const uint8_t* tap, const void* dy,
                                                   const float* mean, const float* rstd, const float* gamma,
                                                   const float* beta, void* dx, float* dgamma, float* dbeta,
                                                   int accumulate) {
    NOTT_CHECK_CTX(ctx);
    NOTT_REQUIRE(ctx, d != nullptr && nott::valid_dtype(dtype), "nott_batchnorm2d_relu_maxpool2d_bwd: bad descriptor");
    NOTT_REQUIRE(ctx, x && tap && dy && mean && rstd, "nott_batchnorm2d_relu_maxpool2d_bwd: null buffer");
    const int64_t n = d->n, c = d->c, hw = d->h * d->w;
    NOTT_REQUIRE(ctx, n > 0 && c > 0 && hw > 0, "nott_batchnorm2d_relu_maxpool2d_bwd: bad shape");
    NOTT_REQUIRE(ctx, c <= 65535 && n * c * hw <= 0xffffffffll, "nott_batchnorm2d_relu_maxpool2d_bwd: tensor too large");
    nott::DeviceScope scope(ctx->device);
    const int64_t splits0 = pick_splits(n, c);
    const int64_t per = nott::ceil_div(n, splits0);
    const int64_t splits = nott::ceil_div(n, per);
    const size_t bn_bytes = sizeof(float) * (size_t)(2 * c * splits + 3 * c);
    if (nott::maxpool_bnrelu_bwd_applies(d, dtype, tap, dy, x, dx ? dx : x)) {
        // the partial sums over the pooled outputs, the coefficients, then the
        // routing with the apply in its epilogue: the routed gradient is never
        // stored
        float* ws = static_cast<float*>(nott::workspace(ctx, bn_bytes));
        if (!ws) return NOTT_ERR_ALLOC;
        float* partial = ws;
        float* coef = ws + 2 * c * splits;
        int st = nott::maxpool_bwd_tap_bnrelu_reduce(ctx, d, dtype, tap, dy, x, gamma, beta, mean, rstd, (int32_t)per,
                                                     (int32_t)splits, partial);
        if (st != NOTT_OK) return st;
        hipLaunchKernelGGL(bn_bwd_finalize, dim3((unsigned)nott::ceil_div(c, 64)), dim3(64), 0, ctx->stream, partial, c,
                           splits, n * hw,
                           mean, rstd, gamma, dgamma, dbeta, accumulate, coef);
        st = nott::launch_status(ctx, "batchnorm_bwd_finalize");
        if (st != NOTT_OK || !dx) return st;
        return nott::maxpool_bwd_tap_bnrelu_apply(ctx, d, dtype, tap, dy, x, coef, gamma, beta, mean, rstd, dx);
    }
    // other shapes: the routed gradient into dx (a workspace plane when dx is
    // null), then the BatchNorm + ReLU backward in place (each element is read
    // before the same thread writes it)
    const size_t zbytes = dx ? 0 : ((size_t)(n * c * hw) * (dtype == NOTT_F32 ? 4 : 2) + 255) / 256 * 256;
    char* ws = static_cast<char*>(nott::workspace(ctx, zbytes + bn_bytes));
    if (!ws) return NOTT_ERR_ALLOC;
    void* dz = dx ? dx : static_cast<void*>(ws);
    int st = nott_maxpool2d_bwd_tap(ctx, d, dtype, tap, dy, dz);
    if (st != NOTT_OK) return st;
    const BnAct act{1, gamma, beta, rstd};
    float* bws = reinterpret_cast<float*>(ws + zbytes);
    return dtype == NOTT_F32
               ? bwd<float>(ctx, n, c, hw, x, dz, mean, rstd, gamma, dx, dgamma, dbeta, accumulate, act, bws)
               : bwd<bf16_t>(ctx, n, c, hw, x, dz, mean, rstd, gamma, dx, dgamma, dbeta, accumulate, act, bws);
}
