// Conv2d forward, dgrad and wgrad as implicit GEMMs on the MFMA engine
// (any kernel size, stride, padding, dilation; NCHW or NHWC; groups = 1).
//
// Replaces the autograd node of torch::nn::Conv2d built by
// build_registered_layer(Owner&, const Conv2dDescriptor&, size_t) (reference
// layer/details/conv.hpp:140-191, module created at :177), i.e. ATen
// convolution and convolution_backward:
//   fwd  : y[n,k,p,q]  = b[k] + Σ_{c,r,s} w[k,c,r,s]·x[n,c,p·sh−ph+r·dh, q·sw−pw+s·dw]
//   dgrad: dx[n,c,h,w] = Σ_{k,r,s} w[k,c,r,s]·dy[n,k,(h+ph−r·dh)/sh,(w+pw−s·dw)/sw]
//          (terms whose division is inexact or out of range drop out)
//   wgrad: dw[k,c,r,s] = Σ_{n,p,q} dy[n,k,p,q]·x[n,c,p·sh−ph+r·dh, q·sw−pw+s·dw]
//   db[k]              = Σ_{n,p,q} dy[n,k,p,q]
// GEMM views: fwd M = n·p·q, N = k, K = c·r·s; dgrad M = n·h·w, N = c,
// K = k·r·s; wgrad M = k, N = c·r·s, K = n·p·q (split-K).  The 3×3 stride-1
// shapes that dominate the configs go to the specialised kernels in
// conv3x3.hip when they apply.
#include "gemm.hpp"
#include "conv_fast.hpp"

namespace {

using namespace nott::gemm;
using ::FastDiv;
using nott::ceil_div;

struct Geom {
    int32_t n, c, h, w, k, r, s, p, q;
    int32_t sh, sw, ph, pw, dh, dw;
    int32_t nhwc;
    FastDiv fd_pq, fd_q, fd_rs, fd_s, fd_hw, fd_w, fd_sh, fd_sw, fd_c;
};

Geom make_geom(const nott_conv2d_desc* d, int64_t p, int64_t q) {
    Geom g;
    g.n = (int32_t)d->n; g.c = (int32_t)d->c; g.h = (int32_t)d->h; g.w = (int32_t)d->w;
    g.k = (int32_t)d->k; g.r = (int32_t)d->r; g.s = (int32_t)d->s; g.p = (int32_t)p; g.q = (int32_t)q;
    g.sh = (int32_t)d->stride_h; g.sw = (int32_t)d->stride_w; g.ph = (int32_t)d->pad_h; g.pw = (int32_t)d->pad_w;
    g.dh = (int32_t)d->dil_h; g.dw = (int32_t)d->dil_w;
    g.nhwc = d->layout == NOTT_NHWC;
    g.fd_pq = FastDiv((uint32_t)(p * q));
    g.fd_q = FastDiv((uint32_t)q);
    g.fd_rs = FastDiv((uint32_t)(d->r * d->s));
    g.fd_s = FastDiv((uint32_t)d->s);
    g.fd_hw = FastDiv((uint32_t)(d->h * d->w));
    g.fd_w = FastDiv((uint32_t)d->w);
    g.fd_sh = FastDiv((uint32_t)d->stride_h);
    g.fd_sw = FastDiv((uint32_t)d->stride_w);
    g.fd_c = FastDiv((uint32_t)d->c);
    return g;
}

__device__ __forceinline__ int64_t x_index(const Geom& g, int32_t n, int32_t c, int32_t h, int32_t w) {
    return g.nhwc ? (((int64_t)n * g.h + h) * g.w + w) * g.c + c : (((int64_t)n * g.c + c) * g.h + h) * g.w + w;
}
__device__ __forceinline__ int64_t y_index(const Geom& g, int32_t n, int32_t k, int32_t p, int32_t q) {
    return g.nhwc ? (((int64_t)n * g.p + p) * g.q + q) * g.k + k : (((int64_t)n * g.k + k) * g.p + p) * g.q + q;
}

// fwd A: R(m = (n,p,q), kk = (c,r,s)) = x[n, c, p·sh−ph+r·dh, q·sw−pw+s·dw].
template <typename T>
struct FwdALoader {
    static constexpr bool kRowFast = true;
    static constexpr int E = KTraits<T>::kElemsPerChunk;
    const T* x;
    Geom g;
    int64_t rows, K;
    __device__ __forceinline__ u32x4 chunk(int64_t m, int64_t k0) const {
        T v[E];
        uint32_t n = 0, pq = 0, p = 0, q = 0;
        if (m < rows) {
            g.fd_pq.divmod((uint32_t)m, n, pq);
            g.fd_q.divmod(pq, p, q);
        }
        const int32_t h0 = (int32_t)p * g.sh - g.ph, w0 = (int32_t)q * g.sw - g.pw;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            T val = T(0);
            const int64_t kk = k0 + e;
            if (m < rows && kk < K) {
                uint32_t c, rs, r, s;
                g.fd_rs.divmod((uint32_t)kk, c, rs);
                g.fd_s.divmod(rs, r, s);
                const int32_t h = h0 + (int32_t)r * g.dh, w = w0 + (int32_t)s * g.dw;
                if (h >= 0 && h < g.h && w >= 0 && w < g.w) val = x[x_index(g, n, c, h, w)];
            }
            v[e] = val;
        }
        return Pack<T>::make(v);
    }
};

// y[n,k,p,q] = acc + b[k]
template <typename T>
struct FwdStore {
    T* y;
    const float* b;
    Geom g;
    int64_t M;
    __device__ __forceinline__ void store(int64_t m, int64_t kout, float v) const {
        if (m >= M || kout >= g.k) return;
        uint32_t n, pq, p, q;
        g.fd_pq.divmod((uint32_t)m, n, pq);
        g.fd_q.divmod(pq, p, q);
        if (b) v += b[kout];
        Io<T>::st(y, y_index(g, n, (int32_t)kout, p, q), v);
    }
};

// dgrad A: R(m = (n,h,w), kk = (k,r,s)) = dy[n, k, p, q] when h+ph−r·dh = p·sh
// and w+pw−s·dw = q·sw exactly, with p, q in range; else 0.
template <typename T>
struct DgradALoader {
    static constexpr bool kRowFast = true;
    static constexpr int E = KTraits<T>::kElemsPerChunk;
    const T* dy;
    Geom g;
    int64_t rows, K;
    __device__ __forceinline__ u32x4 chunk(int64_t m, int64_t k0) const {
        T v[E];
        uint32_t n = 0, hw = 0, h = 0, w = 0;
        if (m < rows) {
            g.fd_hw.divmod((uint32_t)m, n, hw);
            g.fd_w.divmod(hw, h, w);
        }
#pragma unroll
        for (int e = 0; e < E; ++e) {
            T val = T(0);
            const int64_t kk = k0 + e;
            if (m < rows && kk < K) {
                uint32_t ko, rs, r, s;
                g.fd_rs.divmod((uint32_t)kk, ko, rs);
                g.fd_s.divmod(rs, r, s);
                const int32_t ph = (int32_t)h + g.ph - (int32_t)r * g.dh;
                const int32_t pw = (int32_t)w + g.pw - (int32_t)s * g.dw;
                if (ph >= 0 && pw >= 0) {
                    uint32_t p, remh, q, remw;
                    g.fd_sh.divmod((uint32_t)ph, p, remh);
                    g.fd_sw.divmod((uint32_t)pw, q, remw);
                    if (remh == 0 && remw == 0 && (int32_t)p < g.p && (int32_t)q < g.q)
                        val = dy[y_index(g, n, (int32_t)ko, p, q)];
                }
            }
            v[e] = val;
        }
        return Pack<T>::make(v);
    }
};

// dgrad B: R(row = c, kk = (k,r,s)) = w[k, c, r, s].
template <typename T>
struct DgradBLoader {
    static constexpr bool kRowFast = true;
    static constexpr int E = KTraits<T>::kElemsPerChunk;
    const T* w;
    Geom g;
    int64_t rows, K;
    __device__ __forceinline__ u32x4 chunk(int64_t c, int64_t k0) const {
        T v[E];
        const int32_t rs_total = g.r * g.s;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const int64_t kk = k0 + e;
            T val = T(0);
            if (c < rows && kk < K) {
                uint32_t ko, rs;
                g.fd_rs.divmod((uint32_t)kk, ko, rs);
                val = w[((int64_t)ko * g.c + c) * rs_total + rs];
            }
            v[e] = val;
        }
        return Pack<T>::make(v);
    }
};

template <typename T>
struct DgradStore {
    T* dx;
    Geom g;
    int64_t M;
    __device__ __forceinline__ void store(int64_t m, int64_t c, float v) const {
        if (m >= M || c >= g.c) return;
        uint32_t n, hw, h, w;
        g.fd_hw.divmod((uint32_t)m, n, hw);
        g.fd_w.divmod(hw, h, w);
        Io<T>::st(dx, x_index(g, n, (int32_t)c, h, w), v);
    }
};

// wgrad A: R(row = k, kk = (n,p,q)) = dy[n, k, p, q].
template <typename T>
struct WgradALoader {
    static constexpr bool kRowFast = false;
    static constexpr int E = KTraits<T>::kElemsPerChunk;
    const T* dy;
    Geom g;
    int64_t rows, K;
    __device__ __forceinline__ u32x4 chunk(int64_t ko, int64_t k0) const {
        T v[E];
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const int64_t kk = k0 + e;
            T val = T(0);
            if (ko < rows && kk < K) {
                uint32_t n, pq, p, q;
                g.fd_pq.divmod((uint32_t)kk, n, pq);
                g.fd_q.divmod(pq, p, q);
                val = dy[y_index(g, n, (int32_t)ko, p, q)];
            }
            v[e] = val;
        }
        return Pack<T>::make(v);
    }
};

// wgrad B: R(row = (c,r,s), kk = (n,p,q)) = x[n, c, p·sh−ph+r·dh, q·sw−pw+s·dw].
template <typename T>
struct WgradBLoader {
    static constexpr bool kRowFast = false;
    static constexpr int E = KTraits<T>::kElemsPerChunk;
    const T* x;
    Geom g;
    int64_t rows, K;
    __device__ __forceinline__ u32x4 chunk(int64_t col, int64_t k0) const {
        T v[E];
        uint32_t c = 0, rs = 0, r = 0, s = 0;
        if (col < rows) {
            g.fd_rs.divmod((uint32_t)col, c, rs);
            g.fd_s.divmod(rs, r, s);
        }
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const int64_t kk = k0 + e;
            T val = T(0);
            if (col < rows && kk < K) {
                uint32_t n, pq, p, q;
                g.fd_pq.divmod((uint32_t)kk, n, pq);
                g.fd_q.divmod(pq, p, q);
                const int32_t h = (int32_t)p * g.sh - g.ph + (int32_t)r * g.dh;
                const int32_t w = (int32_t)q * g.sw - g.pw + (int32_t)s * g.dw;
                if (h >= 0 && h < g.h && w >= 0 && w < g.w) val = x[x_index(g, n, c, h, w)];
            }
            v[e] = val;
        }
        return Pack<T>::make(v);
    }
};

// dw[k][crs] fp32, row-major = KCRS.
struct WgradStore {
    float* dw;
    int64_t M, N;
    int accumulate;
    __device__ __forceinline__ void store(int64_t ko, int64_t crs, float v) const {
        if (ko >= M || crs >= N) return;
        float* p = dw + ko * N + crs;
        *p = accumulate ? *p + v : v;
    }
};

// db[k] = Σ_{n,p,q} dy[n,k,p,q] in two deterministic passes: workgroup
// (k, z) sums images [z·npb, (z+1)·npb) of channel k into part[z][k], then
// conv_db_finish_kernel adds the kDbSlabs partials of a channel.
constexpr int kDbSlabs = 32;
template <typename T>
__global__ __launch_bounds__(256) void conv_db_partial_kernel(const T* __restrict__ dy, Geom g, int32_t npb,
                                                              float* __restrict__ part) {
    __shared__ float red[4];
    const int32_t ko = blockIdx.x, z = blockIdx.y;
    const int64_t pq = (int64_t)g.p * g.q;
    const int32_t n0 = z * npb, n1 = min(g.n, n0 + npb);
    float s = 0.f;
    for (int32_t n = n0; n < n1; ++n) {
        for (int64_t i = threadIdx.x; i < pq; i += 256) {
            const int64_t idx = g.nhwc ? ((int64_t)n * pq + i) * g.k + ko : ((int64_t)n * g.k + ko) * pq + i;
            s += Io<T>::ld(dy, idx);
        }
    }
    s = block_sum<4>(s, red);
    if (threadIdx.x == 0) part[(int64_t)z * g.k + ko] = s;
}

// One wave per channel: lane z loads slab z's partial (all loads in flight
// at once), and the wave sums them in its fixed butterfly order.
__global__ __launch_bounds__(256) void conv_db_finish_kernel(const float* __restrict__ part, int32_t k,
                                                             float* __restrict__ db, int accumulate) {
    static_assert(kDbSlabs <= 64, "one partial per lane");
    const int32_t ko = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (ko >= k) return;
    const float s = wave_sum(lane < kDbSlabs ? part[(int64_t)lane * k + ko] : 0.f);
    if (lane == 0) db[ko] = accumulate ? db[ko] + s : s;
}

// ---------------------------------------------------------------------------
// Column path (bf16, NCHW) for the shapes the 3×3 stride-1 kernels do not
// take (strided, 1×1, 7×7 stem, small image widths): explicit column buffers
// and the fast bf16 GEMM, instead of element gathers inside the GEMM loads.
// With CRS = c·r·s padded to CRSp (a multiple of 64) and NPQ = n·p·q:
//   col[crs][npq]   = x[n, c, p·sh−ph+r·dh, q·sw−pw+s·dw]   (im2col, 0 outside)
//   dyt[k][npq]     = dy[n, k, p, q]                        (channel-major dy)
//   wp[k][crs]      = w[k, c, r, s]                          (zero-padded rows)
//   fwd  : y[n,k,pq]   = Σ_crs wp[k][crs]·col[crs][npq]      (GEMM M=k, N=npq)
//   wgrad: dw[k][crs]  = Σ_npq dyt[k][npq]·col[crs][npq]     (GEMM M=k, N=crs, K=npq)
//   dgrad: dcol[crs][npq] = Σ_k wp[k][crs]·dyt[k][npq], then
//          dx[n,c,h,w] = Σ_{r,s} dcol[(c,r,s)][(n, (h+ph−r·dh)/sh, (w+pw−s·dw)/sw)]
//          over the exact, in-range quotients (col2im as a gather: no atomics).
// ---------------------------------------------------------------------------
constexpr int64_t kColAlign = 256;
inline int64_t align_up(int64_t v, int64_t a) { return (v + a - 1) / a * a; }

template <typename T>
__global__ __launch_bounds__(256) void pack_w_kernel(const T* __restrict__ w, int32_t K, int32_t CRS, int32_t CRSp,
                                                     T* __restrict__ wp) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)K * CRSp) return;
    const int32_t k = (int32_t)(i / CRSp), j = (int32_t)(i % CRSp);
    wp[i] = j < CRS ? w[(int64_t)k * CRS + j] : T(0);
}

// One thread: one npq column position for kColRows consecutive crs rows, so
// that each load and each store of a wave covers 64 consecutive pixels.
constexpr int kColRows = 8;
template <typename T>
__global__ __launch_bounds__(256) void im2col_kernel(const T* __restrict__ x, Geom g, int32_t CRS, int32_t CRSp,
                                                     int32_t NPQ, T* __restrict__ col) {
    const int32_t m = (int32_t)((int64_t)blockIdx.x * 256 + threadIdx.x);
    if (m >= NPQ) return;
    const int32_t crs0 = (int32_t)blockIdx.y * kColRows;
    uint32_t n, pq, pp, qq;
    g.fd_pq.divmod((uint32_t)m, n, pq);
    g.fd_q.divmod(pq, pp, qq);
    const int32_t hb = (int32_t)pp * g.sh - g.ph, wb = (int32_t)qq * g.sw - g.pw;
    uint32_t c, rs, r, s;
    g.fd_rs.divmod((uint32_t)(crs0 < CRS ? crs0 : 0), c, rs);
    g.fd_s.divmod(rs, r, s);
    int32_t ci = (int32_t)c, ri = (int32_t)r, si = (int32_t)s;
#pragma unroll
    for (int e = 0; e < kColRows; ++e) {
        const int32_t crs = crs0 + e;
        T v = T(0);
        if (crs < CRS) {
            const int32_t h = hb + ri * g.dh, w = wb + si * g.dw;
            if (h >= 0 && h < g.h && w >= 0 && w < g.w) v = x[(((int64_t)n * g.c + ci) * g.h + h) * g.w + w];
        }
        col[(int64_t)crs * NPQ + m] = v;
        if (++si == g.s) {
            si = 0;
            if (++ri == g.r) {
                ri = 0;
                ++ci;
            }
        }
    }
}

// dyt[k][n·PQ + pq] = dy[n][k][pq]; one thread per 8 consecutive npq.
template <typename T>
__global__ __launch_bounds__(256) void to_kn_kernel(const T* __restrict__ dy, Geom g, int32_t NPQ, int vec,
                                                    T* __restrict__ dyt) {
    constexpr int E = 16 / (int)sizeof(T);
    const int32_t per_row = NPQ / E;
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= (int64_t)g.k * per_row) return;
    const int32_t k = (int32_t)(t / per_row), m0 = (int32_t)(t % per_row) * E;
    const int32_t PQ = g.p * g.q;
    T v[E];
    uint32_t n, pq;
    g.fd_pq.divmod((uint32_t)m0, n, pq);
    if (vec) {   // PQ % E == 0, 16-byte aligned dy: the E positions are one aligned run of one plane
        *reinterpret_cast<u32x4*>(dyt + (int64_t)k * NPQ + m0) =
            *reinterpret_cast<const u32x4*>(dy + ((int64_t)n * g.k + k) * PQ + pq);
        return;
    }
    int32_t ni = (int32_t)n, pqi = (int32_t)pq;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        v[e] = dy[((int64_t)ni * g.k + k) * PQ + pqi];
        if (++pqi == PQ) {
            pqi = 0;
            ++ni;
        }
    }
    *reinterpret_cast<u32x4*>(dyt + (int64_t)k * NPQ + m0) = Pack<T>::make(v);
}

// dx[n,c,h,w] = Σ over (r, s) whose source output position is exact and in range.
template <typename T>
__device__ __forceinline__ float col2im_at(const T* __restrict__ dcol, const Geom& g, int32_t NPQ, int64_t i) {
    uint32_t nc, hw, h, w, n, c;
    g.fd_hw.divmod((uint32_t)i, nc, hw);
    g.fd_w.divmod(hw, h, w);
    g.fd_c.divmod(nc, n, c);
    float acc = 0.f;
    for (int32_t r = 0; r < g.r; ++r) {
        const int32_t ph = (int32_t)h + g.ph - r * g.dh;
        if (ph < 0) break;
        uint32_t pp, remh;
        g.fd_sh.divmod((uint32_t)ph, pp, remh);
        if (remh != 0 || (int32_t)pp >= g.p) continue;
        for (int32_t s = 0; s < g.s; ++s) {
            const int32_t pw = (int32_t)w + g.pw - s * g.dw;
            if (pw < 0) break;
            uint32_t qq, remw;
            g.fd_sw.divmod((uint32_t)pw, qq, remw);
            if (remw != 0 || (int32_t)qq >= g.q) continue;
            const int64_t crs = ((int64_t)c * g.r + r) * g.s + s;
            acc += Io<T>::ld(dcol, crs * NPQ + ((int64_t)n * g.p + pp) * g.q + qq);
        }
    }
    return acc;
}

template <typename T>
__global__ __launch_bounds__(256) void col2im_kernel(const T* __restrict__ dcol, Geom g, int32_t NPQ, T* __restrict__ dx) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t total = (int64_t)g.n * g.c * g.h * g.w;
    if (i >= total) return;
    Io<T>::st(dx, i, col2im_at<T>(dcol, g, NPQ, i));
}

// Two horizontally adjacent outputs per thread (even image width): at stride
// 2 the two gather from neighbouring output columns, so consecutive lanes
// read consecutive columns of dcol; one 2-element store.
template <typename T>
__global__ __launch_bounds__(256) void col2im2_kernel(const T* __restrict__ dcol, Geom g, int32_t NPQ,
                                                      T* __restrict__ dx) {
    const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 2;
    const int64_t total = (int64_t)g.n * g.c * g.h * g.w;
    if (i >= total) return;
    const float a = col2im_at<T>(dcol, g, NPQ, i), b = col2im_at<T>(dcol, g, NPQ, i + 1);
    if constexpr (sizeof(T) == 2) {
        *reinterpret_cast<uint32_t*>(dx + i) = (uint32_t)f32_to_bf16(a) | ((uint32_t)f32_to_bf16(b) << 16);
    } else {
        *reinterpret_cast<float2*>(dx + i) = make_float2(a, b);
    }
}

// y[n, k, pq] = acc + b[k] for GEMM (m = k, n = npq).
template <typename T>
struct ColFwdStore {
    T* y;
    const float* b;
    Geom g;
    int64_t NPQ;
    __device__ __forceinline__ void store(int64_t k, int64_t m, float v) const {
        if (k >= g.k || m >= NPQ) return;
        uint32_t n, pq;
        g.fd_pq.divmod((uint32_t)m, n, pq);
        if (b) v += b[k];
        Io<T>::st(y, ((int64_t)n * g.k + k) * ((int64_t)g.p * g.q) + pq, v);
    }
};

struct ColPlan {
    int64_t CRS, CRSp, NPQ;
};

bool col_applies(const nott_conv2d_desc* d, int64_t p, int64_t q, bool need_k64) {
    const int64_t npq = d->n * p * q;
    return d->layout == NOTT_NCHW && npq % 64 == 0 && (!need_k64 || d->k % 64 == 0) &&
           d->c * d->r * d->s <= 65535 * 8 - 64;   // col rows per launch: grid.y = CRSp / 8
}

// Carves aligned pieces out of one workspace request.
struct Carve {
    int64_t off = 0;
    int64_t take(int64_t bytes) {
        const int64_t o = off;
        off = align_up(off + bytes, kColAlign);
        return o;
    }
};

// col[CRSp][NPQ]: consecutive lanes take consecutive columns (coalesced
// gathers from x), each thread kColRows rows.
void launch_im2col(nott_ctx ctx, const bf16_t* x, const Geom& g, int64_t CRS, int64_t CRSp, int64_t NPQ, bf16_t* col) {
    hipLaunchKernelGGL(im2col_kernel<bf16_t>, dim3((unsigned)ceil_div(NPQ, 256), (unsigned)(CRSp / kColRows)), dim3(256),
                       0, ctx->stream, x, g, (int32_t)CRS, (int32_t)CRSp, (int32_t)NPQ, col);
}

int col_fwd(nott_ctx ctx, const nott_conv2d_desc* d, int64_t p, int64_t q, const bf16_t* x, const bf16_t* w,
            const float* b, bf16_t* y) {
    const Geom g = make_geom(d, p, q);
    const int64_t CRS = d->c * d->r * d->s, CRSp = align_up(CRS, 64), NPQ = d->n * p * q;
    Carve cv;
    const int64_t o_wp = cv.take(2 * d->k * CRSp), o_col = cv.take(2 * CRSp * NPQ);
    const int64_t o_part = cv.take(4 * (int64_t)fast::partial_floats(ctx, d->k, NPQ, CRSp));
    char* ws = static_cast<char*>(nott::workspace(ctx, (size_t)cv.off));
    if (!ws) return NOTT_ERR_ALLOC;
    bf16_t* wp = reinterpret_cast<bf16_t*>(ws + o_wp);
    bf16_t* col = reinterpret_cast<bf16_t*>(ws + o_col);
    hipLaunchKernelGGL(pack_w_kernel<bf16_t>, dim3((unsigned)ceil_div(d->k * CRSp, 256)), dim3(256), 0, ctx->stream, w,
                       (int32_t)d->k, (int32_t)CRS, (int32_t)CRSp, wp);
    launch_im2col(ctx, x, g, CRS, CRSp, NPQ, col);
    ColFwdStore<bf16_t> ep{y, b, g, NPQ};
    return fast::run<false, true>(ctx, wp, CRSp, col, NPQ, ep, d->k, NPQ, CRSp, 0,
                                  reinterpret_cast<float*>(ws + o_part));
}

int col_wgrad(nott_ctx ctx, const nott_conv2d_desc* d, int64_t p, int64_t q, const bf16_t* x, const bf16_t* dy,
              float* dw, int accumulate) {
    const Geom g = make_geom(d, p, q);
    const int64_t CRS = d->c * d->r * d->s, CRSp = align_up(CRS, 64), NPQ = d->n * p * q;
    Carve cv;
    const int64_t o_dyt = cv.take(2 * d->k * NPQ), o_col = cv.take(2 * CRSp * NPQ);
    const int64_t o_part = cv.take(4 * (int64_t)fast::partial_floats(ctx, d->k, CRSp, NPQ));
    char* ws = static_cast<char*>(nott::workspace(ctx, (size_t)cv.off));
    if (!ws) return NOTT_ERR_ALLOC;
    bf16_t* dyt = reinterpret_cast<bf16_t*>(ws + o_dyt);
    bf16_t* col = reinterpret_cast<bf16_t*>(ws + o_col);
    hipLaunchKernelGGL(to_kn_kernel<bf16_t>, dim3((unsigned)ceil_div(d->k * (NPQ / 8), 256)), dim3(256), 0, ctx->stream,
                       dy, g, (int32_t)NPQ, (int)((p * q) % 8 == 0 && ((uintptr_t)dy % 16) == 0), dyt);
    launch_im2col(ctx, x, g, CRS, CRSp, NPQ, col);
    WgradStore ep{dw, d->k, CRS, accumulate};
    return fast::run<false, false>(ctx, dyt, NPQ, col, NPQ, ep, d->k, CRSp, NPQ, 0,
                                   reinterpret_cast<float*>(ws + o_part));
}

int col_dgrad(nott_ctx ctx, const nott_conv2d_desc* d, int64_t p, int64_t q, const bf16_t* dy, const bf16_t* w,
              bf16_t* dx) {
    const Geom g = make_geom(d, p, q);
    const int64_t CRS = d->c * d->r * d->s, CRSp = align_up(CRS, 64), NPQ = d->n * p * q;
    Carve cv;
    const int64_t o_wp = cv.take(2 * d->k * CRSp), o_dyt = cv.take(2 * d->k * NPQ), o_dcol = cv.take(2 * CRSp * NPQ);
    const int64_t o_part = cv.take(4 * (int64_t)fast::partial_floats(ctx, CRSp, NPQ, d->k));
    char* ws = static_cast<char*>(nott::workspace(ctx, (size_t)cv.off));
    if (!ws) return NOTT_ERR_ALLOC;
    bf16_t* wp = reinterpret_cast<bf16_t*>(ws + o_wp);
    bf16_t* dyt = reinterpret_cast<bf16_t*>(ws + o_dyt);
    bf16_t* dcol = reinterpret_cast<bf16_t*>(ws + o_dcol);
    hipLaunchKernelGGL(pack_w_kernel<bf16_t>, dim3((unsigned)ceil_div(d->k * CRSp, 256)), dim3(256), 0, ctx->stream, w,
                       (int32_t)d->k, (int32_t)CRS, (int32_t)CRSp, wp);
    hipLaunchKernelGGL(to_kn_kernel<bf16_t>, dim3((unsigned)ceil_div(d->k * (NPQ / 8), 256)), dim3(256), 0, ctx->stream,
                       dy, g, (int32_t)NPQ, (int)((p * q) % 8 == 0 && ((uintptr_t)dy % 16) == 0), dyt);
    RowMajorStore<bf16_t> ep{dcol, NPQ, CRSp, NPQ, nullptr, 0};
    const int st = fast::run<true, true>(ctx, wp, CRSp, dyt, NPQ, ep, CRSp, NPQ, d->k, 0,
                                         reinterpret_cast<float*>(ws + o_part));
    if (st != NOTT_OK) return st;
    if (d->w % 2 == 0 && ((uintptr_t)dx % 4) == 0)
        hipLaunchKernelGGL(col2im2_kernel<bf16_t>, dim3((unsigned)ceil_div(d->n * d->c * d->h * d->w / 2, 256)), dim3(256),
                           0, ctx->stream, dcol, g, (int32_t)NPQ, dx);
    else
        hipLaunchKernelGGL(col2im_kernel<bf16_t>, dim3((unsigned)ceil_div(d->n * d->c * d->h * d->w, 256)), dim3(256), 0,
                           ctx->stream, dcol, g, (int32_t)NPQ, dx);
    return nott::launch_status(ctx, "conv col2im");
}

int64_t out_size(int64_t in, int64_t k, int64_t s, int64_t p, int64_t d) { return (in + 2 * p - d * (k - 1) - 1) / s + 1; }

int check_desc(nott_ctx ctx, const nott_conv2d_desc* d, int64_t* p, int64_t* q) {
    NOTT_REQUIRE(ctx, d != nullptr, "conv2d: null descriptor");
    NOTT_REQUIRE(ctx, d->groups == 1, "conv2d: groups must be 1");
    NOTT_REQUIRE(ctx, d->layout == NOTT_NCHW || d->layout == NOTT_NHWC, "conv2d: bad layout");
    NOTT_REQUIRE(ctx, d->n >= 0 && d->c > 0 && d->h > 0 && d->w > 0 && d->k > 0 && d->r > 0 && d->s > 0,
                 "conv2d: bad shape");
    NOTT_REQUIRE(ctx, d->stride_h > 0 && d->stride_w > 0 && d->dil_h > 0 && d->dil_w > 0 && d->pad_h >= 0 &&
                          d->pad_w >= 0,
                 "conv2d: stride and dilation must be positive, padding non-negative");
    *p = out_size(d->h, d->r, d->stride_h, d->pad_h, d->dil_h);
    *q = out_size(d->w, d->s, d->stride_w, d->pad_w, d->dil_w);
    NOTT_REQUIRE(ctx, *p > 0 && *q > 0, "conv2d: kernel larger than padded input");
    // 32-bit index decompositions inside the kernels.
    const int64_t big = std::max<int64_t>({d->n * d->c * d->h * d->w, d->n * d->k * *p * *q, d->k * d->c * d->r * d->s,
                                           d->n * d->h * d->w, d->n * *p * *q});
    NOTT_REQUIRE(ctx, big < (int64_t(1) << 31), "conv2d: tensor too large for 32-bit indexing");
    return NOTT_OK;
}

// ---------------------------------------------------------------------------
// One input channel, 3×3, stride 1, pad 1, NCHW (the first conv of the
// configs[0] small CNN, conv.hpp:177 on a [n, 1, 28, 28] image): a GEMM with
// K = 9 is all overhead, so these are direct kernels.
//   fwd  : y[n, co, h, w] = b[co] + Σ_{r,s} x[n, 0, h+r−1, w+s−1] · wt[co, 0, r, s]
//   wgrad: dw[co, 0, r, s] = Σ_{n,h,w} dy[n, co, h, w] · x[n, 0, h+r−1, w+s−1]
//   db   : db[co] = Σ_{n,h,w} dy[n, co, h, w]  (a tenth sum of the same pass)
// wgrad is deterministic: workgroup (channel group, slab of images) writes
// 10 partial sums per channel, and a second pass adds the slabs in a fixed
// order (one wave per sum).
// ---------------------------------------------------------------------------
bool cin1_applies(const nott_conv2d_desc* d) {
    return d->layout == NOTT_NCHW && d->groups == 1 && d->c == 1 && d->r == 3 && d->s == 3 && d->stride_h == 1 &&
           d->stride_w == 1 && d->pad_h == 1 && d->pad_w == 1 && d->dil_h == 1 && d->dil_w == 1 && d->k <= 256 &&
           d->n * d->h * d->w < (int64_t(1) << 31);
}

// The 9 taps of x around pixel (h, w) of image plane xp (zero outside).
template <typename T>
__device__ __forceinline__ void cin1_taps(const T* __restrict__ xp, int32_t h, int32_t w, int32_t H, int32_t W,
                                          float (&t)[9]) {
#pragma unroll
    for (int r = 0; r < 3; ++r)
#pragma unroll
        for (int s = 0; s < 3; ++s) {
            const int32_t hh = h + r - 1, ww = w + s - 1;
            t[r * 3 + s] = (hh >= 0 && hh < H && ww >= 0 && ww < W) ? Io<T>::ld(xp, (int64_t)hh * W + ww) : 0.f;
        }
}

// Thread = one pixel for kCin1Co output channels (grid.y = channel group;
// the group's weights and bias in LDS).  Pixel indices are 32-bit
// (cin1_applies bounds n·h·w).
constexpr int kCin1Co = 8;
template <typename T>
__global__ __launch_bounds__(256) void cin1_fwd_kernel(const T* __restrict__ x, const T* __restrict__ wt,
                                                       const float* __restrict__ b, T* __restrict__ y, int32_t n,
                                                       int32_t H, int32_t W, int32_t k, int relu) {
    __shared__ float lw[kCin1Co * 9], lb[kCin1Co];
    const int co0 = blockIdx.y * kCin1Co;
    if (threadIdx.x < kCin1Co * 9) {
        const int co = co0 + (int)threadIdx.x / 9;
        lw[threadIdx.x] = co < k ? Io<T>::ld(wt, co0 * 9 + threadIdx.x) : 0.f;
    }
    if (threadIdx.x < kCin1Co) lb[threadIdx.x] = (b && co0 + (int)threadIdx.x < k) ? b[co0 + threadIdx.x] : 0.f;
    __syncthreads();
    const uint32_t hw = (uint32_t)H * (uint32_t)W;
    const uint32_t pix = blockIdx.x * 256u + threadIdx.x;
    if (pix >= (uint32_t)n * hw) return;
    const uint32_t img = pix / hw, in = pix - img * hw;
    const int32_t h = (int32_t)(in / (uint32_t)W), w = (int32_t)(in - (uint32_t)h * (uint32_t)W);
    float t[9];
    cin1_taps<T>(x + (int64_t)img * hw, h, w, H, W, t);
    T* yp = y + ((int64_t)img * k + co0) * hw + in;
#pragma unroll
    for (int c = 0; c < kCin1Co; ++c) {
        if (co0 + c >= k) break;
        float a = lb[c];
#pragma unroll
        for (int j = 0; j < 9; ++j) a = __builtin_fmaf(t[j], lw[c * 9 + j], a);
        Io<T>::st(yp, (int64_t)c * hw, relu ? relu_out(a) : a);
    }
}

constexpr int kCin1Slabs = 64;

// Workgroup (channel group, slab): for each of kCin1Co channels, 9 tap sums
// and Σ dy over the slab's images.  A thread gathers a pixel's 9 taps once
// and uses them for every channel of the group.
template <typename T>
__global__ __launch_bounds__(256) void cin1_wgrad_partial_kernel(const T* __restrict__ x, const T* __restrict__ dy,
                                                                 int32_t n, int32_t H, int32_t W, int32_t k,
                                                                 float* __restrict__ part) {
    __shared__ float red[4][kCin1Co * 10];
    const int co0 = blockIdx.x * kCin1Co, slab = blockIdx.y;
    const uint32_t hw = (uint32_t)H * (uint32_t)W;
    const int32_t per = (n + kCin1Slabs - 1) / kCin1Slabs;
    const int32_t n0 = slab * per, n1 = min(n, n0 + per);
    const int nco = min(kCin1Co, k - co0);
    float acc[kCin1Co][10];   // per channel: 9 taps, then Σ dy
#pragma unroll
    for (int c = 0; c < kCin1Co; ++c)
#pragma unroll
        for (int j = 0; j < 10; ++j) acc[c][j] = 0.f;
    for (int32_t img = n0; img < n1; ++img) {
        const T* xp = x + (int64_t)img * hw;
        const T* dp = dy + ((int64_t)img * k + co0) * hw;
        for (uint32_t in = threadIdx.x; in < hw; in += 256) {
            const int32_t h = (int32_t)(in / (uint32_t)W), w = (int32_t)(in - (uint32_t)h * (uint32_t)W);
            float t[9];
            cin1_taps<T>(xp, h, w, H, W, t);
#pragma unroll
            for (int c = 0; c < kCin1Co; ++c) {
                const float g = c < nco ? Io<T>::ld(dp, (int64_t)c * hw + in) : 0.f;
#pragma unroll
                for (int j = 0; j < 9; ++j) acc[c][j] = __builtin_fmaf(g, t[j], acc[c][j]);
                acc[c][9] += g;
            }
        }
    }
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
#pragma unroll
    for (int c = 0; c < kCin1Co; ++c)
#pragma unroll
        for (int j = 0; j < 10; ++j) {
            const float v = wave_sum(acc[c][j]);
            if (lane == 0) red[wid][c * 10 + j] = v;
        }
    __syncthreads();
    if (threadIdx.x < nco * 10) {
        const int i = threadIdx.x, c = i / 10, j = i - c * 10;
        part[((int64_t)(co0 + c) * kCin1Slabs + slab) * 10 + j] = (red[0][i] + red[1][i]) + (red[2][i] + red[3][i]);
    }
}

// One wave per output (co·10 + j, j a tap or 9 for the bias): lane z loads
// slab z's partial and the wave sums them in its fixed butterfly order.
__global__ __launch_bounds__(256) void cin1_wgrad_finish_kernel(const float* __restrict__ part, int32_t k,
                                                                float* __restrict__ dw, float* __restrict__ db,
                                                                int accumulate) {
    static_assert(kCin1Slabs <= 64, "one partial per lane");
    const int i = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (i >= k * 10) return;
    const int co = i / 10, j = i - co * 10;
    float* out = j < 9 ? (dw ? dw + co * 9 + j : nullptr) : (db ? db + co : nullptr);
    if (!out) return;
    const float s = wave_sum(lane < kCin1Slabs ? part[((int64_t)co * kCin1Slabs + lane) * 10 + j] : 0.f);
    if (lane == 0) *out = accumulate ? *out + s : s;
}

template <typename T>
int cin1_fwd(nott_ctx ctx, const nott_conv2d_desc* d, const T* x, const T* w, const float* b, T* y, int relu) {
    const int64_t pix = d->n * d->h * d->w;
    hipLaunchKernelGGL(cin1_fwd_kernel<T>, dim3((unsigned)nott::ceil_div(pix, 256), (unsigned)nott::ceil_div(d->k, (int64_t)kCin1Co)),
                       dim3(256), 0, ctx->stream, x, w, b, y, (int32_t)d->n, (int32_t)d->h, (int32_t)d->w,
                       (int32_t)d->k, relu);
    return nott::launch_status(ctx, "conv2d_fwd (1 input channel)");
}

template <typename T>
int cin1_wgrad(nott_ctx ctx, const nott_conv2d_desc* d, const T* x, const T* dy, float* dw, float* db,
               int accumulate) {
    float* part = static_cast<float*>(nott::workspace(ctx, sizeof(float) * (size_t)d->k * kCin1Slabs * 10));
    if (!part) return NOTT_ERR_ALLOC;
    hipLaunchKernelGGL(cin1_wgrad_partial_kernel<T>, dim3((unsigned)nott::ceil_div(d->k, (int64_t)kCin1Co), kCin1Slabs),
                       dim3(256), 0, ctx->stream, x, dy, (int32_t)d->n, (int32_t)d->h, (int32_t)d->w, (int32_t)d->k,
                       part);
    hipLaunchKernelGGL(cin1_wgrad_finish_kernel, dim3((unsigned)nott::ceil_div(d->k * 10, (int64_t)4)), dim3(256), 0,
                       ctx->stream, part, (int32_t)d->k, dw, db, accumulate);
    return nott::launch_status(ctx, "conv2d_bwd_weight (1 input channel)");
}

// Convolution without a fused activation (the paths whose epilogue has none).
template <typename T>
int fwd_plain(nott_ctx ctx, const nott_conv2d_desc* d, int64_t p, int64_t q, const void* x, const void* w,
              const float* b, void* y) {
    const Geom g = make_geom(d, p, q);
    const int64_t M = d->n * p * q, K = d->c * d->r * d->s;
    if constexpr (sizeof(T) == 2) {
        if (col_applies(d, p, q, false))
            return col_fwd(ctx, d, p, q, static_cast<const T*>(x), static_cast<const T*>(w), b, static_cast<T*>(y));
    }
    FwdALoader<T> la{static_cast<const T*>(x), g, M, K};
    const bool v = ((uintptr_t)w % 16) == 0 && ((K * (int64_t)sizeof(T)) % 16) == 0;
    RowKLoader<T> lb{static_cast<const T*>(w), K, d->k, K, v};
    FwdStore<T> ep{static_cast<T*>(y), b, g, M};
    return run<T>(ctx, la, lb, ep, M, d->k, K, 1);
}

// relu = 1: y = relu(conv(x) + b), fused into the 3×3 and single-channel
// epilogues, a separate in-place ReLU pass after the other paths.
template <typename T>
int fwd(nott_ctx ctx, const nott_conv2d_desc* d, int64_t p, int64_t q, const void* x, const void* w, const float* b,
        void* y, int relu) {
    if (nott::conv_fast::fwd_applies(d, sizeof(T)))
        return nott::conv_fast::fwd<T>(ctx, d, static_cast<const T*>(x), static_cast<const T*>(w), b,
                                       static_cast<T*>(y), relu);
    if (cin1_applies(d))
        return cin1_fwd<T>(ctx, d, static_cast<const T*>(x), static_cast<const T*>(w), b, static_cast<T*>(y), relu);
    if (nott::conv_fast::stem_fwd_applies(ctx, d))
        return nott::conv_fast::stem_fwd<T>(ctx, d, static_cast<const T*>(x), static_cast<const T*>(w), b,
                                            static_cast<T*>(y), relu);
    if (nott::conv_fast::tap_fwd_applies(ctx, d, sizeof(T)))
        return nott::conv_fast::tap_fwd<T>(ctx, d, static_cast<const T*>(x), static_cast<const T*>(w), b,
                                           static_cast<T*>(y), relu);
    const int st = fwd_plain<T>(ctx, d, p, q, x, w, b, y);
    if (st != NOTT_OK || !relu) return st;
    return nott_relu_fwd(ctx, sizeof(T) == 2 ? NOTT_BF16 : NOTT_F32, d->n * d->k * p * q, y, y);
}

template <typename T>
int dgrad(nott_ctx ctx, const nott_conv2d_desc* d, int64_t p, int64_t q, const void* dy, const void* w, void* dx) {
    if (nott::conv_fast::dgrad_applies(d, sizeof(T)))
        return nott::conv_fast::dgrad<T>(ctx, d, static_cast<const T*>(dy), static_cast<const T*>(w), static_cast<T*>(dx));
    if (nott::conv_fast::tap_dgrad_applies(ctx, d, sizeof(T)))
        return nott::conv_fast::tap_dgrad<T>(ctx, d, static_cast<const T*>(dy), static_cast<const T*>(w),
                                             static_cast<T*>(dx));
    if constexpr (sizeof(T) == 2) {
        if (col_applies(d, p, q, true))
            return col_dgrad(ctx, d, p, q, static_cast<const T*>(dy), static_cast<const T*>(w), static_cast<T*>(dx));
    }
    const Geom g = make_geom(d, p, q);
    const int64_t M = d->n * d->h * d->w, K = d->k * d->r * d->s;
    DgradALoader<T> la{static_cast<const T*>(dy), g, M, K};
    DgradBLoader<T> lb{static_cast<const T*>(w), g, d->c, K};
    DgradStore<T> ep{static_cast<T*>(dx), g, M};
    return run<T>(ctx, la, lb, ep, M, d->c, K);
}

template <typename T>
int wgrad(nott_ctx ctx, const nott_conv2d_desc* d, int64_t p, int64_t q, const void* x, const void* dy, float* dw,
          float* db, int accumulate) {
    const Geom g = make_geom(d, p, q);
    if (dw) {
        int st;
        const bool aligned = ((uintptr_t)x % 16) == 0 && ((uintptr_t)dy % 16) == 0;
        if (aligned && nott::conv_fast::wgrad_applies(d, sizeof(T))) {
            st = nott::conv_fast::wgrad<T>(ctx, d, static_cast<const T*>(x), static_cast<const T*>(dy), dw, accumulate);
        } else if (nott::conv_fast::stem_wgrad_applies(ctx, d)) {
            st = nott::conv_fast::stem_wgrad<T>(ctx, d, static_cast<const T*>(x), static_cast<const T*>(dy), dw,
                                                accumulate);
        } else if (cin1_applies(d)) {
            // the bias gradient comes out of the same pass
            st = cin1_wgrad<T>(ctx, d, static_cast<const T*>(x), static_cast<const T*>(dy), dw, db, accumulate);
            db = nullptr;
        } else if (sizeof(T) == 2 && col_applies(d, p, q, false)) {
            st = col_wgrad(ctx, d, p, q, reinterpret_cast<const bf16_t*>(x), reinterpret_cast<const bf16_t*>(dy), dw,
                           accumulate);
        } else {
            const int64_t M = d->k, N = d->c * d->r * d->s, K = d->n * p * q;
            WgradALoader<T> la{static_cast<const T*>(dy), g, M, K};
            WgradBLoader<T> lb{static_cast<const T*>(x), g, N, K};
            WgradStore ep{dw, M, N, accumulate};
            st = run<T>(ctx, la, lb, ep, M, N, K);
        }
        if (st != NOTT_OK) return st;
    }
    if (db) {
        float* part = static_cast<float*>(nott::workspace(ctx, sizeof(float) * kDbSlabs * (size_t)d->k));
        if (!part) return NOTT_ERR_ALLOC;
        const int32_t npb = (int32_t)nott::ceil_div((int64_t)d->n, (int64_t)kDbSlabs);
        hipLaunchKernelGGL(conv_db_partial_kernel<T>, dim3((unsigned)d->k, kDbSlabs), dim3(256), 0, ctx->stream,
                           static_cast<const T*>(dy), g, npb, part);
        hipLaunchKernelGGL(conv_db_finish_kernel, dim3((unsigned)nott::ceil_div((int64_t)d->k, (int64_t)4)), dim3(256),
                           0, ctx->stream, part, (int32_t)d->k, db, accumulate);
        return nott::launch_status(ctx, "conv_db");
    }
    return NOTT_OK;
}

}  // namespace

extern "C" int nott_conv2d_fwd_act(nott_ctx ctx, const nott_conv2d_desc* d, nott_dtype dtype, const void* x,
                                   const void* w, const float* b, int relu, void* y) {
    NOTT_CHECK_CTX(ctx);
    NOTT_REQUIRE(ctx, nott::valid_dtype(dtype), "nott_conv2d_fwd: bad dtype");
    NOTT_REQUIRE(ctx, relu == 0 || relu == 1, "nott_conv2d_fwd_act: relu must be 0 or 1");
    int64_t p, q;
    int st = check_desc(ctx, d, &p, &q);
    if (st != NOTT_OK) return st;
    if (d->n == 0) return NOTT_OK;
    NOTT_REQUIRE(ctx, x && w && y, "nott_conv2d_fwd: null buffer");
    nott::DeviceScope scope(ctx->device);
    return dtype == NOTT_F32 ? fwd<float>(ctx, d, p, q, x, w, b, y, relu) : fwd<bf16_t>(ctx, d, p, q, x, w, b, y, relu);
}

extern "C" int nott_conv2d_fwd(nott_ctx ctx, const nott_conv2d_desc* d, nott_dtype dtype, const void* x, const void* w,
                               const float* b, void* y) {
    return nott_conv2d_fwd_act(ctx, d, dtype, x, w, b, 0, y);
}

extern "C" int nott_conv2d_bwd_data(nott_ctx ctx, const nott_conv2d_desc* d, nott_dtype dtype, const void* dy,
                                    const void* w, void* dx) {
    NOTT_CHECK_CTX(ctx);
    NOTT_REQUIRE(ctx, nott::valid_dtype(dtype), "nott_conv2d_bwd_data: bad dtype");
    int64_t p, q;
    int st = check_desc(ctx, d, &p, &q);
    if (st != NOTT_OK) return st;
    if (d->n == 0) return NOTT_OK;
    NOTT_REQUIRE(ctx, dy && w && dx, "nott_conv2d_bwd_data: null buffer");
    nott::DeviceScope scope(ctx->device);
    return dtype == NOTT_F32 ? dgrad<float>(ctx, d, p, q, dy, w, dx) : dgrad<bf16_t>(ctx, d, p, q, dy, w, dx);
}

// The 3×3 stride-1 pass a layer's forward and data gradient both take: its
// weights are re-laid out once per forward for both.
static bool prep_pair_applies(const nott_conv2d_desc* d, nott_dtype dtype) {
    const size_t e = dtype == NOTT_F32 ? 4 : 2;
    return nott::conv_fast::fwd_applies(d, e) && nott::conv_fast::dgrad_applies(d, e);
}

extern "C" int nott_conv2d_dgrad_prep_bytes(const nott_conv2d_desc* d, nott_dtype dtype, int64_t* bytes) {
    if (!d || !bytes || !nott::valid_dtype(dtype)) return NOTT_ERR_INVALID_ARG;
    *bytes = (d->n > 0 && d->groups == 1 && d->layout == NOTT_NCHW && prep_pair_applies(d, dtype))
                 ? nott::conv_fast::dgrad_prep_elems(d) * (dtype == NOTT_F32 ? 4 : 2)
                 : 0;
    return NOTT_OK;
}

extern "C" int nott_conv2d_fwd_prep(nott_ctx ctx, const nott_conv2d_desc* d, nott_dtype dtype, const void* x,
                                    const void* w, const float* b, int relu, void* y, void* wd) {
    NOTT_CHECK_CTX(ctx);
    NOTT_REQUIRE(ctx, nott::valid_dtype(dtype), "nott_conv2d_fwd_prep: bad dtype");
    NOTT_REQUIRE(ctx, relu == 0 || relu == 1, "nott_conv2d_fwd_prep: relu must be 0 or 1");
    int64_t p, q;
    int st = check_desc(ctx, d, &p, &q);
    if (st != NOTT_OK) return st;
    NOTT_REQUIRE(ctx, d->n > 0 && prep_pair_applies(d, dtype),
                 "nott_conv2d_fwd_prep: not a 3x3 stride-1 convolution with prepared data-gradient weights "
                 "(nott_conv2d_dgrad_prep_bytes gives 0)");
    NOTT_REQUIRE(ctx, x && w && y && wd, "nott_conv2d_fwd_prep: null buffer");
    NOTT_REQUIRE(ctx, ((uintptr_t)wd % 16) == 0, "nott_conv2d_fwd_prep: wd must be 16-byte aligned");
    nott::DeviceScope scope(ctx->device);
    if (dtype == NOTT_F32)
        return nott::conv_fast::fwd_prep<float>(ctx, d, static_cast<const float*>(x), static_cast<const float*>(w), b,
                                                static_cast<float*>(y), relu, static_cast<float*>(wd));
    return nott::conv_fast::fwd_prep<bf16_t>(ctx, d, static_cast<const bf16_t*>(x), static_cast<const bf16_t*>(w), b,
                                             static_cast<bf16_t*>(y), relu, static_cast<bf16_t*>(wd));
}

extern "C" int nott_conv2d_bwd_data_prepped(nott_ctx ctx, const nott_conv2d_desc* d, nott_dtype dtype, const void* dy,
                                            const void* wd, void* dx) {
    NOTT_CHECK_CTX(ctx);
    NOTT_REQUIRE(ctx, nott::valid_dtype(dtype), "nott_conv2d_bwd_data_prepped: bad dtype");
    int64_t p, q;
    int st = check_desc(ctx, d, &p, &q);
    if (st != NOTT_OK) return st;
    NOTT_REQUIRE(ctx, d->n > 0 && prep_pair_applies(d, dtype),
                 "nott_conv2d_bwd_data_prepped: not a convolution nott_conv2d_fwd_prep prepares");
    NOTT_REQUIRE(ctx, dy && wd && dx, "nott_conv2d_bwd_data_prepped: null buffer");
    nott::DeviceScope scope(ctx->device);
    if (dtype == NOTT_F32)
        return nott::conv_fast::dgrad_prepared<float>(ctx, d, static_cast<const float*>(dy), static_cast<const float*>(wd),
                                                      static_cast<float*>(dx));
    return nott::conv_fast::dgrad_prepared<bf16_t>(ctx, d, static_cast<const bf16_t*>(dy),
                                                   static_cast<const bf16_t*>(wd), static_cast<bf16_t*>(dx));
}

extern "C" int nott_conv2d_bwd_weight(nott_ctx ctx, const nott_conv2d_desc* d, nott_dtype dtype, const void* x,
                                      const void* dy, float* dw, float* db, int accumulate) {
    NOTT_CHECK_CTX(ctx);
    NOTT_REQUIRE(ctx, nott::valid_dtype(dtype), "nott_conv2d_bwd_weight: bad dtype");
    int64_t p, q;
    int st = check_desc(ctx, d, &p, &q);
    if (st != NOTT_OK) return st;
    nott::DeviceScope scope(ctx->device);
    if (d->n == 0) {
        if (!accumulate) {
            if (dw && nott_zero(ctx, (int64_t)sizeof(float) * d->k * d->c * d->r * d->s, dw) != NOTT_OK) return NOTT_ERR_HIP;
            if (db && nott_zero(ctx, (int64_t)sizeof(float) * d->k, db) != NOTT_OK) return NOTT_ERR_HIP;
        }
        return NOTT_OK;
    }
    NOTT_REQUIRE(ctx, dy && (!dw || x), "nott_conv2d_bwd_weight: null buffer");
    return dtype == NOTT_F32 ? wgrad<float>(ctx, d, p, q, x, dy, dw, db, accumulate)
                             : wgrad<bf16_t>(ctx, d, p, q, x, dy, dw, db, accumulate);
}
