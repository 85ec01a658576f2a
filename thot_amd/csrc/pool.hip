// MaxPool2d forward (values + int64 argmax) and backward (argmax routing), NCHW.
//
// Replaces torch::nn::MaxPool2d built by build_registered_layer(Owner&, const
// PoolingDescriptor&, size_t) (reference layer/details/pooling.hpp:132-149),
// i.e. ATen max_pool2d_with_indices and its backward.
//   forward : window scan rows-then-columns from the first in-bounds tap; the
//             index moves on a strictly greater value or on a NaN; argmax is
//             the flat index ih·w + iw inside the (n, c) plane.
//   backward: dx[argmax] += dy.  Computed as a gather: each input element
//             sums the dy of the windows that cover it and chose it, in
//             output scan order, so overlapping windows need no atomics and
//             the fp32 sum order equals the reference's scatter order.
#include "common.hpp"

#include <initializer_list>

namespace {

typedef long long i64x2 __attribute__((ext_vector_type(2)));

constexpr int kThreads = 256;
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

struct PoolGeom {
    int64_t h, w, oh, ow, kh, kw, sh, sw, ph, pw, dh, dw;
};

template <typename T>
__global__ __launch_bounds__(kThreads) void maxpool_fwd_kernel(const T* __restrict__ x, T* __restrict__ y,
                                                               int64_t* __restrict__ argmax, int64_t planes,
                                                               PoolGeom g) {
    const int64_t o = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    const int64_t per_plane = g.oh * g.ow;
    if (o >= planes * per_plane) return;
    const int64_t pl = o / per_plane;
    const int64_t rem = o - pl * per_plane;
    const int64_t oh = rem / g.ow, ow = rem - oh * g.ow;
    const T* xp = x + pl * g.h * g.w;
    int64_t ih0 = oh * g.sh - g.ph, iw0 = ow * g.sw - g.pw;
    const int64_t ih1 = std::min<int64_t>(ih0 + (g.kh - 1) * g.dh + 1, g.h);
    const int64_t iw1 = std::min<int64_t>(iw0 + (g.kw - 1) * g.dw + 1, g.w);
    while (ih0 < 0) ih0 += g.dh;
    while (iw0 < 0) iw0 += g.dw;
    int64_t best = ih0 * g.w + iw0;
    float bv = -INFINITY;
    for (int64_t ih = ih0; ih < ih1; ih += g.dh)
        for (int64_t iw = iw0; iw < iw1; iw += g.dw) {
            const float v = Io<T>::ld(xp, ih * g.w + iw);
            if (v > bv || v != v) {
                bv = v;
                best = ih * g.w + iw;
            }
        }
    Io<T>::st(y, o, bv);
    argmax[o] = best;
}

template <typename T>
__global__ __launch_bounds__(kThreads) void maxpool_bwd_kernel(const int64_t* __restrict__ argmax,
                                                               const T* __restrict__ dy, T* __restrict__ dx,
                                                               int64_t planes, PoolGeom g) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    const int64_t per_plane = g.h * g.w;
    if (i >= planes * per_plane) return;
    const int64_t pl = i / per_plane;
    const int64_t idx = i - pl * per_plane;
    const int64_t ih = idx / g.w, iw = idx - ih * g.w;
    // Output rows whose window can contain ih: oh·sh − ph ≤ ih ≤ oh·sh − ph + (kh−1)·dh.
    const int64_t num_h = ih + g.ph - (g.kh - 1) * g.dh;
    int64_t oh0 = num_h <= 0 ? 0 : (num_h + g.sh - 1) / g.sh;
    int64_t oh1 = std::min<int64_t>((ih + g.ph) / g.sh, g.oh - 1);
    const int64_t num_w = iw + g.pw - (g.kw - 1) * g.dw;
    int64_t ow0 = num_w <= 0 ? 0 : (num_w + g.sw - 1) / g.sw;
    int64_t ow1 = std::min<int64_t>((iw + g.pw) / g.sw, g.ow - 1);
    const int64_t* ap = argmax + pl * g.oh * g.ow;
    const T* gp = dy + pl * g.oh * g.ow;
    float acc = 0.f;
    for (int64_t oh = oh0; oh <= oh1; ++oh)
        for (int64_t ow = ow0; ow <= ow1; ++ow) {
            const int64_t o = oh * g.ow + ow;
            if (ap[o] == idx) acc += Io<T>::ld(gp, o);
        }
    Io<T>::st(dx, i, acc);
}

// 32-bit index versions (tensors below 2^31 elements, the common case):
// every division is a multiply-high by a precomputed reciprocal.
struct PoolGeom32 {
    int32_t h, w, oh, ow, kh, kw, sh, sw, ph, pw, dh, dw;
    FastDiv fd_out_plane, fd_ow, fd_in_plane, fd_w, fd_sh, fd_sw;
};

template <typename T>
__global__ __launch_bounds__(kThreads) void maxpool_fwd_kernel32(const T* __restrict__ x, T* __restrict__ y,
                                                                 int64_t* __restrict__ argmax, uint32_t total,
                                                                 PoolGeom32 g) {
    const uint32_t o = blockIdx.x * kThreads + threadIdx.x;
    if (o >= total) return;
    uint32_t pl, rem, oh, ow;
    g.fd_out_plane.divmod(o, pl, rem);
    g.fd_ow.divmod(rem, oh, ow);
    const T* xp = x + (int64_t)pl * g.h * g.w;
    int32_t ih0 = (int32_t)oh * g.sh - g.ph, iw0 = (int32_t)ow * g.sw - g.pw;
    const int32_t ih1 = min(ih0 + (g.kh - 1) * g.dh + 1, g.h);
    const int32_t iw1 = min(iw0 + (g.kw - 1) * g.dw + 1, g.w);
    while (ih0 < 0) ih0 += g.dh;
    while (iw0 < 0) iw0 += g.dw;
    int32_t best = ih0 * g.w + iw0;
    float bv = -INFINITY;
    for (int32_t ih = ih0; ih < ih1; ih += g.dh)
        for (int32_t iw = iw0; iw < iw1; iw += g.dw) {
            const float v = Io<T>::ld(xp, ih * g.w + iw);
            if (v > bv || v != v) {
                bv = v;
                best = ih * g.w + iw;
            }
        }
    Io<T>::st(y, o, bv);
    argmax[o] = best;
}

template <typename T>
__global__ __launch_bounds__(kThreads) void maxpool_bwd_kernel32(const int64_t* __restrict__ argmax,
                                                                 const T* __restrict__ dy, T* __restrict__ dx,
                                                                 uint32_t total, PoolGeom32 g) {
    const uint32_t i = blockIdx.x * kThreads + threadIdx.x;
    if (i >= total) return;
    uint32_t pl, idx, ih, iw;
    g.fd_in_plane.divmod(i, pl, idx);
    g.fd_w.divmod(idx, ih, iw);
    // Output rows whose window can contain ih: oh·sh − ph ≤ ih ≤ oh·sh − ph + (kh−1)·dh.
    const int32_t num_h = (int32_t)ih + g.ph - (g.kh - 1) * g.dh;
    const int32_t oh0 = num_h <= 0 ? 0 : (int32_t)g.fd_sh.div((uint32_t)(num_h + g.sh - 1));
    const int32_t oh1 = min((int32_t)g.fd_sh.div(ih + (uint32_t)g.ph), g.oh - 1);
    const int32_t num_w = (int32_t)iw + g.pw - (g.kw - 1) * g.dw;
    const int32_t ow0 = num_w <= 0 ? 0 : (int32_t)g.fd_sw.div((uint32_t)(num_w + g.sw - 1));
    const int32_t ow1 = min((int32_t)g.fd_sw.div(iw + (uint32_t)g.pw), g.ow - 1);
    const int64_t* ap = argmax + (int64_t)pl * g.oh * g.ow;
    const T* gp = dy + (int64_t)pl * g.oh * g.ow;
    float acc = 0.f;
    for (int32_t oh = oh0; oh <= oh1; ++oh)
        for (int32_t ow = ow0; ow <= ow1; ++ow) {
            const int32_t o = oh * g.ow + ow;
            if (ap[o] == (int64_t)idx) acc += Io<T>::ld(gp, o);
        }
    Io<T>::st(dx, i, acc);
}

// Row-tiled versions for the common case of whole planes of moderate width.
// Forward: workgroup (band of kPoolRows output rows, plane) stages the input
// rows its windows touch in LDS (one coalesced read of each row, converted to
// float), then every output scans its window from LDS in the same order and
// with the same NaN / first-maximum rule as the untiled kernel.
constexpr int kPoolRows = 8;
template <typename T, bool VEC>
__global__ __launch_bounds__(kThreads) void maxpool_fwd_tiled_kernel(const T* __restrict__ x, T* __restrict__ y,
                                                                     int64_t* __restrict__ argmax, PoolGeom32 g) {
    // VEC (w and ow multiples of 4, aligned buffers): 4 consecutive elements
    // per thread for the staging loads and for the y / argmax stores.
    constexpr int V = VEC ? 4 : 1;
    extern __shared__ float rows[];
    const int32_t pl = blockIdx.y;
    const int32_t oh0 = blockIdx.x * kPoolRows, oh1 = min(oh0 + kPoolRows, g.oh);
    const int32_t ih_lo = max(0, oh0 * g.sh - g.ph);
    const int32_t ih_hi = min(g.h, (oh1 - 1) * g.sh - g.ph + (g.kh - 1) * g.dh + 1);   // exclusive
    const T* xp = x + (int64_t)pl * g.h * g.w + (int64_t)ih_lo * g.w;
    const int32_t nin = (ih_hi - ih_lo) * g.w;
    if constexpr (VEC) {
        for (int32_t i = threadIdx.x; i < nin / 4; i += kThreads)
            reinterpret_cast<f32x4*>(rows)[i] = Vec4<T>::ld(xp + 4 * i);
    } else {
        for (int32_t i = threadIdx.x; i < nin; i += kThreads) rows[i] = Io<T>::ld(xp, i);
    }
    __syncthreads();
    const int32_t nout = (oh1 - oh0) * g.ow;
    for (int32_t j0 = threadIdx.x * V; j0 < nout; j0 += kThreads * V) {
      f32x4 yv;
      int64_t av[V];
#pragma unroll
      for (int e = 0; e < V; ++e) {
        const int32_t j = j0 + e;
        uint32_t ohl, owu;
        g.fd_ow.divmod((uint32_t)j, ohl, owu);
        const int32_t oh = oh0 + (int32_t)ohl, ow = (int32_t)owu;
        int32_t ih0 = oh * g.sh - g.ph, iw0 = ow * g.sw - g.pw;
        const int32_t ih1 = min(ih0 + (g.kh - 1) * g.dh + 1, g.h);
        const int32_t iw1 = min(iw0 + (g.kw - 1) * g.dw + 1, g.w);
        while (ih0 < 0) ih0 += g.dh;
        while (iw0 < 0) iw0 += g.dw;
        int32_t best = ih0 * g.w + iw0;
        float bv = -INFINITY;
        for (int32_t ih = ih0; ih < ih1; ih += g.dh)
            for (int32_t iw = iw0; iw < iw1; iw += g.dw) {
                const float v = rows[(ih - ih_lo) * g.w + iw];
                if (v > bv || v != v) {
                    bv = v;
                    best = ih * g.w + iw;
                }
            }
        yv[e] = bv;
        av[e] = best;
      }
      const int64_t o = ((int64_t)pl * g.oh + oh0) * g.ow + j0;
      if constexpr (VEC) {
        Vec4<T>::st(y + o, yv);
        // o is a multiple of 4: two 16-byte index stores
        i64x2* ap = reinterpret_cast<i64x2*>(argmax + o);
        ap[0] = i64x2{av[0], av[1]};
        ap[1] = i64x2{av[2], av[3]};
      } else {
        Io<T>::st(y, o, yv[0]);
        argmax[o] = av[0];
      }
    }
}

// Backward: workgroup (band of kPoolRows·sh input rows, plane) stages the
// argmax (as 32-bit in-plane indices) and dy of every output row whose window
// reaches the band in LDS, then each input gathers from the outputs that can
// cover it, in the untiled kernel's order (oh, then ow, ascending): the same
// sums, bit for bit, with each argmax read from HBM about once.
template <typename T, bool VEC>
__global__ __launch_bounds__(kThreads) void maxpool_bwd_tiled_kernel(const int64_t* __restrict__ argmax,
                                                                     const T* __restrict__ dy, T* __restrict__ dx,
                                                                     PoolGeom32 g, int32_t band_rows) {
    // VEC (w and ow multiples of 4, aligned buffers): 4 consecutive elements
    // per thread for the staging loads and for the dx stores.
    constexpr int V = VEC ? 4 : 1;
    extern __shared__ char sm[];
    const int32_t pl = blockIdx.y;
    const int32_t ih_lo = blockIdx.x * band_rows, ih_hi = min(ih_lo + band_rows, g.h);
    const int32_t num = ih_lo + g.ph - (g.kh - 1) * g.dh;
    const int32_t oh_lo = num <= 0 ? 0 : (num + g.sh - 1) / g.sh;
    const int32_t oh_hi = min((ih_hi - 1 + g.ph) / g.sh, g.oh - 1);
    const int32_t nout = oh_hi >= oh_lo ? (oh_hi - oh_lo + 1) * g.ow : 0;
    int32_t* code = reinterpret_cast<int32_t*>(sm);
    float* gv = reinterpret_cast<float*>(sm) + nout;
    const int64_t obase = (int64_t)pl * g.oh * g.ow + (int64_t)oh_lo * g.ow;
    if constexpr (VEC) {
        for (int32_t i = threadIdx.x; i < nout / 4; i += kThreads) {
            const f32x4 d4 = Vec4<T>::ld(dy + obase + 4 * i);
            const i64x2* ap = reinterpret_cast<const i64x2*>(argmax + obase + 4 * i);   // 16-byte index loads
            const i64x2 a01 = ap[0], a23 = ap[1];
            reinterpret_cast<f32x4*>(gv)[i] = d4;
            reinterpret_cast<i32x4*>(code)[i] = i32x4{(int32_t)a01.x, (int32_t)a01.y, (int32_t)a23.x, (int32_t)a23.y};
        }
    } else {
        for (int32_t i = threadIdx.x; i < nout; i += kThreads) {
            code[i] = (int32_t)argmax[obase + i];
            gv[i] = Io<T>::ld(dy, obase + i);
        }
    }
    __syncthreads();
    const int32_t nin = (ih_hi - ih_lo) * g.w;
    for (int32_t j0 = threadIdx.x * V; j0 < nin; j0 += kThreads * V) {
      f32x4 out;
#pragma unroll
      for (int e = 0; e < V; ++e) {
        const int32_t j = j0 + e;
        uint32_t ihl, iwu;
        g.fd_w.divmod((uint32_t)j, ihl, iwu);
        const int32_t ih = ih_lo + (int32_t)ihl, iw = (int32_t)iwu;
        const int32_t idx = ih * g.w + iw;
        const int32_t num_h = ih + g.ph - (g.kh - 1) * g.dh;
        const int32_t oh0 = num_h <= 0 ? 0 : (int32_t)g.fd_sh.div((uint32_t)(num_h + g.sh - 1));
        const int32_t oh1 = min((int32_t)g.fd_sh.div((uint32_t)(ih + g.ph)), g.oh - 1);
        const int32_t num_w = iw + g.pw - (g.kw - 1) * g.dw;
        const int32_t ow0 = num_w <= 0 ? 0 : (int32_t)g.fd_sw.div((uint32_t)(num_w + g.sw - 1));
        const int32_t ow1 = min((int32_t)g.fd_sw.div((uint32_t)(iw + g.pw)), g.ow - 1);
        float acc = 0.f;
        for (int32_t oh = oh0; oh <= oh1; ++oh)
            for (int32_t ow = ow0; ow <= ow1; ++ow) {
                const int32_t o = (oh - oh_lo) * g.ow + ow;
                if (code[o] == idx) acc += gv[o];
            }
        out[e] = acc;
      }
      const int64_t di = (int64_t)pl * g.h * g.w + (int64_t)ih_lo * g.w + j0;
      if constexpr (VEC) Vec4<T>::st(dx + di, out);
      else Io<T>::st(dx, di, out[0]);
    }
}

// The tiled kernels' 4-element path: image and output rows of whole 4-element
// groups, and 4-element groups of the given buffers aligned (8 bytes bf16,
// 16 bytes fp32).
bool vec4_ok(const PoolGeom& g, nott_dtype dtype, std::initializer_list<const void*> ptrs) {
    if (g.w % 4 != 0 || g.ow % 4 != 0) return false;
    const uintptr_t al = dtype == NOTT_F32 ? 16 : 8;
    for (const void* p : ptrs)
        if ((uintptr_t)p % al != 0) return false;
    return true;
}

// LDS bytes of the tiled kernels (0 when a band does not fit).
constexpr size_t kPoolLdsMax = 48 * 1024;
size_t pool_fwd_lds(const PoolGeom& g) {
    const int64_t rows = (int64_t)(kPoolRows - 1) * g.sh + (g.kh - 1) * g.dh + 1;
    const size_t b = sizeof(float) * (size_t)(std::min<int64_t>(rows, g.h) * g.w);
    return b <= kPoolLdsMax ? b : 0;
}
size_t pool_bwd_lds(const PoolGeom& g, int32_t band_rows) {
    const int64_t orows = (band_rows - 1 + (g.kh - 1) * g.dh) / g.sh + 2;
    const size_t b = 8 * (size_t)(std::min<int64_t>(orows, g.oh) * g.ow);
    return b <= kPoolLdsMax ? b : 0;
}

PoolGeom32 geom32(const PoolGeom& g) {
    PoolGeom32 r;
    r.h = (int32_t)g.h; r.w = (int32_t)g.w; r.oh = (int32_t)g.oh; r.ow = (int32_t)g.ow;
    r.kh = (int32_t)g.kh; r.kw = (int32_t)g.kw; r.sh = (int32_t)g.sh; r.sw = (int32_t)g.sw;
    r.ph = (int32_t)g.ph; r.pw = (int32_t)g.pw; r.dh = (int32_t)g.dh; r.dw = (int32_t)g.dw;
    r.fd_out_plane = FastDiv((uint32_t)(g.oh * g.ow));
    r.fd_ow = FastDiv((uint32_t)g.ow);
    r.fd_in_plane = FastDiv((uint32_t)(g.h * g.w));
    r.fd_w = FastDiv((uint32_t)g.w);
    r.fd_sh = FastDiv((uint32_t)g.sh);
    r.fd_sw = FastDiv((uint32_t)g.sw);
    return r;
}

// The 32-bit kernels apply when every flat index (and every window bound the
// scan forms) fits comfortably in int32.
bool fits32(int64_t planes, const PoolGeom& g) {
    const int64_t lim = int64_t(1) << 30;
    return planes * g.h * g.w < lim && planes * g.oh * g.ow < lim && g.h * g.w + g.kh * g.dh * g.w < lim;
}

int64_t pool_out(int64_t in, int64_t k, int64_t s, int64_t p, int64_t d, int ceil_mode) {
    int64_t num = in + 2 * p - d * (k - 1) - 1 + (ceil_mode ? s - 1 : 0);
    int64_t out = (num >= 0 ? num / s : -((-num + s - 1) / s)) + 1;
    if (ceil_mode && (out - 1) * s >= in + p) --out;
    return out;
}

int check_desc(nott_ctx ctx, const nott_pool2d_desc* d, PoolGeom* g) {
    NOTT_REQUIRE(ctx, d != nullptr, "pool: null descriptor");
    NOTT_REQUIRE(ctx, d->layout == NOTT_NCHW, "pool: only NCHW is supported");
    NOTT_REQUIRE(ctx, d->n >= 0 && d->c >= 0 && d->h > 0 && d->w > 0, "pool: bad input shape");
    NOTT_REQUIRE(ctx, d->kh > 0 && d->kw > 0 && d->stride_h > 0 && d->stride_w > 0 && d->dil_h > 0 && d->dil_w > 0,
                 "pool: kernel, stride and dilation must be positive");
    NOTT_REQUIRE(ctx, d->pad_h >= 0 && d->pad_w >= 0 && 2 * d->pad_h <= d->kh && 2 * d->pad_w <= d->kw,
                 "pool: pad should be at most half of the kernel size");
    g->h = d->h; g->w = d->w; g->kh = d->kh; g->kw = d->kw;
    g->sh = d->stride_h; g->sw = d->stride_w; g->ph = d->pad_h; g->pw = d->pad_w;
    g->dh = d->dil_h; g->dw = d->dil_w;
    g->oh = pool_out(d->h, d->kh, d->stride_h, d->pad_h, d->dil_h, d->ceil_mode);
    g->ow = pool_out(d->w, d->kw, d->stride_w, d->pad_w, d->dil_w, d->ceil_mode);
    NOTT_REQUIRE(ctx, g->oh > 0 && g->ow > 0, "pool: output size is too small");
    return NOTT_OK;
}

}  // namespace

extern "C" int nott_maxpool2d_fwd(nott_ctx ctx, const nott_pool2d_desc* d, nott_dtype dtype, const void* x, void* y,
                                  int64_t* argmax) {
    NOTT_CHECK_CTX(ctx);
    NOTT_REQUIRE(ctx, nott::valid_dtype(dtype), "nott_maxpool2d_fwd: bad dtype");
    PoolGeom g;
    int st = check_desc(ctx, d, &g);
    if (st != NOTT_OK) return st;
    const int64_t planes = d->n * d->c, total = planes * g.oh * g.ow;
    if (total == 0) return NOTT_OK;
    NOTT_REQUIRE(ctx, x && y && argmax, "nott_maxpool2d_fwd: null buffer");
    nott::DeviceScope scope(ctx->device);
    const dim3 grid((unsigned)nott::ceil_div(total, kThreads));
    const size_t flds = pool_fwd_lds(g);
    if (fits32(planes, g) && flds > 0 && planes <= 65535) {
        const PoolGeom32 g32 = geom32(g);
        const dim3 tgrid((unsigned)nott::ceil_div(g.oh, (int64_t)kPoolRows), (unsigned)planes);
        const bool vec = vec4_ok(g, dtype, {x, y}) && ((uintptr_t)argmax % 16) == 0;
        if (dtype == NOTT_F32 && vec)
            hipLaunchKernelGGL((maxpool_fwd_tiled_kernel<float, true>), tgrid, dim3(kThreads), flds, ctx->stream,
                               static_cast<const float*>(x), static_cast<float*>(y), argmax, g32);
        else if (dtype == NOTT_F32)
            hipLaunchKernelGGL((maxpool_fwd_tiled_kernel<float, false>), tgrid, dim3(kThreads), flds, ctx->stream,
                               static_cast<const float*>(x), static_cast<float*>(y), argmax, g32);
        else if (vec)
            hipLaunchKernelGGL((maxpool_fwd_tiled_kernel<bf16_t, true>), tgrid, dim3(kThreads), flds, ctx->stream,
                               static_cast<const bf16_t*>(x), static_cast<bf16_t*>(y), argmax, g32);
        else
            hipLaunchKernelGGL((maxpool_fwd_tiled_kernel<bf16_t, false>), tgrid, dim3(kThreads), flds, ctx->stream,
                               static_cast<const bf16_t*>(x), static_cast<bf16_t*>(y), argmax, g32);
    } else if (fits32(planes, g)) {
        const PoolGeom32 g32 = geom32(g);
        if (dtype == NOTT_F32)
            hipLaunchKernelGGL(maxpool_fwd_kernel32<float>, grid, dim3(kThreads), 0, ctx->stream,
                               static_cast<const float*>(x), static_cast<float*>(y), argmax, (uint32_t)total, g32);
        else
            hipLaunchKernelGGL(maxpool_fwd_kernel32<bf16_t>, grid, dim3(kThreads), 0, ctx->stream,
                               static_cast<const bf16_t*>(x), static_cast<bf16_t*>(y), argmax, (uint32_t)total, g32);
    } else if (dtype == NOTT_F32)
        hipLaunchKernelGGL(maxpool_fwd_kernel<float>, grid, dim3(kThreads), 0, ctx->stream,
                           static_cast<const float*>(x), static_cast<float*>(y), argmax, planes, g);
    else
        hipLaunchKernelGGL(maxpool_fwd_kernel<bf16_t>, grid, dim3(kThreads), 0, ctx->stream,
                           static_cast<const bf16_t*>(x), static_cast<bf16_t*>(y), argmax, planes, g);
    return nott::launch_status(ctx, "maxpool_fwd");
}

extern "C" int nott_maxpool2d_bwd(nott_ctx ctx, const nott_pool2d_desc* d, nott_dtype dtype, const int64_t* argmax,
                                  const void* dy, void* dx) {
    NOTT_CHECK_CTX(ctx);
    NOTT_REQUIRE(ctx, nott::valid_dtype(dtype), "nott_maxpool2d_bwd: bad dtype");
    PoolGeom g;
    int st = check_desc(ctx, d, &g);
    if (st != NOTT_OK) return st;
    const int64_t planes = d->n * d->c, total = planes * g.h * g.w;
    if (total == 0) return NOTT_OK;
    NOTT_REQUIRE(ctx, argmax && dy && dx, "nott_maxpool2d_bwd: null buffer");
    nott::DeviceScope scope(ctx->device);
    const dim3 grid((unsigned)nott::ceil_div(total, kThreads));
    const int32_t band_rows = (int32_t)(kPoolRows * g.sh);
    const size_t blds = pool_bwd_lds(g, band_rows);
    if (fits32(planes, g) && blds > 0 && planes <= 65535) {
        const PoolGeom32 g32 = geom32(g);
        const dim3 tgrid((unsigned)nott::ceil_div(g.h, (int64_t)band_rows), (unsigned)planes);
        const bool vec = vec4_ok(g, dtype, {dy, dx}) && ((uintptr_t)argmax % 16) == 0;
        if (dtype == NOTT_F32 && vec)
            hipLaunchKernelGGL((maxpool_bwd_tiled_kernel<float, true>), tgrid, dim3(kThreads), blds, ctx->stream,
                               argmax, static_cast<const float*>(dy), static_cast<float*>(dx), g32, band_rows);
        else if (dtype == NOTT_F32)
            hipLaunchKernelGGL((maxpool_bwd_tiled_kernel<float, false>), tgrid, dim3(kThreads), blds, ctx->stream,
                               argmax, static_cast<const float*>(dy), static_cast<float*>(dx), g32, band_rows);
        else if (vec)
            hipLaunchKernelGGL((maxpool_bwd_tiled_kernel<bf16_t, true>), tgrid, dim3(kThreads), blds, ctx->stream,
                               argmax, static_cast<const bf16_t*>(dy), static_cast<bf16_t*>(dx), g32, band_rows);
        else
            hipLaunchKernelGGL((maxpool_bwd_tiled_kernel<bf16_t, false>), tgrid, dim3(kThreads), blds, ctx->stream,
                               argmax, static_cast<const bf16_t*>(dy), static_cast<bf16_t*>(dx), g32, band_rows);
    } else if (fits32(planes, g)) {
        const PoolGeom32 g32 = geom32(g);
        if (dtype == NOTT_F32)
            hipLaunchKernelGGL(maxpool_bwd_kernel32<float>, grid, dim3(kThreads), 0, ctx->stream, argmax,
                               static_cast<const float*>(dy), static_cast<float*>(dx), (uint32_t)total, g32);
        else
            hipLaunchKernelGGL(maxpool_bwd_kernel32<bf16_t>, grid, dim3(kThreads), 0, ctx->stream, argmax,
                               static_cast<const bf16_t*>(dy), static_cast<bf16_t*>(dx), (uint32_t)total, g32);
    } else if (dtype == NOTT_F32)
        hipLaunchKernelGGL(maxpool_bwd_kernel<float>, grid, dim3(kThreads), 0, ctx->stream, argmax,
                           static_cast<const float*>(dy), static_cast<float*>(dx), planes, g);
    else
        hipLaunchKernelGGL(maxpool_bwd_kernel<bf16_t>, grid, dim3(kThreads), 0, ctx->stream, argmax,
                           static_cast<const bf16_t*>(dy), static_cast<bf16_t*>(dx), planes, g);
    return nott::launch_status(ctx, "maxpool_bwd");
}
