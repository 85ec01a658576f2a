// MaxPool2d forward (values + argmax) and backward (argmax routing), NCHW.
//
// Replaces torch::nn::MaxPool2d built by build_registered_layer(Owner&, const
// PoolingDescriptor&, size_t) (reference layer/details/pooling.hpp:132-149),
// i.e. ATen max_pool2d_with_indices and its backward.
//   forward : window scan rows-then-columns from the first in-bounds tap; the
//             index moves on a strictly greater value or on a NaN; argmax is
//             the flat index ih·w + iw inside the (n, c) plane (int64, ATen's
//             form), or the window tap ((ih − oh·sh + ph)/dh)·kw +
//             (iw − ow·sw + pw)/dw as one byte (the _tap entry points, for
//             callers that keep the indices to themselves; the backward turns
//             a tap back into the flat index, so both forms route identically).
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

// Argmax of output (oh, ow) whose maximum is input (bh, bw), stored as IX:
// int64_t = the flat index, uint8_t = the window tap.
template <typename IX, typename I, typename G>
__device__ __forceinline__ IX encode_ix(I bh, I bw, I oh, I ow, const G& g) {
    if constexpr (sizeof(IX) == 8) {
        return (IX)(bh * g.w + bw);
    } else {
        const I th = bh - (oh * g.sh - g.ph), tw = bw - (ow * g.sw - g.pw);
        return (IX)((g.dh == 1 ? th : th / g.dh) * g.kw + (g.dw == 1 ? tw : tw / g.dw));
    }
}
// The flat in-plane index a stored argmax of output (oh, ow) names.
template <typename I, typename IX, typename G>
__device__ __forceinline__ I decode_ix(IX code, I oh, I ow, const G& g) {
    if constexpr (sizeof(IX) == 8) {
        return (I)code;
    } else {
        const I t = (I)code, th = t / g.kw, tw = t - th * g.kw;
        return (oh * g.sh - g.ph + th * g.dh) * g.w + (ow * g.sw - g.pw + tw * g.dw);
    }
}

template <typename T, typename IX>
__global__ __launch_bounds__(kThreads) void maxpool_fwd_kernel(const T* __restrict__ x, T* __restrict__ y,
                                                               IX* __restrict__ argmax, int64_t planes,
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
    int64_t bh = ih0, bw = iw0;
    float bv = -INFINITY;
    for (int64_t ih = ih0; ih < ih1; ih += g.dh)
        for (int64_t iw = iw0; iw < iw1; iw += g.dw) {
            const float v = Io<T>::ld(xp, ih * g.w + iw);
            if (v > bv || v != v) {
                bv = v;
                bh = ih;
                bw = iw;
            }
        }
    Io<T>::st(y, o, bv);
    argmax[o] = encode_ix<IX>(bh, bw, oh, ow, g);
}

template <typename T, typename IX>
__global__ __launch_bounds__(kThreads) void maxpool_bwd_kernel(const IX* __restrict__ argmax,
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
    const IX* ap = argmax + pl * g.oh * g.ow;
    const T* gp = dy + pl * g.oh * g.ow;
    float acc = 0.f;
    for (int64_t oh = oh0; oh <= oh1; ++oh)
        for (int64_t ow = ow0; ow <= ow1; ++ow) {
            const int64_t o = oh * g.ow + ow;
            if (decode_ix<int64_t>(ap[o], oh, ow, g) == idx) acc += Io<T>::ld(gp, o);
        }
    Io<T>::st(dx, i, acc);
}

// 32-bit index versions (tensors below 2^31 elements, the common case):
// every division is a multiply-high by a precomputed reciprocal.
struct PoolGeom32 {
    int32_t h, w, oh, ow, kh, kw, sh, sw, ph, pw, dh, dw;
    FastDiv fd_out_plane, fd_ow, fd_in_plane, fd_w, fd_sh, fd_sw;
};

template <typename T, typename IX>
__global__ __launch_bounds__(kThreads) void maxpool_fwd_kernel32(const T* __restrict__ x, T* __restrict__ y,
                                                                 IX* __restrict__ argmax, uint32_t total,
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
    int32_t bh = ih0, bw = iw0;
    float bv = -INFINITY;
    for (int32_t ih = ih0; ih < ih1; ih += g.dh)
        for (int32_t iw = iw0; iw < iw1; iw += g.dw) {
            const float v = Io<T>::ld(xp, ih * g.w + iw);
            if (v > bv || v != v) {
                bv = v;
                bh = ih;
                bw = iw;
            }
        }
    Io<T>::st(y, o, bv);
    argmax[o] = encode_ix<IX>(bh, bw, (int32_t)oh, (int32_t)ow, g);
}

template <typename T, typename IX>
__global__ __launch_bounds__(kThreads) void maxpool_bwd_kernel32(const IX* __restrict__ argmax,
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
    const IX* ap = argmax + (int64_t)pl * g.oh * g.ow;
    const T* gp = dy + (int64_t)pl * g.oh * g.ow;
    float acc = 0.f;
    for (int32_t oh = oh0; oh <= oh1; ++oh)
        for (int32_t ow = ow0; ow <= ow1; ++ow) {
            const int32_t o = oh * g.ow + ow;
            if (decode_ix<int64_t>(ap[o], (int64_t)oh, (int64_t)ow, g) == (int64_t)idx) acc += Io<T>::ld(gp, o);
        }
    Io<T>::st(dx, i, acc);
}

// Row-tiled versions for the common case of whole planes of moderate width.
// Forward: workgroup (band of kPoolRows output rows, plane) stages the input
// rows its windows touch in LDS (one coalesced read of each row, converted to
// float), then every output scans its window from LDS in the same order and
// with the same NaN / first-maximum rule as the untiled kernel.
constexpr int kPoolRows = 8;
template <typename T, bool VEC, typename IX>
__global__ __launch_bounds__(kThreads) void maxpool_fwd_tiled_kernel(const T* __restrict__ x, T* __restrict__ y,
                                                                     IX* __restrict__ argmax, PoolGeom32 g) {
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
      IX av[V];
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
        int32_t bh = ih0, bw = iw0;
        float bv = -INFINITY;
        for (int32_t ih = ih0; ih < ih1; ih += g.dh)
            for (int32_t iw = iw0; iw < iw1; iw += g.dw) {
                const float v = rows[(ih - ih_lo) * g.w + iw];
                if (v > bv || v != v) {
                    bv = v;
                    bh = ih;
                    bw = iw;
                }
            }
        yv[e] = bv;
        av[e] = encode_ix<IX>(bh, bw, oh, ow, g);
      }
      const int64_t o = ((int64_t)pl * g.oh + oh0) * g.ow + j0;
      if constexpr (VEC) {
        Vec4<T>::st(y + o, yv);
        if constexpr (sizeof(IX) == 8) {
            // o is a multiple of 4: two 16-byte index stores
            i64x2* ap = reinterpret_cast<i64x2*>(argmax + o);
            ap[0] = i64x2{av[0], av[1]};
            ap[1] = i64x2{av[2], av[3]};
        } else {
            // four taps in one 4-byte store
            *reinterpret_cast<uint32_t*>(argmax + o) =
                (uint32_t)av[0] | ((uint32_t)av[1] << 8) | ((uint32_t)av[2] << 16) | ((uint32_t)av[3] << 24);
        }
      } else {
        Io<T>::st(y, o, yv[0]);
        argmax[o] = av[0];
      }
    }
}

// Backward through the ReLU whose output y is the pool's input (the ReLU
// backward's rule: zero where y <= 0), applied to V consecutive dx values
// before they are stored, so the result equals the two passes bit for bit.
template <typename T, int V>
__device__ __forceinline__ void relu_mask(const T* __restrict__ y, f32x4& out) {
    if constexpr (V == 4) {
        const f32x4 y4 = Vec4<T>::ld(y);
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (y4[e] <= 0.f) out[e] = 0.f;
    } else {
        if (Io<T>::ld(y, 0) <= 0.f) out[0] = 0.f;
    }
}

// Backward: workgroup (band of kPoolRows·sh input rows, plane) stages the
// argmax (as 32-bit in-plane indices) and dy of every output row whose window
// reaches the band in LDS, then each input gathers from the outputs that can
// cover it, in the untiled kernel's order (oh, then ow, ascending): the same
// sums, bit for bit, with each argmax read from HBM about once.
template <typename T, bool VEC, typename IX>
__global__ __launch_bounds__(kThreads) void maxpool_bwd_tiled_kernel(const IX* __restrict__ argmax,
                                                                     const T* __restrict__ dy, T* __restrict__ dx,
                                                                     const T* __restrict__ ry, PoolGeom32 g,
                                                                     int32_t band_rows) {
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
    if constexpr (VEC && sizeof(IX) == 8) {
        for (int32_t i = threadIdx.x; i < nout / 4; i += kThreads) {
            const f32x4 d4 = Vec4<T>::ld(dy + obase + 4 * i);
            const i64x2* ap = reinterpret_cast<const i64x2*>(argmax + obase + 4 * i);   // 16-byte index loads
            const i64x2 a01 = ap[0], a23 = ap[1];
            reinterpret_cast<f32x4*>(gv)[i] = d4;
            reinterpret_cast<i32x4*>(code)[i] = i32x4{(int32_t)a01.x, (int32_t)a01.y, (int32_t)a23.x, (int32_t)a23.y};
        }
    } else if constexpr (VEC) {
        // four taps per 4-byte load, staged as flat indices
        for (int32_t i = threadIdx.x; i < nout / 4; i += kThreads) {
            const f32x4 d4 = Vec4<T>::ld(dy + obase + 4 * i);
            const uint32_t t4 = *reinterpret_cast<const uint32_t*>(argmax + obase + 4 * i);
            uint32_t ohl, owu;
            g.fd_ow.divmod((uint32_t)(4 * i), ohl, owu);   // ow is a multiple of 4: one output row
            const int32_t oh = oh_lo + (int32_t)ohl, ow = (int32_t)owu;
            reinterpret_cast<f32x4*>(gv)[i] = d4;
            reinterpret_cast<i32x4*>(code)[i] =
                i32x4{decode_ix<int32_t>((uint8_t)t4, oh, ow, g), decode_ix<int32_t>((uint8_t)(t4 >> 8), oh, ow + 1, g),
                      decode_ix<int32_t>((uint8_t)(t4 >> 16), oh, ow + 2, g),
                      decode_ix<int32_t>((uint8_t)(t4 >> 24), oh, ow + 3, g)};
        }
    } else {
        for (int32_t i = threadIdx.x; i < nout; i += kThreads) {
            uint32_t ohl, owu;
            g.fd_ow.divmod((uint32_t)i, ohl, owu);
            code[i] = decode_ix<int32_t>(argmax[obase + i], oh_lo + (int32_t)ohl, (int32_t)owu, g);
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
      if (ry) relu_mask<T, V>(ry + di, out);
      if constexpr (VEC) Vec4<T>::st(dx + di, out);
      else Io<T>::st(dx, di, out[0]);
    }
}

// Stride-2, dilation-1, K×K windows with pad P ((K, P) = (3, 1), the
// ResNet-18 stem pool, or (2, 0)), image and output rows of whole 4-element
// groups.  The window geometry is compile-time: the scans unroll, and every
// division by the stride is a shift.
//
// Forward: workgroup = band of kS2Rows output rows of one plane.  The input
// rows the band's windows touch are staged in LDS as fp32 split by column
// parity (even columns, then odd columns, each half 16-byte aligned), so a
// thread's 4 consecutive outputs read each window row as one 16-byte run of
// even and one of odd columns (conflict-free), plus the odd column before
// them when K = 3.  Windows are scanned rows then columns from the first
// in-bounds tap with the generic kernels' rule (strictly greater, or NaN).
constexpr int kS2Rows = 16;
template <typename T, int K, int P, typename IX>
__global__ __launch_bounds__(kThreads) void maxpool_fwd_s2_kernel(const T* __restrict__ x, T* __restrict__ y,
                                                                  IX* __restrict__ argmax, PoolGeom32 g,
                                                                  int32_t half_pitch, const float* __restrict__ bn,
                                                                  int32_t nch) {
    static_assert((K == 3 && P == 1) || (K == 2 && P == 0), "window");
    extern __shared__ float rows[];   // [row][even columns | odd columns], 2·half_pitch floats a row
    const int32_t pl = blockIdx.y;
    const int32_t oh0 = blockIdx.x * kS2Rows, oh1 = min(oh0 + kS2Rows, g.oh);
    const int32_t ih_lo = max(0, 2 * oh0 - P);
    const int32_t ih_hi = min(g.h, 2 * (oh1 - 1) - P + K);   // exclusive
    const T* xp = x + (int64_t)pl * g.h * g.w;
    const int32_t nq = (ih_hi - ih_lo) * (g.w >> 2);
    // bn: the input is relu(a·x + c) of the BatchNorm before the pool, formed
    // here as that layer's apply pass forms and stores it (fma, ReLU with NaN
    // passing, rounding to T), so the window maxima and taps are the same
    float ba = 0.f, bc = 0.f;
    if (bn) {
        const int32_t ch = pl % nch;
        ba = bn[2 * ch];
        bc = bn[2 * ch + 1];
    }
    for (int32_t i = threadIdx.x; i < nq; i += kThreads) {
        uint32_t r, c;
        g.fd_w.divmod((uint32_t)(4 * i), r, c);
        f32x4 v = Vec4<T>::ld(xp + (int64_t)(ih_lo + (int32_t)r) * g.w + c);
        if (bn) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float z = __builtin_fmaf(v[e], ba, bc);
                z = (z > 0.f || z != z) ? z : 0.f;
                if constexpr (sizeof(T) == 2) z = bf16_to_f32(f32_to_bf16(z));
                v[e] = z;
            }
        }
        float* row = rows + r * 2 * half_pitch + (c >> 1);
        *reinterpret_cast<f32x2*>(row) = f32x2{v.x, v.z};
        *reinterpret_cast<f32x2*>(row + half_pitch) = f32x2{v.y, v.w};
    }
    __syncthreads();
    const int32_t ntask = (oh1 - oh0) * (g.ow >> 2);
    for (int32_t i = threadIdx.x; i < ntask; i += kThreads) {
        uint32_t orow, owu;
        g.fd_ow.divmod((uint32_t)(4 * i), orow, owu);
        const int32_t oh = oh0 + (int32_t)orow, ow0 = (int32_t)owu;
        float bv[4];
        int32_t bh[4], bw[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            bv[e] = -INFINITY;
            bh[e] = max(2 * oh - P, 0);
            bw[e] = max(2 * (ow0 + e) - P, 0);
        }
#pragma unroll
        for (int ky = 0; ky < K; ++ky) {
            const int32_t ih = 2 * oh - P + ky;
            if (ih < 0 || ih >= g.h) continue;
            const float* er = rows + (ih - ih_lo) * 2 * half_pitch;
            const f32x4 ev = *reinterpret_cast<const f32x4*>(er + ow0);
            const f32x4 od = *reinterpret_cast<const f32x4*>(er + half_pitch + ow0);
            const float od_m1 = (K == 3 && ow0 > 0) ? er[half_pitch + ow0 - 1] : -INFINITY;
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int kx = 0; kx < K; ++kx) {
                    // iw = 2·ow − P + kx: K = 3: odd[ow−1], even[ow], odd[ow]; K = 2: even[ow], odd[ow]
                    const int32_t iw = 2 * (ow0 + e) - P + kx;
                    if (iw < 0 || iw >= g.w) continue;
                    float v;
                    if constexpr (K == 3)
                        v = kx == 1 ? ev[e] : kx == 2 ? od[e] : (e == 0 ? od_m1 : od[e - 1]);
                    else
                        v = kx == 0 ? ev[e] : od[e];
                    if (v > bv[e] || v != v) {
                        bv[e] = v;
                        bh[e] = ih;
                        bw[e] = iw;
                    }
                }
        }
        const int64_t o = ((int64_t)pl * g.oh + oh) * g.ow + ow0;
        Vec4<T>::st(y + o, f32x4{bv[0], bv[1], bv[2], bv[3]});
        IX av[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) av[e] = encode_ix<IX>(bh[e], bw[e], oh, ow0 + e, g);
        if constexpr (sizeof(IX) == 8) {
            i64x2* ap = reinterpret_cast<i64x2*>(argmax + o);
            ap[0] = i64x2{av[0], av[1]};
            ap[1] = i64x2{av[2], av[3]};
        } else {
            *reinterpret_cast<uint32_t*>(argmax + o) =
                (uint32_t)av[0] | ((uint32_t)av[1] << 8) | ((uint32_t)av[2] << 16) | ((uint32_t)av[3] << 24);
        }
    }
}

// Backward of the same windows: workgroup = band of 2·kS2Rows input rows of
// one plane.  The dy and the argmax (as flat in-plane indices) of the output
// rows whose windows reach the band are staged in LDS.  Inputs 4q..4q+3 of
// row ih can only have been chosen by outputs 2q .. 2q+K−1 (fewer at the
// right edge) of output rows ceil((ih+P−K+1)/2) .. floor((ih+P)/2); a thread
// reads those as short runs and adds the matching dy in (oh, ow) order, the
// generic kernels' order, so the sums are the same bit for bit.
// The forward's z = a·x + c coefficients of a BatchNorm (a = γ·rstd,
// c = β − μ·a, unfused), from which its ReLU mask is recomputed.
__device__ __forceinline__ f32x2 bn_mask_coef(float g, float b, float mu, float rs) {
#pragma clang fp contract(off)
    const float a = g * rs;
    return f32x2{a, b - mu * a};
}

// The backward apply of a BatchNorm + ReLU whose output the pool took
// (x: the BatchNorm's input; abc: dx = A·g + B·x + C per channel from the
// BatchNorm backward's finalize; gamma, beta, mean, rstd: the ReLU mask's
// z = a·x + c, as the forward formed it).  x null: no epilogue.
template <typename T>
struct BnBwdEpi {
    const T* x;
    const float* abc;
    const float* gamma;
    const float* beta;
    const float* mean;
    const float* rstd;
    int32_t nch;
};

template <typename T, int K, int P, typename IX>
__global__ __launch_bounds__(kThreads) void maxpool_bwd_s2_kernel(const IX* __restrict__ argmax,
                                                                  const T* __restrict__ dy, T* __restrict__ dx,
                                                                  const T* __restrict__ ry, PoolGeom32 g,
                                                                  BnBwdEpi<T> epi = BnBwdEpi<T>{}) {
    static_assert((K == 3 && P == 1) || (K == 2 && P == 0), "window");
    constexpr int NC = K;   // candidate output columns of a 4-input group: 2q .. 2q + K − 1 (K ≤ 3)
    extern __shared__ char sm[];
    const int32_t pl = blockIdx.y;
    f32x4 eabc = f32x4{0.f, 0.f, 0.f, 0.f};
    f32x2 ez = f32x2{0.f, 0.f};
    if (epi.x) {
        const int32_t ch = pl % epi.nch;
        eabc = f32x4{epi.abc[3 * ch], epi.abc[3 * ch + 1], epi.abc[3 * ch + 2], 0.f};
        ez = bn_mask_coef(epi.gamma ? epi.gamma[ch] : 1.f, epi.beta ? epi.beta[ch] : 0.f, epi.mean[ch], epi.rstd[ch]);
    }
    const int32_t ih_lo = blockIdx.x * 2 * kS2Rows, ih_hi = min(ih_lo + 2 * kS2Rows, g.h);
    const int32_t oh_lo = max(0, (ih_lo + P - K + 2) >> 1);          // ceil((ih_lo + P − K + 1) / 2)
    const int32_t oh_hi = min(g.oh - 1, (ih_hi - 1 + P) >> 1);       // floor((ih_hi − 1 + P) / 2)
    const int32_t nor = oh_hi - oh_lo + 1;
    int32_t* code = reinterpret_cast<int32_t*>(sm);
    float* gv = reinterpret_cast<float*>(sm) + (nor > 0 ? nor : 0) * g.ow;
    const int64_t obase = (int64_t)pl * g.oh * g.ow + (int64_t)oh_lo * g.ow;
    const int32_t nout4 = nor > 0 ? nor * (g.ow >> 2) : 0;
    for (int32_t i = threadIdx.x; i < nout4; i += kThreads) {
        uint32_t orow, owu;
        g.fd_ow.divmod((uint32_t)(4 * i), orow, owu);
        const int32_t oh = oh_lo + (int32_t)orow, ow = (int32_t)owu;
        const f32x4 d4 = Vec4<T>::ld(dy + obase + 4 * i);
        i32x4 c4;
        if constexpr (sizeof(IX) == 8) {
            const i64x2* ap = reinterpret_cast<const i64x2*>(argmax + obase + 4 * i);
            const i64x2 a01 = ap[0], a23 = ap[1];
            c4 = i32x4{(int32_t)a01.x, (int32_t)a01.y, (int32_t)a23.x, (int32_t)a23.y};
        } else {
            const uint32_t t4 = *reinterpret_cast<const uint32_t*>(argmax + obase + 4 * i);
            c4 = i32x4{decode_ix<int32_t>((uint8_t)t4, oh, ow, g), decode_ix<int32_t>((uint8_t)(t4 >> 8), oh, ow + 1, g),
                       decode_ix<int32_t>((uint8_t)(t4 >> 16), oh, ow + 2, g),
                       decode_ix<int32_t>((uint8_t)(t4 >> 24), oh, ow + 3, g)};
        }
        reinterpret_cast<f32x4*>(gv)[i] = d4;
        reinterpret_cast<i32x4*>(code)[i] = c4;
    }
    __syncthreads();
    const int32_t ntask = (ih_hi - ih_lo) * (g.w >> 2);
    for (int32_t i = threadIdx.x; i < ntask; i += kThreads) {
        uint32_t rr, iwu;
        g.fd_w.divmod((uint32_t)(4 * i), rr, iwu);
        const int32_t ih = ih_lo + (int32_t)rr, iw0 = (int32_t)iwu, q2 = iw0 >> 1;
        const int32_t oa = max(0, (ih + P - K + 2) >> 1), ob = min(g.oh - 1, (ih + P) >> 1);
        float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int dr = 0; dr < 2; ++dr) {
            const int32_t oh = oa + dr;
            if (oh > ob) break;
            const int32_t* cr = code + (oh - oh_lo) * g.ow + q2;
            const float* gr = gv + (oh - oh_lo) * g.ow + q2;
            int32_t cc[NC];
            float gg[NC];
#pragma unroll
            for (int j = 0; j < NC; ++j) {
                const bool in = q2 + j < g.ow;
                cc[j] = in ? cr[j] : -1;
                gg[j] = in ? gr[j] : 0.f;
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int32_t idx = ih * g.w + iw0 + e;
#pragma unroll
                for (int j = 0; j < NC; ++j)
                    // output 2q + j's window columns are 4q + 2j − P .. 4q + 2j − P + K − 1
                    if (2 * j - P <= e && e <= 2 * j - P + K - 1 && cc[j] == idx) acc[e] += gg[j];
            }
        }
        const int64_t di = (int64_t)pl * g.h * g.w + (int64_t)ih * g.w + iw0;
        f32x4 out = f32x4{acc[0], acc[1], acc[2], acc[3]};
        if (ry) relu_mask<T, 4>(ry + di, out);
        if (epi.x) {
            // the routed gradient as the pool's backward would store it, then
            // the BatchNorm + ReLU backward's apply
            const f32x4 xv = Vec4<T>::ld(epi.x + di);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float gr = out[e];
                if constexpr (sizeof(T) == 2) gr = bf16_to_f32(f32_to_bf16(gr));
                if (__builtin_fmaf(xv[e], ez.x, ez.y) <= 0.f) gr = 0.f;
                out[e] = eabc.x * gr + eabc.y * xv[e] + eabc.z;
            }
        }
        Vec4<T>::st(dx + di, out);
    }
}

// The BatchNorm backward's partial sums Σ g and Σ g·(x − μ) over the gradient
// the pool's backward routes into a BatchNorm + ReLU output, taken over the
// pooled outputs instead of the routed plane: each output's dy goes to the
// input its tap names, masked where the BatchNorm's z = a·x + c <= 0.  Grid
// (channel, split), images [y·per_split, ..) of the split; each thread takes
// groups of 4 outputs of a row in a fixed order, then a fixed block tree, so
// the sums do not depend on timing.  Layout of the partials as the BatchNorm
// backward's reduce: partial[(ch·splits + split)·2 + {0, 1}].
template <typename T>
__global__ __launch_bounds__(kThreads) void maxpool_bwd_bn_reduce_kernel(const uint8_t* __restrict__ tap,
                                                                         const T* __restrict__ dy, PoolGeom32 g,
                                                                         BnBwdEpi<T> bn, int32_t n, int32_t per_split,
                                                                         FastDiv fd_pg, FastDiv fd_q,
                                                                         float* __restrict__ partial) {
    __shared__ float red[kThreads / 64];
    const int32_t ch = blockIdx.x;
    const int32_t n0 = (int32_t)blockIdx.y * per_split, n1 = min(n, n0 + per_split);
    const float mu = bn.mean[ch];
    const f32x2 z = bn_mask_coef(bn.gamma ? bn.gamma[ch] : 1.f, bn.beta ? bn.beta[ch] : 0.f, mu, bn.rstd[ch]);
    const int32_t oplane = g.oh * g.ow, iplane = g.h * g.w;
    const uint32_t items = (uint32_t)(n1 - n0) * (uint32_t)(oplane / 4);
    float s1 = 0.f, s2 = 0.f;
    for (uint32_t k = threadIdx.x; k < items; k += kThreads) {
        uint32_t i, j, r, q;
        fd_pg.divmod(k, i, j);
        fd_q.divmod(j, r, q);
        const int32_t pl = (n0 + (int32_t)i) * bn.nch + ch;
        const int32_t o = pl * oplane + 4 * (int32_t)j;   // row r, columns 4q .. 4q + 3
        const uint32_t t4 = *reinterpret_cast<const uint32_t*>(tap + o);
        const f32x4 gv = Vec4<T>::ld(dy + o);
        const T* xp = bn.x + (int64_t)pl * iplane;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int32_t p = decode_ix<int32_t>((uint8_t)(t4 >> (8 * e)), (int32_t)r, 4 * (int32_t)q + e, g);
            const float xv = Io<T>::ld(xp, p);
            const float gg = __builtin_fmaf(xv, z.x, z.y) <= 0.f ? 0.f : gv[e];
            s1 += gg;
            s2 += gg * (xv - mu);
        }
    }
    s1 = block_sum<kThreads / 64>(s1, red);
    s2 = block_sum<kThreads / 64>(s2, red);
    if (threadIdx.x == 0) {
        partial[((int64_t)ch * gridDim.y + blockIdx.y) * 2 + 0] = s1;
        partial[((int64_t)ch * gridDim.y + blockIdx.y) * 2 + 1] = s2;
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

namespace {

// Index alignment the 4-element tiled paths need: two 16-byte stores / loads
// of int64 indices, or one 4-byte word of taps.
template <typename IX>
constexpr uintptr_t ix_align() { return sizeof(IX) == 8 ? 16 : 4; }

// The stride-2 kernels' windows: 3×3 pad 1 or 2×2 pad 0, stride 2, dilation 1.
bool s2_geom(const PoolGeom& g) {
    return g.sh == 2 && g.sw == 2 && g.dh == 1 && g.dw == 1 && g.kh == g.kw && g.ph == g.pw &&
           ((g.kh == 3 && g.ph == 1) || (g.kh == 2 && g.ph == 0));
}
// Half row pitch (floats) of the forward's parity-split rows, and the LDS
// bytes of the two kernels (4 floats of slack past the last row).
int32_t s2_half_pitch(const PoolGeom& g) { return (int32_t)((g.w / 2 + 3) / 4 * 4); }
size_t s2_fwd_lds(const PoolGeom& g) {
    return sizeof(float) * ((size_t)std::min<int64_t>(g.h, 2 * kS2Rows + g.kh - 2) * 2 * s2_half_pitch(g) + 4);
}
size_t s2_bwd_lds(const PoolGeom& g) {
    return 2 * sizeof(float) * ((size_t)std::min<int64_t>(g.oh, kS2Rows + 2) * g.ow + 4);
}

// relu(a_c·x + c_c) of a BatchNorm's apply pass, per element (the fallback
// of the pools that form it while staging).
template <typename T>
__global__ __launch_bounds__(kThreads) void bnrelu_apply_kernel(const T* __restrict__ x, const float* __restrict__ coef,
                                                                int32_t nch, FastDiv fd_hw, T* __restrict__ y,
                                                                int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= n) return;
    const uint32_t plane = fd_hw.div((uint32_t)i);
    const int32_t ch = (int32_t)(plane % (uint32_t)nch);
    float z = __builtin_fmaf(Io<T>::ld(x, i), coef[2 * ch], coef[2 * ch + 1]);
    z = (z > 0.f || z != z) ? z : 0.f;
    Io<T>::st(y, i, z);
}

template <typename IX>
int maxpool_fwd_impl(nott_ctx ctx, const nott_pool2d_desc* d, nott_dtype dtype, const void* x, void* y, IX* argmax,
                     const char* name, const float* bn = nullptr) {
    NOTT_CHECK_CTX(ctx);
    NOTT_REQUIRE(ctx, nott::valid_dtype(dtype), std::string(name) + ": bad dtype");
    PoolGeom g;
    int st = check_desc(ctx, d, &g);
    if (st != NOTT_OK) return st;
    if (sizeof(IX) == 1)
        NOTT_REQUIRE(ctx, g.kh * g.kw <= 256, std::string(name) + ": a window of more than 256 taps needs int64 indices");
    const int64_t planes = d->n * d->c, total = planes * g.oh * g.ow;
    if (total == 0) return NOTT_OK;
    NOTT_REQUIRE(ctx, x && y && argmax, std::string(name) + ": null buffer");
    nott::DeviceScope scope(ctx->device);
    const dim3 grid((unsigned)nott::ceil_div(total, kThreads));
    const size_t flds = pool_fwd_lds(g);
    const auto* xf = static_cast<const float*>(x);
    const auto* xb = static_cast<const bf16_t*>(x);
    auto* yf = static_cast<float*>(y);
    auto* yb = static_cast<bf16_t*>(y);
    if (fits32(planes, g) && planes <= 65535 && s2_geom(g) && vec4_ok(g, dtype, {x, y}) &&
        ((uintptr_t)argmax % ix_align<IX>()) == 0 && s2_fwd_lds(g) <= kPoolLdsMax) {
        const PoolGeom32 g32 = geom32(g);
        const dim3 sgrid((unsigned)nott::ceil_div(g.oh, (int64_t)kS2Rows), (unsigned)planes);
        const size_t lds = s2_fwd_lds(g);
        const int32_t hp = s2_half_pitch(g);
        const int32_t nch = (int32_t)d->c;
        if (g.kh == 3 && dtype == NOTT_F32)
            hipLaunchKernelGGL((maxpool_fwd_s2_kernel<float, 3, 1, IX>), sgrid, dim3(kThreads), lds, ctx->stream, xf, yf,
                               argmax, g32, hp, bn, nch);
        else if (g.kh == 3)
            hipLaunchKernelGGL((maxpool_fwd_s2_kernel<bf16_t, 3, 1, IX>), sgrid, dim3(kThreads), lds, ctx->stream, xb,
                               yb, argmax, g32, hp, bn, nch);
        else if (dtype == NOTT_F32)
            hipLaunchKernelGGL((maxpool_fwd_s2_kernel<float, 2, 0, IX>), sgrid, dim3(kThreads), lds, ctx->stream, xf, yf,
                               argmax, g32, hp, bn, nch);
        else
            hipLaunchKernelGGL((maxpool_fwd_s2_kernel<bf16_t, 2, 0, IX>), sgrid, dim3(kThreads), lds, ctx->stream, xb,
                               yb, argmax, g32, hp, bn, nch);
    } else if (bn) {
        // other geometries: the BatchNorm's output formed in workspace, then
        // the pool
        const int64_t nx = planes * g.h * g.w;
        if (nx >= (int64_t(1) << 32))
            return nott::fail(ctx, NOTT_ERR_UNSUPPORTED, std::string(name) + ": tensor too large");
        void* tmp = nott::workspace(ctx, (size_t)nx * (dtype == NOTT_F32 ? 4 : 2));
        if (!tmp) return NOTT_ERR_ALLOC;
        const dim3 egrid((unsigned)nott::ceil_div(nx, kThreads));
        const FastDiv fd_hw((uint32_t)(g.h * g.w));
        if (dtype == NOTT_F32)
            hipLaunchKernelGGL((bnrelu_apply_kernel<float>), egrid, dim3(kThreads), 0, ctx->stream, xf, bn,
                               (int32_t)d->c, fd_hw, static_cast<float*>(tmp), nx);
        else
            hipLaunchKernelGGL((bnrelu_apply_kernel<bf16_t>), egrid, dim3(kThreads), 0, ctx->stream, xb, bn,
                               (int32_t)d->c, fd_hw, static_cast<bf16_t*>(tmp), nx);
        return maxpool_fwd_impl<IX>(ctx, d, dtype, tmp, y, argmax, name);
    } else if (fits32(planes, g) && flds > 0 && planes <= 65535) {
        const PoolGeom32 g32 = geom32(g);
        const dim3 tgrid((unsigned)nott::ceil_div(g.oh, (int64_t)kPoolRows), (unsigned)planes);
        const bool vec = vec4_ok(g, dtype, {x, y}) && ((uintptr_t)argmax % ix_align<IX>()) == 0;
        if (dtype == NOTT_F32 && vec)
            hipLaunchKernelGGL((maxpool_fwd_tiled_kernel<float, true, IX>), tgrid, dim3(kThreads), flds, ctx->stream, xf,
                               yf, argmax, g32);
        else if (dtype == NOTT_F32)
            hipLaunchKernelGGL((maxpool_fwd_tiled_kernel<float, false, IX>), tgrid, dim3(kThreads), flds, ctx->stream,
                               xf, yf, argmax, g32);
        else if (vec)
            hipLaunchKernelGGL((maxpool_fwd_tiled_kernel<bf16_t, true, IX>), tgrid, dim3(kThreads), flds, ctx->stream,
                               xb, yb, argmax, g32);
        else
            hipLaunchKernelGGL((maxpool_fwd_tiled_kernel<bf16_t, false, IX>), tgrid, dim3(kThreads), flds, ctx->stream,
                               xb, yb, argmax, g32);
    } else if (fits32(planes, g)) {
        const PoolGeom32 g32 = geom32(g);
        if (dtype == NOTT_F32)
            hipLaunchKernelGGL((maxpool_fwd_kernel32<float, IX>), grid, dim3(kThreads), 0, ctx->stream, xf, yf, argmax,
                               (uint32_t)total, g32);
        else
            hipLaunchKernelGGL((maxpool_fwd_kernel32<bf16_t, IX>), grid, dim3(kThreads), 0, ctx->stream, xb, yb, argmax,
                               (uint32_t)total, g32);
    } else if (dtype == NOTT_F32)
        hipLaunchKernelGGL((maxpool_fwd_kernel<float, IX>), grid, dim3(kThreads), 0, ctx->stream, xf, yf, argmax, planes,
                           g);
    else
        hipLaunchKernelGGL((maxpool_fwd_kernel<bf16_t, IX>), grid, dim3(kThreads), 0, ctx->stream, xb, yb, argmax,
                           planes, g);
    return nott::launch_status(ctx, name);
}

template <typename IX>
int maxpool_bwd_impl(nott_ctx ctx, const nott_pool2d_desc* d, nott_dtype dtype, const IX* argmax, const void* dy,
                     void* dx, const char* name, const void* relu_y = nullptr) {
    NOTT_CHECK_CTX(ctx);
    NOTT_REQUIRE(ctx, nott::valid_dtype(dtype), std::string(name) + ": bad dtype");
    PoolGeom g;
    int st = check_desc(ctx, d, &g);
    if (st != NOTT_OK) return st;
    if (sizeof(IX) == 1)
        NOTT_REQUIRE(ctx, g.kh * g.kw <= 256, std::string(name) + ": a window of more than 256 taps needs int64 indices");
    const int64_t planes = d->n * d->c, total = planes * g.h * g.w;
    if (total == 0) return NOTT_OK;
    NOTT_REQUIRE(ctx, argmax && dy && dx, std::string(name) + ": null buffer");
    nott::DeviceScope scope(ctx->device);
    const dim3 grid((unsigned)nott::ceil_div(total, kThreads));
    const int32_t band_rows = (int32_t)(kPoolRows * g.sh);
    const size_t blds = pool_bwd_lds(g, band_rows);
    const auto* df = static_cast<const float*>(dy);
    const auto* db = static_cast<const bf16_t*>(dy);
    auto* xf = static_cast<float*>(dx);
    auto* xb = static_cast<bf16_t*>(dx);
    const auto* rf = static_cast<const float*>(relu_y);
    const auto* rb = static_cast<const bf16_t*>(relu_y);
    bool fused = true;   // the tiled kernels apply relu_y themselves
    if (fits32(planes, g) && planes <= 65535 && s2_geom(g) && vec4_ok(g, dtype, {dy, dx, relu_y}) &&
        ((uintptr_t)argmax % ix_align<IX>()) == 0 && s2_bwd_lds(g) <= kPoolLdsMax) {
        const PoolGeom32 g32 = geom32(g);
        const dim3 sgrid((unsigned)nott::ceil_div(g.h, (int64_t)(2 * kS2Rows)), (unsigned)planes);
        const size_t lds = s2_bwd_lds(g);
        if (g.kh == 3 && dtype == NOTT_F32)
            hipLaunchKernelGGL((maxpool_bwd_s2_kernel<float, 3, 1, IX>), sgrid, dim3(kThreads), lds, ctx->stream, argmax,
                               df, xf, rf, g32);
        else if (g.kh == 3)
            hipLaunchKernelGGL((maxpool_bwd_s2_kernel<bf16_t, 3, 1, IX>), sgrid, dim3(kThreads), lds, ctx->stream,
                               argmax, db, xb, rb, g32);
        else if (dtype == NOTT_F32)
            hipLaunchKernelGGL((maxpool_bwd_s2_kernel<float, 2, 0, IX>), sgrid, dim3(kThreads), lds, ctx->stream, argmax,
                               df, xf, rf, g32);
        else
            hipLaunchKernelGGL((maxpool_bwd_s2_kernel<bf16_t, 2, 0, IX>), sgrid, dim3(kThreads), lds, ctx->stream,
                               argmax, db, xb, rb, g32);
    } else if (fits32(planes, g) && blds > 0 && planes <= 65535) {
        const PoolGeom32 g32 = geom32(g);
        const dim3 tgrid((unsigned)nott::ceil_div(g.h, (int64_t)band_rows), (unsigned)planes);
        const bool vec = vec4_ok(g, dtype, {dy, dx, relu_y}) && ((uintptr_t)argmax % ix_align<IX>()) == 0;
        if (dtype == NOTT_F32 && vec)
            hipLaunchKernelGGL((maxpool_bwd_tiled_kernel<float, true, IX>), tgrid, dim3(kThreads), blds, ctx->stream,
                               argmax, df, xf, rf, g32, band_rows);
        else if (dtype == NOTT_F32)
            hipLaunchKernelGGL((maxpool_bwd_tiled_kernel<float, false, IX>), tgrid, dim3(kThreads), blds, ctx->stream,
                               argmax, df, xf, rf, g32, band_rows);
        else if (vec)
            hipLaunchKernelGGL((maxpool_bwd_tiled_kernel<bf16_t, true, IX>), tgrid, dim3(kThreads), blds, ctx->stream,
                               argmax, db, xb, rb, g32, band_rows);
        else
            hipLaunchKernelGGL((maxpool_bwd_tiled_kernel<bf16_t, false, IX>), tgrid, dim3(kThreads), blds, ctx->stream,
                               argmax, db, xb, rb, g32, band_rows);
    } else if (fits32(planes, g)) {
        const PoolGeom32 g32 = geom32(g);
        fused = false;
        if (dtype == NOTT_F32)
            hipLaunchKernelGGL((maxpool_bwd_kernel32<float, IX>), grid, dim3(kThreads), 0, ctx->stream, argmax, df, xf,
                               (uint32_t)total, g32);
        else
            hipLaunchKernelGGL((maxpool_bwd_kernel32<bf16_t, IX>), grid, dim3(kThreads), 0, ctx->stream, argmax, db, xb,
                               (uint32_t)total, g32);
    } else {
        fused = false;
        if (dtype == NOTT_F32)
            hipLaunchKernelGGL((maxpool_bwd_kernel<float, IX>), grid, dim3(kThreads), 0, ctx->stream, argmax, df, xf,
                               planes, g);
        else
            hipLaunchKernelGGL((maxpool_bwd_kernel<bf16_t, IX>), grid, dim3(kThreads), 0, ctx->stream, argmax, db, xb,
                               planes, g);
    }
    // the untiled kernels take the ReLU's backward as a second, in-place pass
    if (relu_y && !fused) return nott_relu_bwd(ctx, dtype, total, relu_y, dx, dx);
    return nott::launch_status(ctx, name);
}

}  // namespace

extern "C" int nott_maxpool2d_fwd(nott_ctx ctx, const nott_pool2d_desc* d, nott_dtype dtype, const void* x, void* y,
                                  int64_t* argmax) {
    return maxpool_fwd_impl<int64_t>(ctx, d, dtype, x, y, argmax, "nott_maxpool2d_fwd");
}

extern "C" int nott_maxpool2d_bwd(nott_ctx ctx, const nott_pool2d_desc* d, nott_dtype dtype, const int64_t* argmax,
                                  const void* dy, void* dx) {
    return maxpool_bwd_impl<int64_t>(ctx, d, dtype, argmax, dy, dx, "nott_maxpool2d_bwd");
}

extern "C" int nott_maxpool2d_fwd_tap(nott_ctx ctx, const nott_pool2d_desc* d, nott_dtype dtype, const void* x,
                                      void* y, uint8_t* tap) {
    return maxpool_fwd_impl<uint8_t>(ctx, d, dtype, x, y, tap, "nott_maxpool2d_fwd_tap");
}

namespace nott {
// Whether the fused backward of a BatchNorm + ReLU + max-pool (the two
// functions below) takes this shape: stride-2 tap geometries on rows of whole
// 4-element groups, every buffer aligned for them.
bool maxpool_bnrelu_bwd_applies(const nott_pool2d_desc* d, nott_dtype dtype, const uint8_t* tap, const void* dy,
                                const void* x, const void* dx) {
    PoolGeom g;
    if (check_desc(nullptr, d, &g) != NOTT_OK) return false;
    const int64_t planes = d->n * d->c;
    return planes > 0 && fits32(planes, g) && planes <= 65535 && s2_geom(g) && vec4_ok(g, dtype, {dy, dx, x}) &&
           ((uintptr_t)tap % 4) == 0 && s2_bwd_lds(g) <= kPoolLdsMax;
}

// Its first pass: the BatchNorm backward's split partial sums, over the
// pooled outputs (images [s·per_split, ..) in split s of `splits`).
int maxpool_bwd_tap_bnrelu_reduce(nott_ctx ctx, const nott_pool2d_desc* d, nott_dtype dtype, const uint8_t* tap,
                                  const void* dy, const void* x, const float* gamma, const float* beta,
                                  const float* mean, const float* rstd, int32_t per_split, int32_t splits,
                                  float* partial) {
    PoolGeom g;
    int st = check_desc(ctx, d, &g);
    if (st != NOTT_OK) return st;
    nott::DeviceScope scope(ctx->device);
    const PoolGeom32 g32 = geom32(g);
    const FastDiv fd_pg((uint32_t)(g.oh * g.ow / 4)), fd_q((uint32_t)(g.ow / 4));
    const dim3 grid((unsigned)d->c, (unsigned)splits);
    auto go = [&](auto tv) {
        using T = decltype(tv);
        const BnBwdEpi<T> bn{static_cast<const T*>(x), nullptr, gamma, beta, mean, rstd, (int32_t)d->c};
        hipLaunchKernelGGL(maxpool_bwd_bn_reduce_kernel<T>, grid, dim3(kThreads), 0, ctx->stream, tap,
                           static_cast<const T*>(dy), g32, bn, (int32_t)d->n, per_split, fd_pg, fd_q, partial);
    };
    if (dtype == NOTT_F32) go(float{});
    else go(bf16_t{});
    return nott::launch_status(ctx, "maxpool_bwd_bn_reduce");
}

// Its last pass: the max-pool backward with the BatchNorm + ReLU backward's
// apply in its epilogue (abc: dx = A·g + B·x + C per channel).
int maxpool_bwd_tap_bnrelu_apply(nott_ctx ctx, const nott_pool2d_desc* d, nott_dtype dtype, const uint8_t* tap,
                                 const void* dy, const void* x, const float* abc, const float* gamma,
                                 const float* beta, const float* mean, const float* rstd, void* dx) {
    PoolGeom g;
    int st = check_desc(ctx, d, &g);
    if (st != NOTT_OK) return st;
    nott::DeviceScope scope(ctx->device);
    const PoolGeom32 g32 = geom32(g);
    const dim3 sgrid((unsigned)nott::ceil_div(g.h, (int64_t)(2 * kS2Rows)), (unsigned)(d->n * d->c));
    const size_t lds = s2_bwd_lds(g);
    auto go = [&](auto tv, auto kt) {
        using T = decltype(tv);
        constexpr int K = decltype(kt)::value, P = K == 3 ? 1 : 0;
        const BnBwdEpi<T> epi{static_cast<const T*>(x), abc, gamma, beta, mean, rstd, (int32_t)d->c};
        hipLaunchKernelGGL((maxpool_bwd_s2_kernel<T, K, P, uint8_t>), sgrid, dim3(kThreads), lds, ctx->stream, tap,
                           static_cast<const T*>(dy), static_cast<T*>(dx), nullptr, g32, epi);
    };
    if (dtype == NOTT_F32) {
        if (g.kh == 3) go(float{}, std::integral_constant<int, 3>{});
        else go(float{}, std::integral_constant<int, 2>{});
    } else {
        if (g.kh == 3) go(bf16_t{}, std::integral_constant<int, 3>{});
        else go(bf16_t{}, std::integral_constant<int, 2>{});
    }
    return nott::launch_status(ctx, "maxpool_bwd_bnrelu_apply");
}
}  // namespace nott

extern "C" int nott_maxpool2d_fwd_tap_bnrelu(nott_ctx ctx, const nott_pool2d_desc* d, nott_dtype dtype, const void* x,
                                             const float* coef, void* y, uint8_t* tap) {
    NOTT_CHECK_CTX(ctx);
    NOTT_REQUIRE(ctx, coef != nullptr, "nott_maxpool2d_fwd_tap_bnrelu: null coef");
    return maxpool_fwd_impl<uint8_t>(ctx, d, dtype, x, y, tap, "nott_maxpool2d_fwd_tap_bnrelu", coef);
}

extern "C" int nott_maxpool2d_bwd_tap(nott_ctx ctx, const nott_pool2d_desc* d, nott_dtype dtype, const uint8_t* tap,
                                      const void* dy, void* dx) {
    return maxpool_bwd_impl<uint8_t>(ctx, d, dtype, tap, dy, dx, "nott_maxpool2d_bwd_tap");
}

extern "C" int nott_maxpool2d_bwd_tap_relu(nott_ctx ctx, const nott_pool2d_desc* d, nott_dtype dtype,
                                           const uint8_t* tap, const void* dy, const void* y, void* dx) {
    NOTT_CHECK_CTX(ctx);
    NOTT_REQUIRE(ctx, y != nullptr, "nott_maxpool2d_bwd_tap_relu: null y");
    return maxpool_bwd_impl<uint8_t>(ctx, d, dtype, tap, dy, dx, "nott_maxpool2d_bwd_tap_relu", y);
}
