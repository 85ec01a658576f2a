// Specialised kernels for 3x3 / stride 1 / pad 1 / dilation 1 convolutions in
// NCHW (every 3x3 conv of the small CNN, of ResNet-18 outside the stage
// entries, and the standalone configs[1] conv).
//
// conv3x3_same_kernel computes
//   out[n, co, h, w] = b[co] + Σ_{ci,r,s} in[n, ci, h−1+r, w−1+s] · wt[co, ci, r, s]
// which is the forward conv (in = x, wt = w) and also the data gradient
// (in = dy, wt[c, k, r, s] = w[k, c, 2−r, 2−s]): reference conv.hpp:177,
// ATen convolution / convolution_backward (input grad).
//
// Implicit GEMM with M = pixels, N = output channels, K = input channels × 9
// taps.  A workgroup owns 256 consecutive pixels (linearised over n, h, w)
// and 64 output channels.  Per chunk of input channels (32 bf16 / 16 fp32 =
// 64 bytes) it stages in LDS:
//   * the input tile once, as [padded pixel][channel] rows: every image row
//     the tile touches plus one halo row above and below, each padded with a
//     zero column on both sides, so that each of the 9 taps is a plain row
//     offset ((r−1)·(W+2) + s−1) into the same LDS data and image borders read
//     zeros;
//   * the 9 × 64 × chunk weight slice, pre-arranged by conv3x3_wprep_kernel.
// Each wave then runs 9 taps × (4 pixel tiles × 4 channel tiles) of
// v_mfma_f32_16x16x32_bf16 (or 4× v_mfma_f32_16x16x4f32).  LDS rows are 64
// bytes with the 16-byte sub-chunks XOR-swizzled by row so that 16
// consecutive rows read by one MFMA operand hit distinct banks.
//
// conv3x3_wgrad_kernel computes dw[k, c, r, s] = Σ_{n,h,w} dy[n,k,h,w] ·
// x[n, c, h−1+r, w−1+s] (ATen convolution_backward, weight grad).
#include "conv_fast.hpp"

#include <algorithm>

namespace nott {
namespace conv_fast {
namespace {

constexpr int kThreads = 256;
constexpr int kTilePix = 256;       // pixels per workgroup (4 waves × 64)
constexpr int kTileCo = 64;         // output channels per workgroup
constexpr int kRowB = 64;           // bytes per LDS row (one channel chunk)

template <typename T> struct Chunk;
template <> struct Chunk<float> { static constexpr int CC = 16, SUB = 4; };   // channels per chunk / per 16 B
template <> struct Chunk<bf16_t> { static constexpr int CC = 32, SUB = 8; };

__device__ __forceinline__ int swz(int row) { return ((row >> 1) ^ (row >> 3)) & 3; }
__device__ __forceinline__ int lds_off(int row, int sub) { return row * kRowB + ((sub ^ swz(row)) << 4); }

struct SameParams {
    int32_t n, cin, h, w, cout;
    int32_t hw, w2;            // h·w, w+2
    int32_t npix;              // n·h·w
    int32_t in_rows;           // LDS rows reserved for the input tile
    int32_t remap;             // XCD-aware block remap active
    FastDiv fd_hw, fd_w, fd_w2, fd_h2;
};

// wt_prep[cb][cc][tap][co64][CC] from w (fwd) or from the flipped transpose (dgrad).
template <typename T, bool DGRAD>
__global__ __launch_bounds__(256) void conv3x3_wprep_kernel(const T* __restrict__ w, T* __restrict__ wp, int32_t cout,
                                                            int32_t cin) {
    constexpr int CC = Chunk<T>::CC;
    const int64_t total = (int64_t)cout * cin * 9;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= total) return;
    // decompose destination index
    const int32_t cil = (int32_t)(i % CC);
    int64_t rest = i / CC;
    const int32_t col = (int32_t)(rest % kTileCo);
    rest /= kTileCo;
    const int32_t tap = (int32_t)(rest % 9);
    rest /= 9;
    const int32_t ncc = cin / CC;
    const int32_t cc = (int32_t)(rest % ncc);
    const int32_t cb = (int32_t)(rest / ncc);
    const int32_t co = cb * kTileCo + col, ci = cc * CC + cil;
    const int32_t r = tap / 3, s = tap % 3;
    // fwd: wt[co][ci][r][s] = w[co][ci][r][s]; dgrad: wt[co=c][ci=k][r][s] = w[k][c][2-r][2-s]
    // (in dgrad terms w is [k = cin][c = cout][3][3]).
    const int64_t src = DGRAD ? (((int64_t)ci * cout + co) * 9 + (2 - r) * 3 + (2 - s))
                              : (((int64_t)co * cin + ci) * 9 + r * 3 + s);
    wp[i] = w[src];
}

template <typename T>
__device__ __forceinline__ u32x4 pack_sub(const T (&v)[Chunk<T>::SUB]);
template <>
__device__ __forceinline__ u32x4 pack_sub<float>(const float (&v)[4]) {
    return u32x4{__builtin_bit_cast(uint32_t, v[0]), __builtin_bit_cast(uint32_t, v[1]),
                 __builtin_bit_cast(uint32_t, v[2]), __builtin_bit_cast(uint32_t, v[3])};
}
template <>
__device__ __forceinline__ u32x4 pack_sub<bf16_t>(const bf16_t (&v)[8]) {
    return u32x4{(uint32_t)v[0] | ((uint32_t)v[1] << 16), (uint32_t)v[2] | ((uint32_t)v[3] << 16),
                 (uint32_t)v[4] | ((uint32_t)v[5] << 16), (uint32_t)v[6] | ((uint32_t)v[7] << 16)};
}

template <typename T>
__device__ __forceinline__ void mfma_chunk(const u32x4& a, const u32x4& b, f32x4& acc) {
    if constexpr (sizeof(T) == 2) {
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                      acc, 0, 0, 0);
    } else {
        const f32x4 af = __builtin_bit_cast(f32x4, a), bf = __builtin_bit_cast(f32x4, b);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(af.x, bf.x, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(af.y, bf.y, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(af.z, bf.z, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(af.w, bf.w, acc, 0, 0, 0);
    }
}

template <typename T>
__global__ __launch_bounds__(kThreads, 2) void conv3x3_same_kernel(const T* __restrict__ in, const T* __restrict__ wp,
                                                                  const float* __restrict__ bias, T* __restrict__ out,
                                                                  SameParams p) {
    constexpr int CC = Chunk<T>::CC, SUB = Chunk<T>::SUB;
    extern __shared__ __attribute__((aligned(16))) char smem[];
    char* lds_in = smem;
    char* lds_w = smem + p.in_rows * kRowB;

    // Block -> pixel tile.  Consecutive tiles share halo rows; with the
    // remap, tiles that run on the same XCD (block ids ≡ mod 8) are adjacent.
    int32_t tile = blockIdx.x;
    if (p.remap) tile = (int32_t)((blockIdx.x & 7) * (gridDim.x >> 3) + (blockIdx.x >> 3));
    const int32_t cb = blockIdx.y;
    const int32_t m0 = tile * kTilePix;
    const int32_t m_last = min(m0 + kTilePix, p.npix) - 1;

    uint32_t n0, hw0, h0, w0_;
    p.fd_hw.divmod((uint32_t)m0, n0, hw0);
    p.fd_w.divmod(hw0, h0, w0_);
    const int32_t v_lo = (int32_t)n0 * (p.h + 2) + (int32_t)h0;    // halo row above the first pixel
    uint32_t n1, hw1, h1, w1_;
    p.fd_hw.divmod((uint32_t)m_last, n1, hw1);
    p.fd_w.divmod(hw1, h1, w1_);
    const int32_t v_hi = (int32_t)n1 * (p.h + 2) + (int32_t)h1 + 2;  // halo row below the last pixel
    const int32_t nrows = (v_hi - v_lo + 1) * p.w2;                   // LDS rows used by this tile

    const int wid = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r16 = lane & 15, kq = lane >> 4;

    // This lane's LDS row (tap r=1, s=1) for each of its 4 pixel tiles.
    int32_t abase[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
        const int32_t m = min(m0 + wid * 64 + mt * 16 + r16, m_last);
        uint32_t n, hw, h, w;
        p.fd_hw.divmod((uint32_t)m, n, hw);
        p.fd_w.divmod(hw, h, w);
        const int32_t vrow = (int32_t)n * (p.h + 2) + (int32_t)h + 1;
        abase[mt] = (vrow - v_lo) * p.w2 + (int32_t)w + 1;
    }

    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int32_t nchunks = p.cin / CC;
    const T* wblk = wp + (int64_t)cb * nchunks * 9 * kTileCo * CC;
    for (int32_t cc = 0; cc < nchunks; ++cc) {
        // ---- stage the input tile: task = (LDS row, 16-byte sub-chunk) ----
        const int32_t ntask = nrows * 4;
        for (int32_t t = threadIdx.x; t < ntask; t += kThreads) {
            const int32_t sub = t / nrows;        // consecutive lanes -> consecutive pixels
            const int32_t row = t - sub * nrows;
            uint32_t vr, col;
            p.fd_w2.divmod((uint32_t)row, vr, col);
            uint32_t img, hh;
            p.fd_h2.divmod((uint32_t)(v_lo + (int32_t)vr), img, hh);
            const int32_t h = (int32_t)hh - 1, w = (int32_t)col - 1;
            T v[SUB];
            if (h >= 0 && h < p.h && w >= 0 && w < p.w && (int32_t)img < p.n) {
                const T* src = in + (((int64_t)img * p.cin + cc * CC + sub * SUB) * p.h + h) * p.w + w;
#pragma unroll
                for (int j = 0; j < SUB; ++j) v[j] = src[(int64_t)j * p.hw];
            } else {
#pragma unroll
                for (int j = 0; j < SUB; ++j) v[j] = T(0);
            }
            *reinterpret_cast<u32x4*>(lds_in + lds_off(row, sub)) = pack_sub<T>(v);
        }
        // ---- stage the weight slice: 9 taps × 64 co × 64 bytes ----
        const u32x4* wsrc = reinterpret_cast<const u32x4*>(wblk + (int64_t)cc * 9 * kTileCo * CC);
#pragma unroll
        for (int j = 0; j < (9 * kTileCo * 4) / kThreads; ++j) {
            const int t = threadIdx.x + j * kThreads;
            const int row = t >> 2, sub = t & 3;
            *reinterpret_cast<u32x4*>(lds_w + lds_off(row, sub)) = wsrc[t];
        }
        __syncthreads();
#pragma unroll
        for (int tap = 0; tap < 9; ++tap) {
            const int32_t toff = (tap / 3 - 1) * p.w2 + (tap % 3 - 1);
            u32x4 a[4], b[4];
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
                const int32_t row = abase[mt] + toff;
                a[mt] = *reinterpret_cast<const u32x4*>(lds_in + lds_off(row, kq));
            }
#pragma unroll
            for (int nt = 0; nt < 4; ++nt) {
                const int row = tap * kTileCo + nt * 16 + r16;
                b[nt] = *reinterpret_cast<const u32x4*>(lds_w + lds_off(row, kq));
            }
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                for (int nt = 0; nt < 4; ++nt) mfma_chunk<T>(a[mt], b[nt], acc[mt][nt]);
        }
        __syncthreads();
    }

    // ---- epilogue: lane holds column co = nt·16 + (lane % 16), pixels 4·(lane/16)+e ----
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
        const int32_t co = cb * kTileCo + nt * 16 + r16;
        const float bv = bias ? bias[co] : 0.f;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int32_t m = m0 + wid * 64 + mt * 16 + kq * 4 + e;
                if (m <= m_last) {
                    uint32_t n, hw;
                    p.fd_hw.divmod((uint32_t)m, n, hw);
                    Io<T>::st(out, ((int64_t)n * p.cout + co) * p.hw + hw, acc[mt][nt][e] + bv);
                }
            }
        }
    }
}

bool same_shape(const nott_conv2d_desc* d) {
    return d->layout == NOTT_NCHW && d->groups == 1 && d->r == 3 && d->s == 3 && d->stride_h == 1 &&
           d->stride_w == 1 && d->pad_h == 1 && d->pad_w == 1 && d->dil_h == 1 && d->dil_w == 1 && d->w <= 64;
}

int32_t in_rows_bound(int32_t h, int32_t w) {
    const int32_t hw = h * w;
    // A run of kTilePix pixels starting at any column touches at most
    // floor((kTilePix − 1 + w − 1)/w) + 1 image rows and, likewise, images;
    // each image adds its two halo rows.
    const int32_t rows = (kTilePix - 1 + w - 1) / w + 1;
    const int32_t imgs = (kTilePix - 1 + hw - 1) / hw + 1;
    return (rows + 2 * imgs) * (w + 2);
}

template <typename T, bool DGRAD>
int run_same(nott_ctx ctx, int32_t n, int32_t cin, int32_t h, int32_t w, int32_t cout, const T* in, const T* wsrc,
             const float* bias, T* out) {
    constexpr int CC = Chunk<T>::CC;
    const size_t wbytes = sizeof(T) * (size_t)cout * cin * 9;
    const int32_t in_rows = in_rows_bound(h, w);
    const size_t lds = (size_t)in_rows * kRowB + (size_t)9 * kTileCo * kRowB;
    if (lds > 80 * 1024) return fail(ctx, NOTT_ERR_UNSUPPORTED, "conv3x3: tile does not fit in LDS");
    T* wp = static_cast<T*>(workspace(ctx, wbytes));
    if (!wp) return NOTT_ERR_ALLOC;
    const int64_t welems = (int64_t)cout * cin * 9;
    hipLaunchKernelGGL((conv3x3_wprep_kernel<T, DGRAD>), dim3((unsigned)ceil_div(welems, 256)), dim3(256), 0,
                       ctx->stream, wsrc, wp, cout, cin);
    SameParams p;
    p.n = n; p.cin = cin; p.h = h; p.w = w; p.cout = cout;
    p.hw = h * w; p.w2 = w + 2; p.npix = n * h * w; p.in_rows = in_rows;
    p.fd_hw = FastDiv((uint32_t)(h * w));
    p.fd_w = FastDiv((uint32_t)w);
    p.fd_w2 = FastDiv((uint32_t)(w + 2));
    p.fd_h2 = FastDiv((uint32_t)(h + 2));
    const int64_t tiles = ceil_div((int64_t)p.npix, kTilePix);
    p.remap = (tiles % 8 == 0) ? 1 : 0;
    static bool attr_set[2] = {false, false};
    if (!attr_set[sizeof(T) == 2]) {
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&conv3x3_same_kernel<T>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, 80 * 1024);
        attr_set[sizeof(T) == 2] = true;
    }
    hipLaunchKernelGGL((conv3x3_same_kernel<T>), dim3((unsigned)tiles, (unsigned)(cout / kTileCo)), dim3(kThreads), lds,
                       ctx->stream, in, wp, bias, out, p);
    return launch_status(ctx, "conv3x3_same");
}

}  // namespace

bool fwd_applies(const nott_conv2d_desc* d, size_t elem) {
    const int cc = elem == 2 ? Chunk<bf16_t>::CC : Chunk<float>::CC;
    return same_shape(d) && d->c % cc == 0 && d->k % kTileCo == 0;
}

bool dgrad_applies(const nott_conv2d_desc* d, size_t elem) {
    const int cc = elem == 2 ? Chunk<bf16_t>::CC : Chunk<float>::CC;
    // dgrad's input channels are the conv's outputs (k), its outputs the conv's inputs (c).
    return same_shape(d) && d->k % cc == 0 && d->c % kTileCo == 0;
}

bool wgrad_applies(const nott_conv2d_desc*, size_t) { return false; }

template <typename T>
int fwd(nott_ctx ctx, const nott_conv2d_desc* d, const T* x, const T* w, const float* b, T* y) {
    return run_same<T, false>(ctx, (int32_t)d->n, (int32_t)d->c, (int32_t)d->h, (int32_t)d->w, (int32_t)d->k, x, w, b, y);
}

template <typename T>
int dgrad(nott_ctx ctx, const nott_conv2d_desc* d, const T* dy, const T* w, T* dx) {
    return run_same<T, true>(ctx, (int32_t)d->n, (int32_t)d->k, (int32_t)d->h, (int32_t)d->w, (int32_t)d->c, dy, w,
                             nullptr, dx);
}

template <typename T>
int wgrad(nott_ctx ctx, const nott_conv2d_desc*, const T*, const T*, float*, int) {
    return fail(ctx, NOTT_ERR_UNSUPPORTED, "conv3x3 wgrad");
}

template int fwd<float>(nott_ctx, const nott_conv2d_desc*, const float*, const float*, const float*, float*);
template int fwd<bf16_t>(nott_ctx, const nott_conv2d_desc*, const bf16_t*, const bf16_t*, const float*, bf16_t*);
template int dgrad<float>(nott_ctx, const nott_conv2d_desc*, const float*, const float*, float*);
template int dgrad<bf16_t>(nott_ctx, const nott_conv2d_desc*, const bf16_t*, const bf16_t*, bf16_t*);
template int wgrad<float>(nott_ctx, const nott_conv2d_desc*, const float*, const float*, float*, int);
template int wgrad<bf16_t>(nott_ctx, const nott_conv2d_desc*, const bf16_t*, const bf16_t*, float*, int);

}  // namespace conv_fast
}  // namespace nott
