// LDS-staged implicit-GEMM convolutions for the NCHW shapes the 3x3 stride-1
// kernels do not take: strided 3x3 (ResNet-18's stage entries), strided 1x1
// (its projection shortcuts) and other kernels up to 9 taps (reference
// layer/details/conv.hpp:177, i.e. ATen convolution / convolution_backward).
//
// Forward:  out[n, co, oh, ow] = b[co] + Σ_{ci,t} in[n, ci, oh·sh + dh_t, ow·sw + dw_t] · w_t[co, ci]
// with tap t = (r, s), dh = r − pad_h, dw = s − pad_w.  Data gradient of a
// stride-(sh, sw) convolution: dx pixels split into sh·sw parity classes
// (a, b); pixel (2i + a, 2j + b) (for stride 2) receives only the taps with
// a + pad_h − r and b + pad_w − s divisible by the stride, from
// dy[i + (a + pad_h − r)/sh, j + (b + pad_w − s)/sw], so each class is a
// stride-1 correlation over dy with its own 1–4 taps and no wasted products
// (dx = Σ_{k,r,s} w[k,c,r,s] · dy[n,k,(h+ph−r)/sh,(w+pw−s)/sw] over the exact
// quotients).
//
// As in conv3x3_same_kernel, a workgroup owns 256 consecutive output pixels
// of one class and 64 output channels, and per 64-byte channel chunk stages
// the input rows its pixels touch in LDS as [padded pixel][channel] rows,
// so every tap is a constant LDS row offset from the pixel's base row:
//   * rows: padded row U = h + pad_top; when every tap of a stride-2 pass
//     reads one row parity only (1x1 stride 2), only those rows are stored
//     (rs = 2);
//   * columns: padded column u = w + pad_left; stride 2 stores the even
//     columns first and the odd ones after them (cm = 1), so that the 16
//     consecutive output pixels of an MFMA operand, two input columns apart,
//     still read 16 consecutive LDS rows (conflict-free); when every tap
//     reads even columns only, the odd ones are not stored (cm = 2).
// Pixels outside the image read LDS rows that the fill never writes (zeroed
// once).  Small grids split the channel chunks over blockIdx.z into fp32
// partials reduced in a fixed order.
#include "conv_tile.hpp"

#include <algorithm>
#include <vector>

namespace nott {
namespace conv_fast {
namespace {

constexpr int kMaxClass = 4;
constexpr int kMaxTaps = 9;

struct TapClass {
    int32_t ntap;             // taps of this class
    int32_t ho, wo;           // virtual output grid
    int32_t npix;             // n·ho·wo
    int32_t tiles;            // 256-pixel tiles
    int32_t rmin, rmax;       // smallest / largest tap row offset (LDS padded rows)
    int32_t oa, ob;           // output position (oh·osh + oa, ow·osw + ob)
    int32_t vec_store;        // whole 16-byte output runs inside one plane (unit output step)
    int32_t remap;            // XCD-aware tile order
    int32_t toff[kMaxTaps];   // LDS row offset of each tap from the pixel's base row
    int64_t wslice;           // first weight element of the class's slices
    FastDiv fd_howo, fd_wo;
};

struct TapParams {
    int32_t n, cin, hin, win, cout;
    int32_t hout, wout;       // output tensor plane
    int32_t osh, osw;         // output step per virtual pixel
    int32_t hpr;              // LDS padded rows per image
    int32_t shl;              // LDS padded rows per output row
    int32_t rs;               // input rows per LDS padded row (1 or 2)
    int32_t pt;               // padded row U = h + pt
    int32_t pl, h2;           // padded column u = w + pl; start of the odd columns (cm 1)
    int32_t w2;               // LDS rows per padded row (odd)
    int32_t in_rows;          // LDS rows reserved for the input tile
    int32_t relu;
    int32_t cc_per_split, splits;
    int32_t npix_max;
    float* partial;           // [class][split][cout][npix_max] fp32, or null
    FastDiv fd_hpr, fd_w2;
    TapClass cls[kMaxClass];
};

// LDS position of padded column u.
template <int CM>
__device__ __forceinline__ int32_t col_pos(int32_t u, int32_t h2) {
    if constexpr (CM == 0) return u;
    else if constexpr (CM == 1) return (u & 1) ? h2 + (u >> 1) : (u >> 1);
    else return u >> 1;
}

// Weight slices, per class: [cb][cc][tap][64 columns][CC] in the LDS order of
// lds_off (as conv3x3_wprep_kernel).  Forward: column co, channel ci reads
// w[co][ci][r][s]; data gradient (TRANS): column c, channel k reads
// w[k][c][r][s].  Columns past cout are zero weights.
struct TapPrep {
    int32_t nclass;
    int32_t ntap[kMaxClass];
    int32_t rs_tap[kMaxClass][kMaxTaps];   // r·S + s of each tap
    int64_t begin[kMaxClass + 1];          // first destination element per class
};

// Grid: x over one slice's ntap·64·CC elements, y = (cb, cc) slice of the
// class, z = class; the fastest thread index runs over the source's
// contiguous dimension (ci forward, co for TRANS).
template <typename T, bool TRANS>
__global__ __launch_bounds__(256) void conv_tap_wprep_kernel(const T* __restrict__ w, T* __restrict__ wp,
                                                             int32_t cout, int32_t cin, int32_t rsz, TapPrep tp) {
    constexpr int CC = Chunk<T>::CC, SUB = Chunk<T>::SUB;
    const int32_t cl = blockIdx.z;
    const int32_t ntap = tp.ntap[cl];
    const int32_t j = (int32_t)blockIdx.x * 256 + (int32_t)threadIdx.x;
    if (j >= ntap * kTileCo * CC) return;
    const int32_t ncc = cin / CC;
    const int32_t cb = (int32_t)blockIdx.y / ncc, cc = (int32_t)blockIdx.y % ncc;
    const int32_t tap = j / (kTileCo * CC), rem = j % (kTileCo * CC);
    const int32_t cil = TRANS ? rem / kTileCo : rem % CC;
    const int32_t col = TRANS ? rem % kTileCo : rem / CC;
    const int32_t co = cb * kTileCo + col, ci = cc * CC + cil;
    const int32_t rsi = tp.rs_tap[cl][tap];
    const int64_t src = TRANS ? (((int64_t)ci * cout + co) * rsz + rsi) : (((int64_t)co * cin + ci) * rsz + rsi);
    const int64_t slice = tp.begin[cl] + ((int64_t)cb * ncc + cc) * ntap * kTileCo * CC;
    T val = T(0);
    if (co < cout) val = w[src];
    wp[slice + (int64_t)(lds_off(tap * kTileCo + col, cil / SUB) >> 4) * SUB + cil % SUB] = val;
}

template <typename T, bool VEC, int LW, int NTMAX, int CM>
__global__ __launch_bounds__(kThreads, 2) void conv_tap_kernel(const T* __restrict__ in, const T* __restrict__ wp,
                                                               const float* __restrict__ bias, T* __restrict__ out,
                                                               TapParams p) {
    constexpr int CC = Chunk<T>::CC, SUB = Chunk<T>::SUB;
    constexpr int VT = VEC ? VecTasks<T>::VT : 1;
    extern __shared__ __attribute__((aligned(16))) char smem[];
    char* lds_in = smem;
    char* lds_w = smem + p.in_rows * kRowB;

    const int32_t ci_ = blockIdx.z / p.splits, split = blockIdx.z - ci_ * p.splits;
    const TapClass& C = p.cls[ci_];
    if ((int32_t)blockIdx.x >= C.tiles) return;
    int32_t tile = blockIdx.x;
    if (C.remap) tile = (int32_t)((blockIdx.x & 7) * (gridDim.x >> 3) + (blockIdx.x >> 3));
    const int32_t ntap = C.ntap;
    const int32_t cb = blockIdx.y;
    const int32_t m0 = tile * kTilePix;
    const int32_t m_last = min(m0 + kTilePix, C.npix) - 1;

    auto base_row = [&](int32_t m) -> int32_t {
        uint32_t n, r, oh, ow;
        C.fd_howo.divmod((uint32_t)m, n, r);
        C.fd_wo.divmod(r, oh, ow);
        return (int32_t)n * p.hpr + (int32_t)oh * p.shl;
    };
    const int32_t v_lo = base_row(m0) + C.rmin;
    const int32_t v_hi = base_row(m_last) + C.rmax;
    const int32_t nvr = v_hi - v_lo + 1;
    const int32_t nrows = nvr * p.w2;

    const int wid = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r16 = lane & 15, kq = lane >> 4;

    // This lane's LDS base row (before the tap offset) for its 4 pixel tiles.
    int32_t abase[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
        const int32_t m = min(m0 + wid * 64 + mt * 16 + r16, m_last);
        uint32_t n, r, oh, ow;
        C.fd_howo.divmod((uint32_t)m, n, r);
        C.fd_wo.divmod(r, oh, ow);
        abase[mt] = ((int32_t)n * p.hpr + (int32_t)oh * p.shl - v_lo) * p.w2 + (int32_t)ow;
    }
    auto aoff = [&](int tap, int mt) -> int32_t { return lds_off(abase[mt] + C.toff[tap], kq); };
    const int32_t boff = lds_off(r16, kq);

    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int32_t ncc = p.cin / CC;
    const int32_t cc0 = split * p.cc_per_split;
    const int32_t cc1 = min(ncc, cc0 + p.cc_per_split);
    const T* wblk = wp + C.wslice + (int64_t)cb * ncc * ntap * kTileCo * CC;

    // Input row of LDS padded row vr (< 0: outside the image).
    auto in_row = [&](int32_t vr, uint32_t& img) -> int32_t {
        uint32_t j;
        p.fd_hpr.divmod((uint32_t)(v_lo + vr), img, j);
        return (int32_t)j * p.rs - p.pt;
    };

    // Vector fill (see conv3x3_same_kernel): task = (w-chunk of SUB input
    // pixels, padded row, channel group of SUB), SUB 16-byte loads, a
    // register transpose, one 16-byte LDS write per stored pixel.
    constexpr int WG = 16 / SUB;
    const int32_t wchunks = (p.win + SUB - 1) / SUB;
    const int32_t wgroups = (wchunks + WG - 1) / WG;
    const int32_t ntask = nvr * wgroups * WG * 4;
    auto task_of = [&](int32_t t, int32_t& wc, int32_t& vr, int32_t& cig) {
        const int32_t u = t / WG, u2 = u / nvr;
        vr = u - u2 * nvr;
        cig = u2 / wgroups;
        wc = (u2 - cig * wgroups) * WG + (t % WG);
    };
    u32x4 rin[VT][SUB];
    auto fetch_task = [&](int32_t t, int32_t cc, u32x4 (&r)[SUB]) {
        int32_t wc, vr, cig;
        task_of(t, wc, vr, cig);
        uint32_t img;
        const int32_t h = in_row(vr, img);
        if (t < ntask && wc < wchunks && h >= 0 && h < p.hin && (int32_t)img < p.n) {
            const T* src = in + (((int64_t)img * p.cin + cc * CC + cig * SUB) * p.hin + h) * p.win;
            const int64_t plane = (int64_t)p.hin * p.win;
#pragma unroll
            for (int i = 0; i < SUB; ++i) r[i] = load_chunk<T, LW, true>(src + (int64_t)i * plane, wc, p.win);
        }
    };
    auto stash_task = [&](int32_t t, const u32x4 (&r)[SUB], char* dst) {
        int32_t wc, vr, cig;
        task_of(t, wc, vr, cig);
        uint32_t img;
        const int32_t h = in_row(vr, img);
        if (t < ntask && wc < wchunks && h >= 0 && h < p.hin && (int32_t)img < p.n) {
            u32x4 tr[SUB];
            transpose_block(r, tr);
#pragma unroll
            for (int i = 0; i < SUB; ++i) {
                const int32_t w = wc * SUB + i, u = w + p.pl;
                if ((LW == 16 || w < p.win) && (CM != 2 || (u & 1) == 0))
                    *reinterpret_cast<u32x4*>(dst + lds_off(vr * p.w2 + col_pos<CM>(u, p.h2), cig)) = tr[i];
            }
        }
    };
    const int WT = ntap * kTileCo * 4;      // 16-byte weight pieces per chunk
    auto stash = [&](int32_t cc) {
        if constexpr (VEC) {
#pragma unroll
            for (int j = 0; j < VT; ++j) stash_task(threadIdx.x + j * kThreads, rin[j], lds_in);
            for (int32_t t = threadIdx.x + VT * kThreads; t < ntask; t += kThreads) {
                u32x4 r[SUB];
                fetch_task(t, cc, r);
                stash_task(t, r, lds_in);
            }
        } else {
            // One LDS row (pixel) × SUB channels per task, element loads.
            for (int32_t t = threadIdx.x; t < nrows * 4; t += kThreads) {
                const int32_t sub = t / nrows;
                const int32_t row = t - sub * nrows;
                uint32_t vr, pos;
                p.fd_w2.divmod((uint32_t)row, vr, pos);
                int32_t u;
                if constexpr (CM == 0) u = (int32_t)pos;
                else if constexpr (CM == 1) u = (int32_t)pos < p.h2 ? 2 * (int32_t)pos : 2 * ((int32_t)pos - p.h2) + 1;
                else u = 2 * (int32_t)pos;
                uint32_t img;
                const int32_t h = in_row((int32_t)vr, img), w = u - p.pl;
                T v[SUB];
                if (h >= 0 && h < p.hin && w >= 0 && w < p.win && (int32_t)img < p.n) {
                    const T* src = in + (((int64_t)img * p.cin + cc * CC + sub * SUB) * p.hin + h) * p.win + w;
#pragma unroll
                    for (int j = 0; j < SUB; ++j) v[j] = src[(int64_t)j * p.hin * p.win];
                } else {
#pragma unroll
                    for (int j = 0; j < SUB; ++j) v[j] = T(0);
                }
                *reinterpret_cast<u32x4*>(lds_in + lds_off(row, sub)) = pack_sub<T>(v);
            }
        }
        const u32x4* wsrc = reinterpret_cast<const u32x4*>(wblk + (int64_t)cc * ntap * kTileCo * CC);
        for (int32_t j = threadIdx.x; j < WT; j += kThreads)
            *reinterpret_cast<u32x4*>(lds_w + j * 16) = wsrc[j];
    };

    if constexpr (VEC) {
        for (int32_t t = threadIdx.x; t < ((nrows + 15) >> 4) * 64; t += kThreads)
            *reinterpret_cast<u32x4*>(lds_in + t * 16) = u32x4{0u, 0u, 0u, 0u};
        if (cc0 < cc1) {
#pragma unroll
            for (int j = 0; j < VT; ++j) fetch_task(threadIdx.x + j * kThreads, cc0, rin[j]);
        }
    }
    for (int32_t cc = cc0; cc < cc1; ++cc) {
        __syncthreads();
        stash(cc);
        __syncthreads();
        if constexpr (VEC) {
            if (cc + 1 < cc1) {
#pragma unroll
                for (int j = 0; j < VT; ++j) fetch_task(threadIdx.x + j * kThreads, cc + 1, rin[j]);
            }
        }
        u32x4 a[2][4], b[2][4];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) a[0][mt] = *reinterpret_cast<const u32x4*>(lds_in + aoff(0, mt));
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) b[0][nt] = *reinterpret_cast<const u32x4*>(lds_w + boff + nt * 1024);
#pragma unroll
        for (int tap = 0; tap < NTMAX; ++tap) {
            if (tap < ntap) {
                const int cur = tap & 1, nxt = cur ^ 1;
                if (tap + 1 < NTMAX && tap + 1 < ntap) {
#pragma unroll
                    for (int mt = 0; mt < 4; ++mt)
                        a[nxt][mt] = *reinterpret_cast<const u32x4*>(lds_in + aoff(tap + 1, mt));
#pragma unroll
                    for (int nt = 0; nt < 4; ++nt)
                        b[nxt][nt] = *reinterpret_cast<const u32x4*>(lds_w + boff + ((tap + 1) * 4 + nt) * 1024);
                }
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                    for (int nt = 0; nt < 4; ++nt) mfma_chunk<T>(a[cur][mt], b[cur][nt], acc[mt][nt]);
            }
        }
    }

    if (p.partial) {
        float* dst = p.partial + ((int64_t)ci_ * p.splits + split) * p.cout * p.npix_max;
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) {
            const int32_t co = cb * kTileCo + nt * 16 + r16;
            if (co >= p.cout) continue;
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
                const int32_t m = m0 + wid * 64 + mt * 16 + kq * 4;
                float* d = dst + (int64_t)co * p.npix_max + m;
                if (m + 3 <= m_last && (p.npix_max & 3) == 0) {
                    *reinterpret_cast<f32x4*>(d) = acc[mt][nt];
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (m + e <= m_last) d[e] = acc[mt][nt][e];
                }
            }
        }
        return;
    }

    // Epilogue through LDS as [co][pixel] rows (see conv3x3_same_kernel).
    __syncthreads();
    constexpr int OP = kTilePix * (int)sizeof(T) + 16;
    char* lds_o = smem;
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
        const int32_t col = nt * 16 + r16;
        const float bv = bias && cb * kTileCo + col < p.cout ? bias[cb * kTileCo + col] : 0.f;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            const int px = wid * 64 + mt * 16 + kq * 4;
            f32x4 v = acc[mt][nt] + bv;
            if (p.relu) {
                v.x = relu_out(v.x); v.y = relu_out(v.y); v.z = relu_out(v.z); v.w = relu_out(v.w);
            }
            Vec4<T>::st(reinterpret_cast<T*>(lds_o + col * OP + px * (int)sizeof(T)), v);
        }
    }
    __syncthreads();
    const int64_t oplane = (int64_t)p.hout * p.wout;
    if (C.vec_store) {
        constexpr int E16 = 16 / (int)sizeof(T);
        constexpr int RUNS = kTilePix / E16;
        for (int t = threadIdx.x; t < kTileCo * RUNS; t += kThreads) {
            const int col = t / RUNS, j = t % RUNS;
            const int32_t m = m0 + j * E16;
            const int32_t co = cb * kTileCo + col;
            if (m > m_last || co >= p.cout) continue;
            const char* src = lds_o + col * OP + j * 16;
            uint32_t n, hw;
            C.fd_howo.divmod((uint32_t)m, n, hw);
            if (m + E16 - 1 <= m_last) {
                *reinterpret_cast<u32x4*>(out + ((int64_t)n * p.cout + co) * oplane + hw) =
                    *reinterpret_cast<const u32x4*>(src);
            } else {
                for (int e = 0; e < E16 && m + e <= m_last; ++e) {
                    uint32_t ne, hwe;
                    C.fd_howo.divmod((uint32_t)(m + e), ne, hwe);
                    out[((int64_t)ne * p.cout + co) * oplane + hwe] = reinterpret_cast<const T*>(src)[e];
                }
            }
        }
    } else {
        for (int t = threadIdx.x; t < kTileCo * kTilePix; t += kThreads) {
            const int col = t / kTilePix, j = t % kTilePix;
            const int32_t m = m0 + j;
            const int32_t co = cb * kTileCo + col;
            if (m > m_last || co >= p.cout) continue;
            uint32_t n, r, oh, ow;
            C.fd_howo.divmod((uint32_t)m, n, r);
            C.fd_wo.divmod(r, oh, ow);
            out[((int64_t)n * p.cout + co) * oplane + (int64_t)((int32_t)oh * p.osh + C.oa) * p.wout +
                (int32_t)ow * p.osw + C.ob] = reinterpret_cast<const T*>(lds_o + col * OP)[j];
        }
    }
}

// out = bias + Σ_split partial (splits in order), ReLU if set, at each
// class's output positions.  Thread = 4 consecutive pixels of one (class,
// channel) row (16-byte partial loads when rows are whole 4-float groups).
template <typename T>
__global__ __launch_bounds__(256) void conv_tap_reduce_kernel(TapParams p, int32_t nclass, const float* __restrict__ bias,
                                                              T* __restrict__ out) {
    const int32_t groups = (p.npix_max + 3) >> 2;
    const int64_t per_rows = (int64_t)nclass * p.cout;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= per_rows * groups) return;
    const int64_t row = i / groups;
    const int32_t m = (int32_t)(i - row * groups) * 4;
    const int32_t cl = (int32_t)(row / p.cout), co = (int32_t)(row - (int64_t)cl * p.cout);
    const TapClass& C = p.cls[cl];
    if (m >= C.npix) return;
    const int64_t per = (int64_t)p.cout * p.npix_max;
    const float* src = p.partial + (int64_t)cl * p.splits * per + (int64_t)co * p.npix_max + m;
    float s[4] = {0.f, 0.f, 0.f, 0.f};
    const int ne = min(4, C.npix - m);
    if (ne == 4 && (p.npix_max & 3) == 0) {
        const f32x4 a = ordered_sum4(src, per, p.splits);
        s[0] = a.x; s[1] = a.y; s[2] = a.z; s[3] = a.w;
    } else {
        for (int e = 0; e < ne; ++e) s[e] = ordered_sum1(src + e, per, p.splits);
    }
    const float bv = bias ? bias[co] : 0.f;
    for (int e = 0; e < ne; ++e) {
        float v = s[e] + bv;
        if (p.relu) v = relu_out(v);
        uint32_t n, r, oh, ow;
        C.fd_howo.divmod((uint32_t)(m + e), n, r);
        C.fd_wo.divmod(r, oh, ow);
        Io<T>::st(out,
                  ((int64_t)n * p.cout + co) * p.hout * p.wout + (int64_t)((int32_t)oh * p.osh + C.oa) * p.wout +
                      (int32_t)ow * p.osw + C.ob,
                  v);
    }
}

// ------------------------------------------------------------------ host
struct TapSpec {                 // one class as the host plans it
    int32_t ho, wo, oa, ob;
    std::vector<int32_t> dh, dw, rsi;   // per tap: input row / column offset, r·S + s
};

struct Plan {
    TapParams p;
    TapPrep prep;
    int cm = 0, ntmax = 1;
    size_t lds = 0;
    int64_t welems = 0;
    int64_t blocks = 0;
};

int ntmax_for(int ntap) { return ntap <= 1 ? 1 : ntap <= 4 ? 4 : 9; }

// Builds the launch plan; false when the shape does not fit (LDS, channels).
template <typename T>
bool make_plan(const nott_ctx ctx, int32_t n, int32_t cin, int32_t hin, int32_t win, int32_t cout, int32_t sh, int32_t sw,
               int32_t hout, int32_t wout, int32_t osh, int32_t osw, const std::vector<TapSpec>& specs, Plan& pl) {
    constexpr int CC = Chunk<T>::CC;
    if (cin % CC != 0 || cout % 16 != 0 || specs.empty() || (int)specs.size() > kMaxClass) return false;
    TapParams& p = pl.p;
    p = TapParams{};
    p.n = n; p.cin = cin; p.hin = hin; p.win = win; p.cout = cout;
    p.hout = hout; p.wout = wout;
    p.osh = osh;
    p.osw = osw;
    // Padding that every tap of every class stays inside.
    int32_t dh_min = 0, dh_hi = 0, dw_min = 0, dw_hi = 0, ntap_max = 0;
    bool first = true;
    for (auto& s : specs) {
        if ((int)s.dh.size() > kMaxTaps) return false;
        ntap_max = std::max<int32_t>(ntap_max, (int32_t)s.dh.size());
        for (size_t t = 0; t < s.dh.size(); ++t) {
            const int32_t hi = s.dh[t] + (s.ho - 1) * sh, wi = s.dw[t] + (s.wo - 1) * sw;
            if (first) { dh_min = s.dh[t]; dh_hi = hi; dw_min = s.dw[t]; dw_hi = wi; first = false; }
            dh_min = std::min(dh_min, s.dh[t]); dh_hi = std::max(dh_hi, hi);
            dw_min = std::min(dw_min, s.dw[t]); dw_hi = std::max(dw_hi, wi);
        }
    }
    if (first) return false;
    const int32_t pt = std::max(0, -dh_min), pb = std::max(0, dh_hi - (hin - 1));
    const int32_t pleft = std::max(0, -dw_min), pr = std::max(0, dw_hi - (win - 1));
    if ((sh != 1 && sh != 2) || (sw != 1 && sw != 2)) return false;
    // Row storage: every other padded row when all taps read one parity.
    int32_t rs = 1;
    if (sh == 2) {
        bool one = true;
        for (auto& s : specs)
            for (int32_t d : s.dh) one = one && ((d + pt) % 2 == 0);
        if (one) rs = 2;
    }
    int cm = 0;
    if (sw == 2) {
        bool even = true;
        for (auto& s : specs)
            for (int32_t d : s.dw) even = even && ((d + pleft) % 2 == 0);
        cm = even ? 2 : 1;
    }
    const int32_t hp = hin + pt + pb, wpad = pleft + win + pr;
    p.hpr = (hp + rs - 1) / rs;
    p.shl = sh / rs;
    p.rs = rs;
    p.pt = pt;
    p.pl = pleft;
    p.h2 = (wpad + 1) / 2;
    p.w2 = (cm == 0 ? wpad : cm == 1 ? 2 * p.h2 : p.h2) | 1;
    p.fd_hpr = FastDiv((uint32_t)p.hpr);
    p.fd_w2 = FastDiv((uint32_t)p.w2);
    // Classes.
    const int64_t cbc = ceil_div(cout, kTileCo);
    TapPrep& tp = pl.prep;
    tp = TapPrep{};
    tp.nclass = (int32_t)specs.size();
    int64_t wofs = 0;
    int32_t max_nvr = 0, npix_max = 0;
    int64_t tiles_total = 0;
    for (size_t c = 0; c < specs.size(); ++c) {
        const TapSpec& s = specs[c];
        TapClass& C = p.cls[c];
        C.ntap = (int32_t)s.dh.size();
        C.ho = s.ho; C.wo = s.wo;
        C.npix = n * s.ho * s.wo;
        C.tiles = (int32_t)ceil_div(C.npix, kTilePix);
        C.oa = s.oa; C.ob = s.ob;
        C.fd_howo = FastDiv((uint32_t)(s.ho * s.wo));
        C.fd_wo = FastDiv((uint32_t)s.wo);
        int32_t rmin = 0, rmax = 0;
        for (int t = 0; t < C.ntap; ++t) {
            const int32_t ro = (pt + s.dh[t]) / rs, u = pleft + s.dw[t];
            const int32_t co = cm == 0 ? u : cm == 1 ? ((u & 1) ? p.h2 + (u >> 1) : (u >> 1)) : (u >> 1);
            C.toff[t] = ro * p.w2 + co;
            rmin = t == 0 ? ro : std::min(rmin, ro);
            rmax = t == 0 ? ro : std::max(rmax, ro);
            tp.rs_tap[c][t] = s.rsi[t];
        }
        C.rmin = rmin; C.rmax = rmax;
        // Largest LDS row span of a tile: the tile starts repeat with period howo.
        const int64_t howo = (int64_t)s.ho * s.wo;
        const int64_t probe = std::min<int64_t>(C.tiles, howo + 1);
        for (int64_t t = 0; t < probe; ++t) {
            const int64_t m0 = t * kTilePix, m1 = std::min<int64_t>(m0 + kTilePix, C.npix) - 1;
            auto br = [&](int64_t m) { return (m / howo) * p.hpr + ((m % howo) / s.wo) * p.shl; };
            max_nvr = std::max<int32_t>(max_nvr, (int32_t)(br(m1) - br(m0) + rmax - rmin + 1));
        }
        C.remap = 0;
        C.wslice = wofs;
        tp.ntap[c] = C.ntap;
        tp.begin[c] = wofs;
        wofs += cbc * kTileCo * (int64_t)cin * C.ntap;
        npix_max = std::max(npix_max, C.npix);
        tiles_total += C.tiles;
    }
    tp.begin[specs.size()] = wofs;
    pl.welems = wofs;
    pl.ntmax = ntmax_for(ntap_max);
    pl.cm = cm;
    p.in_rows = (max_nvr * p.w2 + 15) & ~15;
    const size_t lds_fill = (size_t)p.in_rows * kRowB + (size_t)ntap_max * kTileCo * kRowB;
    const size_t lds_epi = (size_t)kTileCo * (kTilePix * sizeof(T) + 16);
    pl.lds = std::max(lds_fill, lds_epi);
    if (pl.lds > 160 * 1024) return false;
    int32_t max_tiles = 0;
    for (size_t c = 0; c < specs.size(); ++c) max_tiles = std::max(max_tiles, p.cls[c].tiles);
    for (size_t c = 0; c < specs.size(); ++c) {
        TapClass& C = p.cls[c];
        C.remap = (C.tiles == max_tiles && C.tiles % 8 == 0) ? 1 : 0;
        // 16-byte output runs: unit output step and whole runs per plane (the
        // launch also requires a 16-byte aligned output).
        C.vec_store = (osh == 1 && osw == 1 && C.oa == 0 && C.ob == 0 && C.ho == hout && C.wo == wout &&
                       (C.ho * C.wo) % (16 / (int)sizeof(T)) == 0) ? 1 : 0;
    }
    p.npix_max = npix_max;
    // Split the channel chunks when the grid would not fill every resident
    // workgroup slot (two per CU when the tile leaves room, else one).
    const int32_t nchunks = cin / CC;
    const int64_t blocks = tiles_total * cbc;
    const int64_t slots = (int64_t)ctx->num_cu * (pl.lds <= 80 * 1024 ? 2 : 1);
    int32_t splits = 1;
    if (blocks < slots && nchunks > 1) splits = pick_chunk_splits(blocks, nchunks, slots, sizeof(T));
    p.cc_per_split = (int32_t)ceil_div(nchunks, splits);
    p.splits = (int32_t)ceil_div(nchunks, p.cc_per_split);
    pl.blocks = blocks;
    return true;
}

template <typename T, bool VEC, int LW, int NT, int CM>
void launch_tap(nott_ctx ctx, const Plan& pl, dim3 grid, const T* in, const T* wp, const float* bias, T* out) {
    auto fn = &conv_tap_kernel<T, VEC, LW, NT, CM>;
    static bool attr = false;
    if (!attr) {
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                                  160 * 1024);
        attr = true;
    }
    hipLaunchKernelGGL((conv_tap_kernel<T, VEC, LW, NT, CM>), grid, dim3(kThreads), pl.lds, ctx->stream, in, wp, bias,
                       out, pl.p);
}

template <typename T, int NT, int CM>
void launch_fill(nott_ctx ctx, const Plan& pl, dim3 grid, bool vec, int lw, const T* in, const T* wp,
                 const float* bias, T* out) {
    if (!vec) launch_tap<T, false, 16, NT, CM>(ctx, pl, grid, in, wp, bias, out);
    else if (lw == 16) launch_tap<T, true, 16, NT, CM>(ctx, pl, grid, in, wp, bias, out);
    else launch_tap<T, true, 8, NT, CM>(ctx, pl, grid, in, wp, bias, out);
}

constexpr int kNotApplicable = 1;

// Weight prep, the conv launch and (split) the ordered reduce.  w is
// [cout][cin][R][S] (forward) or [cin][cout][R][S] (TRANS, data gradient).
template <typename T>
int run_plan(nott_ctx ctx, Plan& pl, const T* in, const T* w, bool trans, int32_t rsz, const float* bias, T* out,
             int relu) {
    TapParams& p = pl.p;
    // Kernel variants built: (taps ≤ 9, 4, 1) × column mode as the plans
    // below produce them.
    const bool ok = (pl.ntmax == 9 && (pl.cm == 0 || pl.cm == 1)) || (pl.ntmax == 4 && (pl.cm == 0 || pl.cm == 1)) ||
                    (pl.ntmax == 1 && (pl.cm == 0 || pl.cm == 2));
    if (!ok) return kNotApplicable;
    p.relu = relu;
    const int nclass = pl.prep.nclass;
    const size_t wbytes = ((size_t)pl.welems * sizeof(T) + 255) & ~(size_t)255;
    const size_t pbytes = p.splits > 1 ? sizeof(float) * (size_t)nclass * p.splits * p.cout * (size_t)p.npix_max : 0;
    char* ws = static_cast<char*>(workspace(ctx, wbytes + pbytes));
    if (!ws) return NOTT_ERR_ALLOC;
    T* wp = reinterpret_cast<T*>(ws);
    p.partial = p.splits > 1 ? reinterpret_cast<float*>(ws + wbytes) : nullptr;
    int32_t ntap_max = 1;
    for (int c = 0; c < nclass; ++c) ntap_max = std::max(ntap_max, pl.prep.ntap[c]);
    constexpr int CC = Chunk<T>::CC;
    const dim3 gw((unsigned)ceil_div(ntap_max * kTileCo * CC, 256), (unsigned)(ceil_div(p.cout, kTileCo) * (p.cin / CC)),
                  (unsigned)nclass);
    if (trans)
        hipLaunchKernelGGL((conv_tap_wprep_kernel<T, true>), gw, dim3(256), 0, ctx->stream, w, wp, p.cout, p.cin, rsz,
                           pl.prep);
    else
        hipLaunchKernelGGL((conv_tap_wprep_kernel<T, false>), gw, dim3(256), 0, ctx->stream, w, wp, p.cout, p.cin, rsz,
                           pl.prep);
    const bool aligned_out = ((uintptr_t)out % 16) == 0;
    int32_t max_tiles = 0;
    for (int c = 0; c < nclass; ++c) {
        if (!aligned_out) p.cls[c].vec_store = 0;
        max_tiles = std::max(max_tiles, p.cls[c].tiles);
    }
    const int lw = wgrad_load_width(p.win, sizeof(T));
    const bool vec = ((uintptr_t)in % 16) == 0 && lw >= 8;
    const dim3 grid((unsigned)max_tiles, (unsigned)ceil_div(p.cout, kTileCo), (unsigned)(nclass * p.splits));
    if (pl.ntmax == 9 && pl.cm == 0) launch_fill<T, 9, 0>(ctx, pl, grid, vec, lw, in, wp, bias, out);
    else if (pl.ntmax == 9) launch_fill<T, 9, 1>(ctx, pl, grid, vec, lw, in, wp, bias, out);
    else if (pl.ntmax == 4 && pl.cm == 0) launch_fill<T, 4, 0>(ctx, pl, grid, vec, lw, in, wp, bias, out);
    else if (pl.ntmax == 4) launch_fill<T, 4, 1>(ctx, pl, grid, vec, lw, in, wp, bias, out);
    else if (pl.cm == 0) launch_fill<T, 1, 0>(ctx, pl, grid, vec, lw, in, wp, bias, out);
    else launch_fill<T, 1, 2>(ctx, pl, grid, vec, lw, in, wp, bias, out);
    if (p.splits > 1) {
        const int64_t total = (int64_t)nclass * p.cout * ((p.npix_max + 3) / 4);
        hipLaunchKernelGGL(conv_tap_reduce_kernel<T>, dim3((unsigned)ceil_div(total, 256)), dim3(256), 0, ctx->stream, p,
                           nclass, bias, out);
    }
    return launch_status(ctx, "conv_tap");
}

bool tap_shape(const nott_conv2d_desc* d) {
    return d->layout == NOTT_NCHW && d->groups == 1 && d->dil_h == 1 && d->dil_w == 1 &&
           (d->stride_h == 1 || d->stride_h == 2) && (d->stride_w == 1 || d->stride_w == 2) && d->r * d->s <= kMaxTaps;
}

int64_t out_dim(int64_t in, int64_t k, int64_t s, int64_t p) { return (in + 2 * p - k) / s + 1; }

// Forward: one class, every tap.
template <typename T>
bool fwd_plan(nott_ctx ctx, const nott_conv2d_desc* d, Plan& pl) {
    if (!tap_shape(d)) return false;
    const int32_t p = (int32_t)out_dim(d->h, d->r, d->stride_h, d->pad_h);
    const int32_t q = (int32_t)out_dim(d->w, d->s, d->stride_w, d->pad_w);
    TapSpec s;
    s.ho = p; s.wo = q; s.oa = 0; s.ob = 0;
    for (int r = 0; r < d->r; ++r)
        for (int c = 0; c < d->s; ++c) {
            s.dh.push_back(r - (int32_t)d->pad_h);
            s.dw.push_back(c - (int32_t)d->pad_w);
            s.rsi.push_back(r * (int32_t)d->s + c);
        }
    return make_plan<T>(ctx, (int32_t)d->n, (int32_t)d->c, (int32_t)d->h, (int32_t)d->w, (int32_t)d->k,
                        (int32_t)d->stride_h, (int32_t)d->stride_w, p, q, 1, 1, {s}, pl);
}

// Data gradient: one class per output parity (a, b) that any tap reaches;
// `zero_rest` reports parities no tap reaches (their dx stays zero).
template <typename T>
bool dgrad_plan(nott_ctx ctx, const nott_conv2d_desc* d, Plan& pl, bool& zero_rest) {
    if (!tap_shape(d)) return false;
    const int32_t sh = (int32_t)d->stride_h, sw = (int32_t)d->stride_w;
    const int32_t p = (int32_t)out_dim(d->h, d->r, sh, d->pad_h);
    const int32_t q = (int32_t)out_dim(d->w, d->s, sw, d->pad_w);
    std::vector<TapSpec> specs;
    zero_rest = false;
    for (int32_t a = 0; a < sh; ++a)
        for (int32_t b = 0; b < sw; ++b) {
            TapSpec s;
            s.ho = (int32_t)ceil_div(d->h - a, sh);
            s.wo = (int32_t)ceil_div(d->w - b, sw);
            s.oa = a; s.ob = b;
            if (s.ho <= 0 || s.wo <= 0) continue;
            for (int r = 0; r < d->r; ++r) {
                const int32_t tr = a + (int32_t)d->pad_h - r;
                if (((tr % sh) + sh) % sh) continue;
                for (int c = 0; c < d->s; ++c) {
                    const int32_t tc = b + (int32_t)d->pad_w - c;
                    if (((tc % sw) + sw) % sw) continue;
                    // exact division of a possibly negative numerator
                    s.dh.push_back(tr >= 0 ? tr / sh : -((-tr) / sh));
                    s.dw.push_back(tc >= 0 ? tc / sw : -((-tc) / sw));
                    s.rsi.push_back(r * (int32_t)d->s + c);
                }
            }
            if (s.dh.empty()) zero_rest = true;
            else specs.push_back(std::move(s));
        }
    if (specs.empty()) return false;
    // Input: dy (k channels, p × q), stepped one dy pixel per class pixel.
    return make_plan<T>(ctx, (int32_t)d->n, (int32_t)d->k, p, q, (int32_t)d->c, 1, 1, (int32_t)d->h, (int32_t)d->w, sh,
                        sw, specs, pl);
}

}  // namespace

// The forward takes the tap kernel where it measured faster than the
// column (bf16) or generic (fp32) path on ResNet-18's strided shapes: at
// least 4 taps (a 1-tap pass is all fill), and for bf16 a grid that needs no
// channel split.  The data gradient takes it wherever it applies.
bool tap_fwd_applies(nott_ctx ctx, const nott_conv2d_desc* d, size_t elem) {
    if (!ctx->conv_tap) return false;
    Plan pl;
    const bool ok = elem == 2 ? fwd_plan<bf16_t>(ctx, d, pl) : fwd_plan<float>(ctx, d, pl);
    return ok && pl.p.cls[0].ntap >= 4 && (elem == 4 || pl.p.splits == 1);
}

bool tap_dgrad_applies(nott_ctx ctx, const nott_conv2d_desc* d, size_t elem) {
    if (!ctx->conv_tap) return false;
    Plan pl;
    bool z;
    return elem == 2 ? dgrad_plan<bf16_t>(ctx, d, pl, z) : dgrad_plan<float>(ctx, d, pl, z);
}

template <typename T>
int tap_fwd(nott_ctx ctx, const nott_conv2d_desc* d, const T* x, const T* w, const float* b, T* y, int relu) {
    Plan pl;
    if (!fwd_plan<T>(ctx, d, pl)) return fail(ctx, NOTT_ERR_UNSUPPORTED, "conv_tap: shape not supported");
    const int st = run_plan<T>(ctx, pl, x, w, false, (int32_t)(d->r * d->s), b, y, relu);
    return st == kNotApplicable ? fail(ctx, NOTT_ERR_UNSUPPORTED, "conv_tap: no kernel variant") : st;
}

template <typename T>
int tap_dgrad(nott_ctx ctx, const nott_conv2d_desc* d, const T* dy, const T* w, T* dx) {
    Plan pl;
    bool zero_rest = false;
    if (!dgrad_plan<T>(ctx, d, pl, zero_rest)) return fail(ctx, NOTT_ERR_UNSUPPORTED, "conv_tap: shape not supported");
    if (zero_rest) {
        const int zs = nott_zero(ctx, (int64_t)sizeof(T) * d->n * d->c * d->h * d->w, dx);
        if (zs != NOTT_OK) return zs;
    }
    const int st = run_plan<T>(ctx, pl, dy, w, true, (int32_t)(d->r * d->s), nullptr, dx, 0);
    return st == kNotApplicable ? fail(ctx, NOTT_ERR_UNSUPPORTED, "conv_tap: no kernel variant") : st;
}

template int tap_fwd<float>(nott_ctx, const nott_conv2d_desc*, const float*, const float*, const float*, float*, int);
template int tap_fwd<bf16_t>(nott_ctx, const nott_conv2d_desc*, const bf16_t*, const bf16_t*, const float*, bf16_t*,
                             int);
template int tap_dgrad<float>(nott_ctx, const nott_conv2d_desc*, const float*, const float*, float*);
template int tap_dgrad<bf16_t>(nott_ctx, const nott_conv2d_desc*, const bf16_t*, const bf16_t*, bf16_t*);

}  // namespace conv_fast
}  // namespace nott
