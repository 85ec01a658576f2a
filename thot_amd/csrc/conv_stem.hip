// Forward of ResNet-18's stem convolution: NCHW, 3 input channels, 7x7,
// column stride 2 (reference layer/details/conv.hpp:177, i.e. ATen
// convolution; configs[4]: x[64,3,224,224] -> y[64,64,112,112]).
//
//   y[n, co, oh, ow] = b[co] + Σ_{c,r,s} w[co, c, r, s] · x[n, c, oh·sh − ph + r, 2·ow − pw + s]
//
// With 3 channels a channel-chunked implicit GEMM wastes most of every K
// step, and an explicit im2col moves 147 columns per pixel through HBM.
// Here the GEMM's K runs over (c, r, s) with s padded to 8, in groups of
// 16 bytes of one (c, r) input row: 8 bf16 (or two groups of 4 fp32) at
// input columns 2·ow − pw + s0 .. +7.  A workgroup owns 256 consecutive
// output pixels and all 64 output channels; it stages the raw input rows
// its pixels touch (every channel, whole padded rows) in LDS once, with the
// left padding chosen so that each lane's 16-byte operand starts on a
// 4-byte boundary: the A fragment is four (bf16) or two (fp32) aligned LDS
// reads at consecutive addresses across lanes, no im2col.  The weights are
// pre-arranged in global memory in MFMA-fragment order and read from there.
#include "conv_tile.hpp"

#include <algorithm>

namespace nott {
namespace conv_fast {
namespace {

constexpr int kStemC = 3, kStemR = 7, kStemS8 = 8;   // channels, kernel rows, kernel columns (padded)
constexpr int kStemCo = 64;                            // output channels per workgroup

template <typename T> struct StemK {
    static constexpr int SUBK = 16 / (int)sizeof(T);                 // k values per 16-byte group
    static constexpr int NS = kStemS8 / SUBK;                        // groups per (c, r) row
    static constexpr int G = kStemC * kStemR * NS;                   // groups
    static constexpr int KSTEPS = (G + 3) / 4;                       // 4 groups (one per kq) per K step
};

struct StemParams {
    int32_t n, hin, win, cout, ho, wo, sh, ph, pw, s;
    int32_t hp;          // padded rows per image: hin + ph + pad below
    int32_t wrow;        // LDS elements per staged row (even)
    int32_t in_rows;     // staged (image, row) rows reserved
    int32_t npix, tiles, remap, vec_store, relu;
    FastDiv fd_howo, fd_wo, fd_hp;
};

// wf[j][nt][lane][16 B]: lane (col = lane % 16, kq = lane / 16) of K step j
// and 16-channel block nt holds group g = 4j + kq of output channel
// co = nt·16 + col: w[co, c, r, s0 .. s0 + SUBK − 1] with (c, r, s0) the
// group's row and first column, zero past the kernel or the last group.
template <typename T>
__global__ __launch_bounds__(256) void stem_wprep_kernel(const T* __restrict__ w, T* __restrict__ wf, int32_t cout,
                                                         int32_t s) {
    using K = StemK<T>;
    const int64_t total = (int64_t)(cout / 16) * K::KSTEPS * 64 * K::SUBK;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= total) return;
    const int e = (int)(i % K::SUBK);
    int64_t rest = i / K::SUBK;
    const int lane = (int)(rest % 64);
    rest /= 64;
    const int nt = (int)(rest % (cout / 16));
    const int j = (int)(rest / (cout / 16));
    const int g = 4 * j + (lane >> 4), co = nt * 16 + (lane & 15);
    T v = T(0);
    if (g < K::G) {
        const int si = g % K::NS, cr = g / K::NS;
        const int c = cr / kStemR, r = cr % kStemR;
        const int sc = si * K::SUBK + e;
        if (sc < s) v = w[(((int64_t)co * kStemC + c) * kStemR + r) * s + sc];
    }
    // destination: [j][nt][lane][e]
    wf[(((int64_t)j * (cout / 16) + nt) * 64 + lane) * K::SUBK + e] = v;
}

template <typename T>
__device__ __forceinline__ u32x4 stem_afrag(const char* p) {
    if constexpr (sizeof(T) == 2) {
        const uint32_t* q = reinterpret_cast<const uint32_t*>(p);   // 4-byte aligned
        return u32x4{q[0], q[1], q[2], q[3]};
    } else {
        const uint2* q = reinterpret_cast<const uint2*>(p);         // 8-byte aligned
        const uint2 a = q[0], b = q[1];
        return u32x4{a.x, a.y, b.x, b.y};
    }
}

// Stages input rows v_lo .. v_lo + nvr − 1 (padded-row numbering, every
// channel) in LDS as [row][c][wrow]: element u of a row is input column
// u − padl (zero outside the image).  A 16-byte piece that is a whole,
// aligned run of the input row is one vector load; others are element
// loads.  XU pieces per thread are loaded before any is stored, so their
// latencies overlap.
template <typename T, int XU>
__device__ __forceinline__ void stem_stage_rows(const T* __restrict__ x, char* lds_x, const StemParams& p, int32_t v_lo,
                                                int32_t nvr, int32_t padl, bool vec_rows) {
    constexpr int E = (int)sizeof(T), SUBK = 16 / E;
    const int32_t cpr = (p.wrow * E) / 16;
    const int32_t total = nvr * kStemC * cpr;
    for (int32_t base = 0; base < total; base += XU * kThreads) {
        u32x4 v[XU];
#pragma unroll
        for (int j = 0; j < XU; ++j) {
            const int32_t t = base + j * kThreads + (int32_t)threadIdx.x;
            v[j] = u32x4{0u, 0u, 0u, 0u};
            if (t >= total) continue;
            const int32_t piece = t % cpr, rc = t / cpr;
            const int32_t c = rc % kStemC, vr = rc / kStemC;
            uint32_t img, hh;
            p.fd_hp.divmod((uint32_t)(v_lo + vr), img, hh);
            const int32_t h = (int32_t)hh - p.ph;
            if (h < 0 || h >= p.hin || (int32_t)img >= p.n) continue;
            const T* row = x + (((int64_t)img * kStemC + c) * p.hin + h) * p.win;
            const int32_t w0 = piece * SUBK - padl;
            if (vec_rows && w0 >= 0 && w0 + SUBK <= p.win && (w0 % SUBK) == 0) {
                v[j] = *reinterpret_cast<const u32x4*>(row + w0);
            } else {
                T e[SUBK];
#pragma unroll
                for (int q = 0; q < SUBK; ++q) {
                    const int32_t w = w0 + q;
                    e[q] = (w >= 0 && w < p.win) ? row[w] : T(0);
                }
                if constexpr (E == 2) {
#pragma unroll
                    for (int q = 0; q < 4; ++q) v[j][q] = (uint32_t)e[2 * q] | ((uint32_t)e[2 * q + 1] << 16);
                } else {
#pragma unroll
                    for (int q = 0; q < 4; ++q) v[j][q] = __builtin_bit_cast(uint32_t, e[q]);
                }
            }
        }
#pragma unroll
        for (int j = 0; j < XU; ++j) {
            const int32_t t = base + j * kThreads + (int32_t)threadIdx.x;
            if (t >= total) continue;
            const int32_t piece = t % cpr, rc = t / cpr;
            const int32_t c = rc % kStemC, vr = rc / kStemC;
            *reinterpret_cast<u32x4*>(lds_x + (size_t)(vr * kStemC + c) * p.wrow * E + piece * 16) = v[j];
        }
    }
}

template <typename T>
__global__ __launch_bounds__(kThreads, 2) void stem_fwd_kernel(const T* __restrict__ x, const T* __restrict__ wf,
                                                               const float* __restrict__ bias, T* __restrict__ y,
                                                               StemParams p) {
    using K = StemK<T>;
    constexpr int E = (int)sizeof(T);
    extern __shared__ __attribute__((aligned(16))) char smem[];
    const int32_t rowb = p.wrow * E;                          // bytes per staged channel row
    char* lds_x = smem;                                        // [row][c][wrow]

    int32_t tile = blockIdx.x;
    if (p.remap) tile = (int32_t)((blockIdx.x & 7) * (gridDim.x >> 3) + (blockIdx.x >> 3));
    const int32_t m0 = tile * kTilePix;
    const int32_t m_last = min(m0 + kTilePix, p.npix) - 1;
    auto base_row = [&](int32_t m) -> int32_t {   // padded row of kernel row r = 0
        uint32_t n, r, oh, ow;
        p.fd_howo.divmod((uint32_t)m, n, r);
        p.fd_wo.divmod(r, oh, ow);
        return (int32_t)n * p.hp + (int32_t)oh * p.sh;
    };
    const int32_t v_lo = base_row(m0);
    const int32_t nvr = base_row(m_last) + kStemR - v_lo;

    // Staged rows: padded column u = w + pw at element u (so that a lane's
    // first column 2·ow − pw + s0 sits at the even element 2·ow + s0).
    stem_stage_rows<T, 4>(x, lds_x, p, v_lo, nvr, p.pw, false);
    __syncthreads();

    const int wid = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r16 = lane & 15, kq = lane >> 4;
    // Byte offset of this lane's pixel (kernel row 0, channel 0, column 2·ow).
    int32_t abase[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
        const int32_t m = min(m0 + wid * 64 + mt * 16 + r16, m_last);
        uint32_t n, r, oh, ow;
        p.fd_howo.divmod((uint32_t)m, n, r);
        p.fd_wo.divmod(r, oh, ow);
        abase[mt] = ((int32_t)n * p.hp + (int32_t)oh * p.sh - v_lo) * kStemC * rowb + 2 * (int32_t)ow * E;
    }

    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    // The B fragments (the pre-arranged weights, the same for every
    // workgroup) are read from global memory, where they stay cached, one
    // K step ahead: no weight copy in LDS, so more workgroups fit per CU.
    const u32x4* wfv = reinterpret_cast<const u32x4*>(wf);
    u32x4 bn[4];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) bn[nt] = wfv[nt * 64 + lane];
#pragma unroll
    for (int j = 0; j < K::KSTEPS; ++j) {
        const int g = 4 * j + kq;
        // (c, r, s0) of this lane's group; groups past G read zeros weights,
        // so any in-tile address serves (group 0's).
        const int gg = g < K::G ? g : 0;
        const int si = gg % K::NS, cr = gg / K::NS;
        const int32_t goff = ((cr % kStemR) * kStemC + cr / kStemR) * rowb + si * 16;
        u32x4 a[4], b[4];
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) b[nt] = bn[nt];
        if (j + 1 < K::KSTEPS) {
#pragma unroll
            for (int nt = 0; nt < 4; ++nt) bn[nt] = wfv[((j + 1) * (p.cout / 16) + nt) * 64 + lane];
        }
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) a[mt] = stem_afrag<T>(lds_x + abase[mt] + goff);
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int nt = 0; nt < 4; ++nt) mfma_chunk<T>(a[mt], b[nt], acc[mt][nt]);
    }

    // Epilogue through LDS as [co][pixel] rows, 16-byte runs of one plane,
    // 32 channels at a time.
    const int64_t plane = (int64_t)p.ho * p.wo;
    constexpr int OP = kTilePix * E + 16;
    constexpr int E16 = 16 / E;
    constexpr int RUNS = kTilePix / E16;
    char* lds_o = smem;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
        __syncthreads();
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int nt = 2 * half + h;
            const int32_t col = nt * 16 + r16;
            const float bv = bias ? bias[col] : 0.f;
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
                const int px = wid * 64 + mt * 16 + kq * 4;
                f32x4 v = acc[mt][nt] + bv;
                if (p.relu) {
                    v.x = relu_out(v.x); v.y = relu_out(v.y); v.z = relu_out(v.z); v.w = relu_out(v.w);
                }
                Vec4<T>::st(reinterpret_cast<T*>(lds_o + (h * 16 + r16) * OP + px * E), v);
            }
        }
        __syncthreads();
        for (int t = threadIdx.x; t < (kStemCo / 2) * RUNS; t += kThreads) {
            const int cl = t / RUNS, jr = t % RUNS;
            const int col = half * (kStemCo / 2) + cl;
            const int32_t m = m0 + jr * E16;
            if (m > m_last) continue;
            const char* src = lds_o + cl * OP + jr * 16;
            uint32_t n, hw;
            p.fd_howo.divmod((uint32_t)m, n, hw);
            if (p.vec_store && m + E16 - 1 <= m_last) {
                *reinterpret_cast<u32x4*>(y + ((int64_t)n * p.cout + col) * plane + hw) =
                    *reinterpret_cast<const u32x4*>(src);
            } else {
                for (int e = 0; e < E16 && m + e <= m_last; ++e) {
                    uint32_t ne, hwe;
                    p.fd_howo.divmod((uint32_t)(m + e), ne, hwe);
                    y[((int64_t)ne * p.cout + col) * plane + hwe] = reinterpret_cast<const T*>(src)[e];
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Weight gradient: dw[co, c, r, s] = Σ_{n,oh,ow} dy[n, co, oh, ow] · x[n, c, oh·sh − ph + r, 2·ow − pw + s].
// GEMM with M = 64 output channels, N = (c, r, s) with s padded to 8 (168
// columns, 11 blocks of 16) and the reduction over output pixels.  Per
// 256-pixel tile a workgroup stages dy as [co][pixel] (an A fragment is 8
// consecutive pixels of one channel: one aligned 16-byte read) and the raw
// input rows as in the forward (a B fragment is the 8 stride-2 input columns
// of one (c, r, s) at 8 consecutive pixels: element reads).  Wave w owns
// column blocks w, w+4, w+8 for all 64 channels.  Each workgroup sums
// several tiles in registers and writes one fp32 partial; the partials are
// added in workgroup order (deterministic).
constexpr int kStemNB = (kStemC * kStemR * kStemS8 + 15) / 16;   // 11 column blocks

struct StemWgParams {
    StemParams g;
    int32_t tiles_per_wg;
    int32_t padl;        // staged element of input column 0 (a multiple of 16 bytes, ≥ pw)
    int32_t vec_rows;    // input rows are whole, aligned 16-byte runs
    int32_t row_runs;    // output rows hold whole runs of SUBK pixels (wo % SUBK == 0)
};

template <typename T>
__global__ __launch_bounds__(kThreads, 2) void stem_wgrad_kernel(const T* __restrict__ x, const T* __restrict__ dy,
                                                                 float* __restrict__ part, StemWgParams q) {
    const StemParams& p = q.g;
    constexpr int E = (int)sizeof(T);
    constexpr int SUBK = 16 / E;                 // pixels per lane per K step
    constexpr int KPIX = 4 * SUBK;               // pixels per K step
    extern __shared__ __attribute__((aligned(16))) char smem[];
    const int32_t rowb = p.wrow * E;
    char* lds_dy = smem;                                    // [64 co][256 px]
    char* lds_x = smem + kStemCo * kTilePix * E;            // [row][c][wrow]
    const int wid = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r16 = lane & 15, kq = lane >> 4;
    const int64_t plane = (int64_t)p.ho * p.wo;

    // This lane's B columns (one per owned column block): LDS offset of
    // (c, r) row and column s, or −1 past the 168 real columns / s ≥ S.
    int32_t bcol[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const int nb = wid + 4 * i;
        const int col = nb * 16 + r16;
        bcol[i] = -1;
        if (nb < kStemNB && col < kStemC * kStemR * kStemS8) {
            const int sc = col % kStemS8, cr = col / kStemS8;
            const int c = cr / kStemR, r = cr % kStemR;
            if (sc < p.s) bcol[i] = (r * kStemC + c) * rowb + (sc - p.pw + q.padl) * E;
        }
    }
    f32x4 acc[4][3];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int32_t it = 0; it < q.tiles_per_wg; ++it) {
        const int32_t tile = blockIdx.x + it * gridDim.x;
        if (tile >= p.tiles) break;
        const int32_t m0 = tile * kTilePix;
        const int32_t m_last = min(m0 + kTilePix, p.npix) - 1;
        auto base_row = [&](int32_t m) -> int32_t {
            uint32_t n, r, oh, ow;
            p.fd_howo.divmod((uint32_t)m, n, r);
            p.fd_wo.divmod(r, oh, ow);
            return (int32_t)n * p.hp + (int32_t)oh * p.sh;
        };
        const int32_t v_lo = base_row(m0);
        const int32_t nvr = base_row(m_last) + kStemR - v_lo;
        __syncthreads();   // the previous tile's operands are read
        // dy tile: 16-byte runs of SUBK pixels (element loads where a run
        // leaves the image plane or the last tile), all loads of a thread
        // issued before its stores.
        constexpr int DYT = kStemCo * (kTilePix / SUBK) / kThreads;
        u32x4 rdy[DYT];
#pragma unroll
        for (int i = 0; i < DYT; ++i) {
            const int32_t t = i * kThreads + (int32_t)threadIdx.x;
            const int32_t co = t / (kTilePix / SUBK), j = t % (kTilePix / SUBK);
            const int32_t m = m0 + j * SUBK;
            uint32_t n, hw;
            p.fd_howo.divmod((uint32_t)min(m, m_last), n, hw);
            u32x4 v = u32x4{0u, 0u, 0u, 0u};
            const T* src = dy + ((int64_t)n * p.cout + co) * plane + hw;
            if (m + SUBK - 1 <= m_last && (int64_t)hw + SUBK <= plane && p.vec_store) {
                v = *reinterpret_cast<const u32x4*>(src);
            } else {
                T e8[SUBK];
#pragma unroll
                for (int e = 0; e < SUBK; ++e) {
                    e8[e] = T(0);
                    if (m + e <= m_last) {
                        uint32_t ne, hwe;
                        p.fd_howo.divmod((uint32_t)(m + e), ne, hwe);
                        e8[e] = dy[((int64_t)ne * p.cout + co) * plane + hwe];
                    }
                }
                if constexpr (E == 2) {
#pragma unroll
                    for (int w = 0; w < 4; ++w)
                        v[w] = (uint32_t)e8[2 * w] | ((uint32_t)e8[2 * w + 1] << 16);
                } else {
#pragma unroll
                    for (int w = 0; w < 4; ++w) v[w] = __builtin_bit_cast(uint32_t, e8[w]);
                }
            }
            rdy[i] = v;
        }
#pragma unroll
        for (int i = 0; i < DYT; ++i) {
            const int32_t t = i * kThreads + (int32_t)threadIdx.x;
            const int32_t co = t / (kTilePix / SUBK), j = t % (kTilePix / SUBK);
            *reinterpret_cast<u32x4*>(lds_dy + (size_t)co * kTilePix * E + j * 16) = rdy[i];
        }
        // raw input rows with a 16-byte-multiple left pad: whole aligned runs
        // of the input row are single vector loads
        stem_stage_rows<T, 4>(x, lds_x, p, v_lo, nvr, q.padl, q.vec_rows != 0);
        __syncthreads();
        for (int32_t k0 = 0; k0 < kTilePix; k0 += KPIX) {
            // This lane's SUBK pixels of the K step: LDS base of each pixel's
            // kernel row 0, channel 0, column 2·ow (pixels past the tile: dy 0).
            // When output rows hold whole runs of SUBK pixels, the run starts
            // a row and its pixels are consecutive columns of it.
            int32_t pbase[SUBK];
            auto base_of = [&](int32_t m) {
                uint32_t n, r, oh, ow;
                p.fd_howo.divmod((uint32_t)m, n, r);
                p.fd_wo.divmod(r, oh, ow);
                return ((int32_t)n * p.hp + (int32_t)oh * p.sh - v_lo) * kStemC * rowb + 2 * (int32_t)ow * E;
            };
            if (q.row_runs) {
                // A run never crosses m_last (tiles end on whole runs); one
                // that starts past it repeats pixel m_last, whose staged x is
                // finite (its dy is zero).
                const int32_t ms = m0 + k0 + kq * SUBK;
                const int32_t b0 = base_of(min(ms, m_last)), step = ms <= m_last ? 2 * E : 0;
#pragma unroll
                for (int e = 0; e < SUBK; ++e) pbase[e] = b0 + e * step;
            } else {
#pragma unroll
                for (int e = 0; e < SUBK; ++e) pbase[e] = base_of(min(m0 + k0 + kq * SUBK + e, m_last));
            }
            u32x4 a[4], b[3];
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
                a[mt] = *reinterpret_cast<const u32x4*>(lds_dy + (size_t)(mt * 16 + r16) * kTilePix * E +
                                                         (k0 + kq * SUBK) * E);
#pragma unroll
            for (int i = 0; i < 3; ++i) {
                u32x4 v = u32x4{0u, 0u, 0u, 0u};
                if (bcol[i] >= 0) {
                    if constexpr (E == 2) {
                        uint16_t e8[8];
#pragma unroll
                        for (int e = 0; e < 8; ++e)
                            e8[e] = *reinterpret_cast<const uint16_t*>(lds_x + pbase[e] + bcol[i]);
#pragma unroll
                        for (int w = 0; w < 4; ++w) v[w] = (uint32_t)e8[2 * w] | ((uint32_t)e8[2 * w + 1] << 16);
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e) v[e] = *reinterpret_cast<const uint32_t*>(lds_x + pbase[e] + bcol[i]);
                    }
                }
                b[i] = v;
            }
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                for (int i = 0; i < 3; ++i) mfma_chunk<T>(a[mt], b[i], acc[mt][i]);
        }
    }
    // partial[wg][co][col] (fp32, 176 columns)
    float* dst = part + (int64_t)blockIdx.x * kStemCo * kStemNB * 16;
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const int nb = wid + 4 * i;
        if (nb >= kStemNB) continue;
        const int col = nb * 16 + r16;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int e = 0; e < 4; ++e) dst[(int64_t)(mt * 16 + kq * 4 + e) * kStemNB * 16 + col] = acc[mt][i][e];
    }
}

// dw[co][c][r][s] (+)= Σ_wg partial[wg][co][(c·R + r)·8 + s].  A block owns
// 64 partial columns (lane = column, so each wave load is one 256-byte run);
// its 16 waves take the workgroups round-robin with 8 loads in flight (512
// partial rows in four rounds) and combine in LDS in wave order, so the
// summation order is fixed.
constexpr int kStemRedWaves = 16;
__global__ __launch_bounds__(64 * kStemRedWaves) void stem_wgrad_reduce_kernel(const float* __restrict__ part,
                                                                               int32_t nwg, int32_t s,
                                                                               float* __restrict__ dw, int accumulate) {
    __shared__ float red[kStemRedWaves][64];
    constexpr int32_t kCols = kStemCo * kStemNB * 16;
    constexpr int W = kStemRedWaves;
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int32_t i = blockIdx.x * 64 + lane;           // partial column: co·176 + col
    float a = 0.f;
    if (i < kCols) {
        const float* src = part + i;
        int32_t w = wid;
        for (; w + 7 * W < nwg; w += 8 * W) {
            float t[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) t[u] = src[(int64_t)(w + W * u) * kCols];
#pragma unroll
            for (int u = 0; u < 8; ++u) a += t[u];
        }
        for (; w < nwg; w += W) a += src[(int64_t)w * kCols];
    }
    red[wid][lane] = a;
    __syncthreads();
    if (wid != 0 || i >= kCols) return;
    float t = 0.f;
#pragma unroll
    for (int k = 0; k < W; ++k) t += red[k][lane];
    const int32_t co = i / (kStemNB * 16), col = i % (kStemNB * 16);
    const int32_t sc = col % kStemS8, cr = col / kStemS8;
    if (cr >= kStemC * kStemR || sc >= s) return;
    const int32_t c = cr / kStemR, r = cr % kStemR;
    float* o = dw + (((int64_t)co * kStemC + c) * kStemR + r) * s + sc;
    *o = accumulate ? *o + t : t;
}

int64_t stem_out(int64_t in, int64_t k, int64_t s, int64_t p) { return (in + 2 * p - k) / s + 1; }

}  // namespace

bool stem_fwd_applies(nott_ctx ctx, const nott_conv2d_desc* d) {
    return ctx->conv_tap && d->layout == NOTT_NCHW && d->groups == 1 && d->c == kStemC && d->r == kStemR && d->s >= 1 &&
           d->s <= kStemS8 && d->stride_w == 2 && d->stride_h >= 1 && d->dil_h == 1 && d->dil_w == 1 &&
           d->k == kStemCo && d->pad_h >= 0 && d->pad_w >= 0 && d->pad_w < 64;
}

template <typename T>
int stem_fwd(nott_ctx ctx, const nott_conv2d_desc* d, const T* x, const T* w, const float* b, T* y, int relu) {
    using K = StemK<T>;
    constexpr int E = (int)sizeof(T);
    StemParams p;
    p.n = (int32_t)d->n; p.hin = (int32_t)d->h; p.win = (int32_t)d->w; p.cout = (int32_t)d->k;
    p.ho = (int32_t)stem_out(d->h, d->r, d->stride_h, d->pad_h);
    p.wo = (int32_t)stem_out(d->w, d->s, d->stride_w, d->pad_w);
    p.sh = (int32_t)d->stride_h; p.ph = (int32_t)d->pad_h; p.pw = (int32_t)d->pad_w; p.s = (int32_t)d->s;
    if (p.ho <= 0 || p.wo <= 0) return fail(ctx, NOTT_ERR_INVALID_ARG, "stem conv: empty output");
    // Rows every pixel's 7 kernel rows stay inside: pad above ph, below as needed.
    const int32_t pb = std::max<int32_t>(0, (p.ho - 1) * p.sh - p.ph + kStemR - 1 - (p.hin - 1));
    p.hp = p.hin + p.ph + pb;
    // Staged row: padded columns 0 .. 2·(wo−1) + 7 (s padded to 8), whole
    // 16-byte pieces.  (A pitch that spreads the four kernel rows of a K step
    // over distinct LDS bank quarters measured slower: the extra zero fill
    // costs more than the conflicts.)
    const int32_t need = std::max<int32_t>(2 * (p.wo - 1) + kStemS8, p.pw + p.win);
    p.wrow = (int32_t)ceil_div(need, 16 / E) * (16 / E);
    p.npix = p.n * p.ho * p.wo;
    p.tiles = (int32_t)ceil_div(p.npix, kTilePix);
    p.fd_howo = FastDiv((uint32_t)(p.ho * p.wo));
    p.fd_wo = FastDiv((uint32_t)p.wo);
    p.fd_hp = FastDiv((uint32_t)p.hp);
    // Largest staged-row span of a tile (the pattern repeats with period ho·wo).
    const int64_t howo = (int64_t)p.ho * p.wo;
    int32_t max_nvr = 0;
    for (int64_t t = 0; t < std::min<int64_t>(p.tiles, howo + 1); ++t) {
        const int64_t m0 = t * kTilePix, m1 = std::min<int64_t>(m0 + kTilePix, p.npix) - 1;
        auto br = [&](int64_t m) { return (m / howo) * p.hp + ((m % howo) / p.wo) * p.sh; };
        max_nvr = std::max<int32_t>(max_nvr, (int32_t)(br(m1) + kStemR - br(m0)));
    }
    p.in_rows = max_nvr;
    const size_t wbytes = (size_t)K::KSTEPS * (p.cout / 16) * 64 * 16;
    const size_t lds_fill = (size_t)p.in_rows * kStemC * p.wrow * E;
    const size_t lds_epi = (size_t)(kStemCo / 2) * (kTilePix * E + 16);
    const size_t lds = std::max(lds_fill, lds_epi);
    if (lds > 160 * 1024) return fail(ctx, NOTT_ERR_UNSUPPORTED, "stem conv: tile does not fit in LDS");
    p.remap = (p.tiles % 8 == 0) ? 1 : 0;
    p.vec_store = (howo % (16 / E) == 0 && ((uintptr_t)y % 16) == 0) ? 1 : 0;
    p.relu = relu;
    T* wf = static_cast<T*>(workspace(ctx, wbytes));
    if (!wf) return NOTT_ERR_ALLOC;
    const int64_t welems = (int64_t)wbytes / E;
    hipLaunchKernelGGL(stem_wprep_kernel<T>, dim3((unsigned)ceil_div(welems, 256)), dim3(256), 0, ctx->stream, w, wf,
                       p.cout, p.s);
    static bool attr = false;
    if (!attr) {
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&stem_fwd_kernel<T>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        attr = true;
    }
    hipLaunchKernelGGL(stem_fwd_kernel<T>, dim3((unsigned)p.tiles), dim3(kThreads), lds, ctx->stream, x, wf, b, y, p);
    return launch_status(ctx, "stem_fwd");
}

template int stem_fwd<float>(nott_ctx, const nott_conv2d_desc*, const float*, const float*, const float*, float*, int);
template int stem_fwd<bf16_t>(nott_ctx, const nott_conv2d_desc*, const bf16_t*, const bf16_t*, const float*, bf16_t*,
                              int);

bool stem_wgrad_applies(nott_ctx ctx, const nott_conv2d_desc* d) { return stem_fwd_applies(ctx, d); }

template <typename T>
int stem_wgrad(nott_ctx ctx, const nott_conv2d_desc* d, const T* x, const T* dy, float* dw, int accumulate) {
    constexpr int E = (int)sizeof(T);
    StemWgParams q;
    StemParams& p = q.g;
    p.n = (int32_t)d->n; p.hin = (int32_t)d->h; p.win = (int32_t)d->w; p.cout = (int32_t)d->k;
    p.ho = (int32_t)stem_out(d->h, d->r, d->stride_h, d->pad_h);
    p.wo = (int32_t)stem_out(d->w, d->s, d->stride_w, d->pad_w);
    p.sh = (int32_t)d->stride_h; p.ph = (int32_t)d->pad_h; p.pw = (int32_t)d->pad_w; p.s = (int32_t)d->s;
    if (p.ho <= 0 || p.wo <= 0) return fail(ctx, NOTT_ERR_INVALID_ARG, "stem conv: empty output");
    const int32_t pb = std::max<int32_t>(0, (p.ho - 1) * p.sh - p.ph + kStemR - 1 - (p.hin - 1));
    p.hp = p.hin + p.ph + pb;
    // Staged elements: input column w at w + padl; reads reach column
    // 2·(wo−1) − pw + 7.
    q.padl = (int32_t)ceil_div(p.pw, 16 / E) * (16 / E);
    const int32_t need = std::max<int32_t>(2 * (p.wo - 1) - p.pw + kStemS8 + q.padl, q.padl + p.win);
    p.wrow = (int32_t)ceil_div(need, 16 / E) * (16 / E);
    q.vec_rows = (p.win % (16 / E) == 0 && ((uintptr_t)x % 16) == 0) ? 1 : 0;
    p.npix = p.n * p.ho * p.wo;
    p.tiles = (int32_t)ceil_div(p.npix, kTilePix);
    p.fd_howo = FastDiv((uint32_t)(p.ho * p.wo));
    p.fd_wo = FastDiv((uint32_t)p.wo);
    p.fd_hp = FastDiv((uint32_t)p.hp);
    const int64_t howo = (int64_t)p.ho * p.wo;
    int32_t max_nvr = 0;
    for (int64_t t = 0; t < std::min<int64_t>(p.tiles, howo + 1); ++t) {
        const int64_t m0 = t * kTilePix, m1 = std::min<int64_t>(m0 + kTilePix, p.npix) - 1;
        auto br = [&](int64_t m) { return (m / howo) * p.hp + ((m % howo) / p.wo) * p.sh; };
        max_nvr = std::max<int32_t>(max_nvr, (int32_t)(br(m1) + kStemR - br(m0)));
    }
    p.in_rows = max_nvr;
    const size_t lds = (size_t)kStemCo * kTilePix * E + (size_t)p.in_rows * kStemC * p.wrow * E;
    if (lds > 160 * 1024) return fail(ctx, NOTT_ERR_UNSUPPORTED, "stem conv: tile does not fit in LDS");
    // dy runs of 16 bytes stay 16-byte aligned inside a plane.
    p.vec_store = (howo % (16 / E) == 0 && ((uintptr_t)dy % 16) == 0) ? 1 : 0;
    p.remap = 0;
    p.relu = 0;
    const int32_t per_cu = lds <= 80 * 1024 ? 2 : 1;
    const int32_t nwg = (int32_t)std::min<int64_t>(p.tiles, (int64_t)per_cu * ctx->num_cu);
    q.tiles_per_wg = (int32_t)ceil_div(p.tiles, nwg);
    q.row_runs = (p.wo % (16 / (int)sizeof(T)) == 0) ? 1 : 0;
    const size_t pbytes = sizeof(float) * (size_t)nwg * kStemCo * kStemNB * 16;
    float* part = static_cast<float*>(workspace(ctx, pbytes));
    if (!part) return NOTT_ERR_ALLOC;
    static bool attr = false;
    if (!attr) {
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&stem_wgrad_kernel<T>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        attr = true;
    }
    hipLaunchKernelGGL(stem_wgrad_kernel<T>, dim3((unsigned)nwg), dim3(kThreads), lds, ctx->stream, x, dy, part, q);
    hipLaunchKernelGGL(stem_wgrad_reduce_kernel, dim3((unsigned)ceil_div(kStemCo * kStemNB * 16, 64)),
                       dim3(64 * kStemRedWaves), 0,
                       ctx->stream, part, nwg, p.s, dw, accumulate);
    return launch_status(ctx, "stem_wgrad");
}

template int stem_wgrad<float>(nott_ctx, const nott_conv2d_desc*, const float*, const float*, float*, int);
template int stem_wgrad<bf16_t>(nott_ctx, const nott_conv2d_desc*, const bf16_t*, const bf16_t*, float*, int);

}  // namespace conv_fast
}  // namespace nott
