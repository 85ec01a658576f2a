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
//     zero column on both sides (row pitch P = W+2 rounded up to odd), so
//     that each of the 9 taps is a plain row offset ((r−1)·P + s−1) into the
//     same LDS data and image borders read zeros;
//   * the 9 × 64 × chunk weight slice, pre-arranged by conv3x3_wprep_kernel.
// Each wave then runs 9 taps × (4 pixel tiles × 4 channel tiles) of
// v_mfma_f32_16x16x32_bf16 (or 4× v_mfma_f32_16x16x4f32), loading the next
// tap's operands while the current tap's MFMAs run.  LDS rows are 64 bytes,
// grouped by 16 (lds_off) so that 16 consecutive rows read by one MFMA
// operand hit distinct banks.
//
// conv3x3_wgrad_kernel computes dw[k, c, r, s] = Σ_{n,h,w} dy[n,k,h,w] ·
// x[n, c, h−1+r, w−1+s] (ATen convolution_backward, weight grad).
#include "conv_tile.hpp"

#include <algorithm>

namespace nott {
namespace conv_fast {
namespace {


struct SameParams {
    int32_t n, cin, h, w, cout;
    int32_t hw, w2;            // h·w, LDS row pitch of a padded image row (odd, ≥ w+2)
    int32_t npix;              // n·h·w
    int32_t in_rows;           // LDS rows reserved for the input tile
    int32_t remap;             // XCD-aware block remap active
    int32_t vec_store;         // 16-byte output runs stay inside one image plane
    int32_t relu;              // ReLU on the output (forward with a fused activation)
    int32_t cc_per_split;      // channel chunks per split (blockIdx.z, or per tail piece)
    int32_t remap_n;           // blocks under the XCD remap (a multiple of 8)
    int32_t tail_first;        // tail split: blocks ≥ tail_first are pieces of tiles ≥ tail_first
    int32_t tail_splits;       // pieces per tail tile (0: no tail split)
    int32_t part_m0, part_npix;   // pixels [part_m0, part_m0 + part_npix) have partials
    float* partial;            // split partials [split][cout][part_npix] (fp32, no bias), or null
    FastDiv fd_hw, fd_w, fd_w2, fd_h2;
};

// Weight slices from w (fwd) or from its flipped transpose (dgrad): slice
// (cb, cc) holds rows (tap, co) = tap·64 + co of CC channels, stored in the
// LDS order of lds_off(row, sub) (16-row groups, sub-chunk-major inside a
// group), so the kernels copy a slice to LDS linearly: contiguous 16-byte
// pieces per lane, bank-conflict-free writes.  Grid: x over one slice's
// 9·64·CC elements, y = channel chunk cc, z = 64-channel block cb; the
// fastest thread index runs over the source's contiguous dimension.
template <typename T, bool DGRAD>
__global__ __launch_bounds__(256) void conv3x3_wprep_kernel(const T* __restrict__ w, T* __restrict__ wp, int32_t cout,
                                                            int32_t cin) {
    // Slices cover whole 64-channel blocks; channels from cout up to the
    // block end are zero weights.
    constexpr int CC = Chunk<T>::CC, SUB = Chunk<T>::SUB;
    constexpr int32_t SLICE = 9 * kTileCo * CC;
    const int32_t j = (int32_t)blockIdx.x * 256 + (int32_t)threadIdx.x;
    if (j >= SLICE) return;
    const int32_t cc = blockIdx.y, cb = blockIdx.z;
    const int32_t tap = j / (kTileCo * CC), rem = j % (kTileCo * CC);
    // fwd reads w[co][ci][r][s] (ci fastest); dgrad reads w[k = ci][c = co] (co fastest).
    const int32_t cil = DGRAD ? rem / kTileCo : rem % CC;
    const int32_t col = DGRAD ? rem % kTileCo : rem / CC;
    const int32_t co = cb * kTileCo + col, ci = cc * CC + cil;
    const int32_t r = tap / 3, s = tap % 3;
    // fwd: wt[co][ci][r][s] = w[co][ci][r][s]; dgrad: wt[co=c][ci=k][r][s] = w[k][c][2-r][2-s]
    // (in dgrad terms w is [k = cin][c = cout][3][3]).
    const int64_t src = DGRAD ? (((int64_t)ci * cout + co) * 9 + (2 - r) * 3 + (2 - s))
                              : (((int64_t)co * cin + ci) * 9 + r * 3 + s);
    const int64_t slice = ((int64_t)cb * (cin / CC) + cc) * SLICE;
    T val = T(0);
    if (co < cout) val = w[src];
    wp[slice + (int64_t)(lds_off(tap * kTileCo + col, cil / SUB) >> 4) * SUB + cil % SUB] = val;
}


// Both layouts of one weight tensor in one launch: blockIdx.z below cbf
// writes the forward slices (conv3x3_wprep_kernel<T, false> of w as
// [cout][cin]), the rest the data-gradient slices (<T, true>, cout and cin
// exchanged) into wd.
template <typename T>
__global__ __launch_bounds__(256) void conv3x3_wprep2_kernel(const T* __restrict__ w, T* __restrict__ wf,
                                                             T* __restrict__ wd, int32_t cout, int32_t cin,
                                                             int32_t cbf) {
    constexpr int CC = Chunk<T>::CC, SUB = Chunk<T>::SUB;
    constexpr int32_t SLICE = 9 * kTileCo * CC;
    const int32_t j = (int32_t)blockIdx.x * 256 + (int32_t)threadIdx.x;
    const bool dg = (int32_t)blockIdx.z >= cbf;
    // in the data gradient's terms the input channels are cout, the outputs cin
    const int32_t ocount = dg ? cin : cout, icount = dg ? cout : cin;
    const int32_t cc = blockIdx.y, cb = dg ? (int32_t)blockIdx.z - cbf : (int32_t)blockIdx.z;
    if (j >= SLICE || cc >= icount / CC) return;
    const int32_t tap = j / (kTileCo * CC), rem = j % (kTileCo * CC);
    const int32_t cil = dg ? rem / kTileCo : rem % CC;
    const int32_t col = dg ? rem % kTileCo : rem / CC;
    const int32_t co = cb * kTileCo + col, ci = cc * CC + cil;
    const int32_t r = tap / 3, s = tap % 3;
    const int64_t src = dg ? (((int64_t)ci * cin + co) * 9 + (2 - r) * 3 + (2 - s))
                           : (((int64_t)co * cin + ci) * 9 + r * 3 + s);
    T val = T(0);
    if (co < ocount) val = w[src];
    T* dst = dg ? wd : wf;
    const int64_t slice = ((int64_t)cb * (icount / CC) + cc) * SLICE;
    dst[slice + (int64_t)(lds_off(tap * kTileCo + col, cil / SUB) >> 4) * SUB + cil % SUB] = val;
}

// The same two layouts when cout and cin are whole 64-channel blocks (no zero
// rows), one 16-byte destination chunk per thread and tap: thread t < cout·cin/SUB
// takes output channel co and the SUB input channels ci0.. of the forward
// slices and reads their 9·SUB weights as one contiguous run; the rest take
// (c, k0..) of the data-gradient slices, reading SUB runs of 9.
template <typename T>
__global__ __launch_bounds__(256) void conv3x3_wprep2v_kernel(const T* __restrict__ w, T* __restrict__ wf,
                                                              T* __restrict__ wd, int32_t cout, int32_t cin) {
    constexpr int CC = Chunk<T>::CC, SUB = Chunk<T>::SUB;
    constexpr int32_t SLICE = 9 * kTileCo * CC;
    constexpr int EB = (int)sizeof(T);
    const int64_t per = (int64_t)cout * (cin / SUB);
    int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const bool dg = t >= per;
    if (dg) t -= per;
    if (t >= per) return;
    // v[tap] holds the SUB input channels' weights of one tap, packed
    uint32_t v[9][SUB * EB / 4];
    int32_t co, ci0, icount;
    if (!dg) {
        co = (int32_t)(t / (cin / SUB));
        ci0 = (int32_t)(t % (cin / SUB)) * SUB;
        icount = cin;
        // 9·SUB contiguous weights w[co][ci0 + e][tap] (144 bytes, 16-byte aligned)
        const u32x4* src = reinterpret_cast<const u32x4*>(w + ((int64_t)co * cin + ci0) * 9);
        uint32_t raw[9 * SUB * EB / 4];
#pragma unroll
        for (int q = 0; q < 9 * SUB * EB / 16; ++q) {
            const u32x4 u = src[q];
            raw[4 * q] = u.x; raw[4 * q + 1] = u.y; raw[4 * q + 2] = u.z; raw[4 * q + 3] = u.w;
        }
#pragma unroll
        for (int tap = 0; tap < 9; ++tap) {
            if constexpr (EB == 4) {
#pragma unroll
                for (int e = 0; e < SUB; ++e) v[tap][e] = raw[e * 9 + tap];
            } else {
#pragma unroll
                for (int e = 0; e < SUB; e += 2) {
                    const int j0 = e * 9 + tap, j1 = (e + 1) * 9 + tap;   // element indices in the run
                    const uint32_t lo = (raw[j0 >> 1] >> (16 * (j0 & 1))) & 0xffffu;
                    const uint32_t hi = (raw[j1 >> 1] >> (16 * (j1 & 1))) & 0xffffu;
                    v[tap][e / 2] = lo | (hi << 16);
                }
            }
        }
    } else {
        // the data gradient's pass: output channel co = c, input channels k0 ..
        co = (int32_t)(t / (cout / SUB));
        ci0 = (int32_t)(t % (cout / SUB)) * SUB;
        icount = cout;
        const T* src = w + ((int64_t)ci0 * cin + co) * 9;
#pragma unroll
        for (int tap = 0; tap < 9; ++tap) {
            uint32_t x[SUB];
#pragma unroll
            for (int e = 0; e < SUB; ++e) {
                T val = src[(int64_t)e * cin * 9 + (8 - tap)];
                if constexpr (EB == 4) x[e] = __builtin_bit_cast(uint32_t, val);
                else x[e] = (uint32_t)__builtin_bit_cast(uint16_t, val);
            }
#pragma unroll
            for (int e = 0; e < SUB * EB / 4; ++e) v[tap][e] = EB == 4 ? x[e] : (x[2 * e] | (x[2 * e + 1] << 16));
        }
    }
    T* dst = dg ? wd : wf;
    const int64_t slice = ((int64_t)(co / kTileCo) * (icount / CC) + ci0 / CC) * SLICE;
#pragma unroll
    for (int tap = 0; tap < 9; ++tap)
        *reinterpret_cast<u32x4*>(dst + slice + (int64_t)(lds_off(tap * kTileCo + co % kTileCo, (ci0 % CC) / SUB) >> 4) * SUB) =
            u32x4{v[tap][0], v[tap][1], v[tap][2], v[tap][3]};
}

template <typename T, bool VEC, int LW>
__global__ __launch_bounds__(kThreads, 2) void conv3x3_same_kernel(const T* __restrict__ in, const T* __restrict__ wp,
                                                                  const float* __restrict__ bias, T* __restrict__ out,
                                                                  SameParams p) {
    constexpr int CC = Chunk<T>::CC, SUB = Chunk<T>::SUB;
    constexpr int VT = VEC ? VecTasks<T>::VT : 1;
    extern __shared__ __attribute__((aligned(16))) char smem[];
    char* lds_in = smem;
    char* lds_w = smem + p.in_rows * kRowB;

    // Block -> pixel tile.  Consecutive tiles share halo rows; with the
    // remap, tiles that run on the same XCD (block ids ≡ mod 8) are adjacent.
    // Tail split (one channel block, more tiles than one round of slots):
    // blocks below tail_first are whole tiles, the rest are tail_splits
    // channel-chunk pieces of each later tile, which fill the slots that the
    // last whole tiles leave free instead of running a round of their own.
    int32_t tile = blockIdx.x, split = blockIdx.z;
    bool part = p.partial != nullptr;
    int32_t cc0 = split * p.cc_per_split, cc1 = min(p.cin / CC, cc0 + p.cc_per_split);
    if (p.tail_splits > 0) {
        if (tile >= p.tail_first) {
            const int32_t q = tile - p.tail_first;
            tile = p.tail_first + q / p.tail_splits;
            split = q - (tile - p.tail_first) * p.tail_splits;
            cc0 = split * p.cc_per_split;
            cc1 = min(p.cin / CC, cc0 + p.cc_per_split);
        } else {
            part = false;
            cc0 = 0;
            cc1 = p.cin / CC;
        }
    }
    if (p.remap && tile < p.remap_n)
        tile = (int32_t)((tile & 7) * (p.remap_n >> 3) + (tile >> 3));
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
    const int32_t nvr = v_hi - v_lo + 1;                              // padded image rows in the tile
    const int32_t nrows = nvr * p.w2;                                 // LDS rows used by this tile

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
    // LDS byte offsets of this lane's A fragments for every tap, and of its B
    // fragments (tap · 4 + nt)·1024 past boff: the tap loop does no address
    // arithmetic.
    // Offsets are below 64 KiB: two per register.
    uint32_t aoff2[9][2];
#pragma unroll
    for (int tap = 0; tap < 9; ++tap)
#pragma unroll
        for (int h = 0; h < 2; ++h)
            aoff2[tap][h] = (uint32_t)lds_off(abase[2 * h] + (tap / 3 - 1) * p.w2 + (tap % 3 - 1), kq) |
                            ((uint32_t)lds_off(abase[2 * h + 1] + (tap / 3 - 1) * p.w2 + (tap % 3 - 1), kq) << 16);
    auto aoff = [&](int tap, int mt) -> uint32_t {
        return (mt & 1) ? (aoff2[tap][mt >> 1] >> 16) : (aoff2[tap][mt >> 1] & 0xffffu);
    };
    const int32_t boff = lds_off(r16, kq);

    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Channel chunks [cc0, cc1) of this split or piece (all of them for a whole tile).
    const T* wblk = wp + (int64_t)cb * (p.cin / CC) * 9 * kTileCo * CC;

    // Vector fill: task = (w-chunk of SUB pixels, padded row, channel group of
    // SUB): SUB 16-byte loads (one per channel), a register transpose, SUB
    // 16-byte LDS writes (one per pixel).  Halo rows / columns are zeroed once.
    // Task order: the fastest lanes take WG consecutive w-chunks, then padded
    // rows, then channel groups.  With an odd row pitch the 16 lanes of a
    // quarter-wave then start their SUB-row runs at 16 distinct rows mod 16,
    // so each of the SUB transposed writes is conflict-free.
    constexpr int WG = 16 / SUB;
    const int32_t wchunks = (p.w + SUB - 1) / SUB;      // the last chunk of a row may be partial
    const int32_t wgroups = (wchunks + WG - 1) / WG;
    const int32_t ntask = nvr * wgroups * WG * 4;
    auto task_of = [&](int32_t t, int32_t& wc, int32_t& vr, int32_t& cig) {
        const int32_t u = t / WG, u2 = u / nvr;
        vr = u - u2 * nvr;
        cig = u2 / wgroups;
        wc = (u2 - cig * wgroups) * WG + (t % WG);
    };
    u32x4 rin[VT][SUB];
    // VEC fill task t of chunk cc: SUB global loads into r ...
    auto fetch_task = [&](int32_t t, int32_t cc, u32x4 (&r)[SUB]) {
        int32_t wc, vr, cig;
        task_of(t, wc, vr, cig);
        uint32_t img, hh;
        p.fd_h2.divmod((uint32_t)(v_lo + vr), img, hh);
        const int32_t h = (int32_t)hh - 1;
        if (t < ntask && wc < wchunks && h >= 0 && h < p.h) {
            const T* src = in + (((int64_t)img * p.cin + cc * CC + cig * SUB) * p.h + h) * p.w;
#pragma unroll
            for (int i = 0; i < SUB; ++i) r[i] = load_chunk<T, LW, true>(src + (int64_t)i * p.hw, wc, p.w);
        }
    };
    // ... and the transpose + SUB LDS row writes into buffer `dst`.
    auto stash_task = [&](int32_t t, const u32x4 (&r)[SUB], char* dst) {
        int32_t wc, vr, cig;
        task_of(t, wc, vr, cig);
        uint32_t img, hh;
        p.fd_h2.divmod((uint32_t)(v_lo + vr), img, hh);
        const int32_t h = (int32_t)hh - 1;
        if (t < ntask && wc < wchunks && h >= 0 && h < p.h) {
            u32x4 tr[SUB];
            transpose_block(r, tr);
            const int32_t row0 = vr * p.w2 + 1 + wc * SUB;
#pragma unroll
            for (int i = 0; i < SUB; ++i)     // pixels past the row end stay zero (right halo)
                if (LW == 16 || wc * SUB + i < p.w) *reinterpret_cast<u32x4*>(dst + lds_off(row0 + i, cig)) = tr[i];
        }
    };
    // Fill of chunk cc: VEC tasks from the registers loaded by fetch_task, or
    // element loads straight into packed LDS rows; then the weight slice.
    constexpr int WT = (9 * kTileCo * 4) / kThreads;    // weight chunks per thread per channel chunk
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
            for (int32_t t = threadIdx.x; t < nrows * 4; t += kThreads) {
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
        }
        const u32x4* wsrc = reinterpret_cast<const u32x4*>(wblk + (int64_t)cc * 9 * kTileCo * CC);
        u32x4 rw[WT];
#pragma unroll
        for (int j = 0; j < WT; ++j) rw[j] = wsrc[threadIdx.x + j * kThreads];
#pragma unroll
        for (int j = 0; j < WT; ++j) *reinterpret_cast<u32x4*>(lds_w + (threadIdx.x + j * kThreads) * 16) = rw[j];
    };

    if constexpr (VEC) {
        // Halo rows / columns stay zero; the fill writes interior rows only.
        for (int32_t t = threadIdx.x; t < ((nrows + 15) >> 4) * 64; t += kThreads)
            *reinterpret_cast<u32x4*>(lds_in + t * 16) = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
        for (int j = 0; j < VT; ++j) fetch_task(threadIdx.x + j * kThreads, cc0, rin[j]);
    }
    for (int32_t cc = cc0; cc < cc1; ++cc) {
        __syncthreads();     // previous chunk fully read (and, at cc = 0, the halo zeroing done)
        stash(cc);
        __syncthreads();
        if constexpr (VEC) {
            if (cc + 1 < cc1) {
#pragma unroll
                for (int j = 0; j < VT; ++j) fetch_task(threadIdx.x + j * kThreads, cc + 1, rin[j]);
            }
        }
        // 9 taps × 16 MFMAs with the next tap's 8 operand fragments loaded
        // while the current tap's MFMAs run (LDS addresses precomputed).
        u32x4 a[2][4], b[2][4];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) a[0][mt] = *reinterpret_cast<const u32x4*>(lds_in + aoff(0, mt));
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) b[0][nt] = *reinterpret_cast<const u32x4*>(lds_w + boff + nt * 1024);
#pragma unroll
        for (int tap = 0; tap < 9; ++tap) {
            const int cur = tap & 1, nxt = cur ^ 1;
            if (tap + 1 < 9) {
#pragma unroll
                for (int mt = 0; mt < 4; ++mt)
                    a[nxt][mt] = *reinterpret_cast<const u32x4*>(lds_in + aoff(tap + 1, mt));
#pragma unroll
                for (int nt = 0; nt < 4; ++nt)
                    b[nxt][nt] = *reinterpret_cast<const u32x4*>(lds_w + boff + ((tap + 1) * 4 + nt) * 1024);
            }
            // keep the next tap's loads ahead of this tap's MFMAs
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                for (int nt = 0; nt < 4; ++nt) mfma_chunk<T>(a[cur][mt], b[cur][nt], acc[mt][nt]);
        }
    }

    if (part) {
        // Split-K: fp32 partial sums straight from the accumulators; lane holds
        // pixels 4·(lane/16) + e (consecutive, 16-byte aligned) of column co.
        float* dst = p.partial + (int64_t)split * p.cout * p.part_npix;
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) {
            const int32_t co = cb * kTileCo + nt * 16 + r16;
            if (co >= p.cout) continue;
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
                const int32_t m = m0 + wid * 64 + mt * 16 + kq * 4, ml = m - p.part_m0;
                if (m + 3 <= m_last) {
                    *reinterpret_cast<f32x4*>(dst + (int64_t)co * p.part_npix + ml) = acc[mt][nt];
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (m + e <= m_last) dst[(int64_t)co * p.part_npix + ml + e] = acc[mt][nt][e];
                }
            }
        }
        return;
    }

    // ---- epilogue: the 256-pixel × 64-channel tile goes through LDS as
    // [co][pixel] rows so that global stores are whole 16-byte runs of one
    // output plane.  Lane holds column co = nt·16 + (lane % 16) and pixels
    // 4·(lane/16) + e of each 16×16 accumulator tile.
    __syncthreads();                       // all waves done with the input/weight tiles
    constexpr int OP = kTilePix * (int)sizeof(T) + 16;   // LDS bytes per channel row
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
    constexpr int E16 = 16 / (int)sizeof(T);                 // pixels per 16-byte run
    constexpr int RUNS = kTilePix / E16;                      // runs per channel row
    const bool whole = p.vec_store != 0;                      // runs never cross an image or the tensor end
    for (int t = threadIdx.x; t < kTileCo * RUNS; t += kThreads) {
        const int col = t / RUNS, j = t % RUNS;
        const int32_t m = m0 + j * E16;
        const int32_t co = cb * kTileCo + col;
        if (m > m_last || co >= p.cout) continue;
        const char* src = lds_o + col * OP + j * 16;
        uint32_t n, hw;
        p.fd_hw.divmod((uint32_t)m, n, hw);
        if (whole && m + E16 - 1 <= m_last) {
            *reinterpret_cast<u32x4*>(out + ((int64_t)n * p.cout + co) * p.hw + hw) =
                *reinterpret_cast<const u32x4*>(src);
        } else {
            for (int e = 0; e < E16 && m + e <= m_last; ++e) {
                uint32_t ne, hwe;
                p.fd_hw.divmod((uint32_t)(m + e), ne, hwe);
                out[((int64_t)ne * p.cout + co) * p.hw + hwe] = reinterpret_cast<const T*>(src)[e];
            }
        }
    }
}

// out[n][co][hw] = bias[co] + Σ_split partial[split][co][m − m0] for the
// npix pixels m = n·hw + hw from m0 on (m0 a multiple of 4), splits added in
// order.  Thread = 4 consecutive pixels of one channel.
template <typename T>
__global__ __launch_bounds__(256) void conv3x3_split_reduce_kernel(const float* __restrict__ partial, int32_t splits,
                                                                   int32_t cout, int32_t m0, int32_t npix,
                                                                   FastDiv fd_hw, int32_t hw,
                                                                   const float* __restrict__ bias,
                                                                   T* __restrict__ out, int relu) {
    const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;     // group of 4 pixels
    const int32_t groups = npix >> 2;
    if (q >= (int64_t)groups * cout) return;
    const int32_t co = (int32_t)(q / groups), ml = (int32_t)(q - (int64_t)co * groups) * 4, m = m0 + ml;
    const int64_t stride = (int64_t)cout * npix;
    const f32x4 s = ordered_sum4(partial + (int64_t)co * npix + ml, stride, splits);
    const float bv = bias ? bias[co] : 0.f;
    f32x4 v;
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = relu ? relu_out(s[e] + bv) : s[e] + bv;
    if ((hw & 3) == 0) {
        // the 4 pixels lie in one image plane: one 4-element store
        uint32_t n, pix;
        fd_hw.divmod((uint32_t)m, n, pix);
        Vec4<T>::st(out + ((int64_t)n * cout + co) * hw + pix, v);
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            uint32_t n, pix;
            fd_hw.divmod((uint32_t)(m + e), n, pix);
            Io<T>::st(out, ((int64_t)n * cout + co) * hw + pix, v[e]);
        }
    }
}

bool same_shape(const nott_conv2d_desc* d) {
    return d->layout == NOTT_NCHW && d->groups == 1 && d->r == 3 && d->s == 3 && d->stride_h == 1 &&
           d->stride_w == 1 && d->pad_h == 1 && d->pad_w == 1 && d->dil_h == 1 && d->dil_w == 1 && d->w <= 64;
}

// LDS rows per padded image row: w + 2 (two halo columns), made odd so that
// rows of consecutive image rows start at distinct offsets mod 16.
int32_t row_pitch(int32_t w) { return (w + 2) | 1; }

int32_t in_rows_bound(int32_t h, int32_t w) {
    const int32_t hw = h * w;
    // A run of kTilePix pixels starting at any column touches at most
    // floor((kTilePix − 1 + w − 1)/w) + 1 image rows and, likewise, images;
    // each image adds its two halo rows.
    const int32_t rows = (kTilePix - 1 + w - 1) / w + 1;
    const int32_t imgs = (kTilePix - 1 + hw - 1) / hw + 1;
    return (rows + 2 * imgs) * row_pitch(w);
}

size_t same_lds_bytes(int32_t h, int32_t w, size_t elem) {
    const int32_t in_rows = (in_rows_bound(h, w) + 15) & ~15;   // whole 16-row LDS groups
    return std::max((size_t)in_rows * kRowB + (size_t)9 * kTileCo * kRowB, (size_t)kTileCo * (kTilePix * elem + 16));
}
constexpr size_t kSameLdsMax = 80 * 1024;   // two workgroups per CU


// Elements of the prepared weight slices of a cin → cout 3×3 pass.
int64_t prep_elems(int64_t cin, int64_t cout) { return ceil_div(cout, kTileCo) * kTileCo * cin * 9; }

// wsrc is w in the pass's own terms; `prepared` (optional) is its slices
// already written by a prep launch; `dg_out` (forward only, optional)
// receives the data gradient's slices of w from the same prep launch.
template <typename T, bool DGRAD>
int run_same(nott_ctx ctx, int32_t n, int32_t cin, int32_t h, int32_t w, int32_t cout, const T* in, const T* wsrc,
             const float* bias, T* out, int relu = 0, const T* prepared = nullptr, T* dg_out = nullptr) {
    constexpr int CC = Chunk<T>::CC;
    if constexpr (sizeof(T) == 2) {
        // bf16 shapes the DMA kernel takes.  Prepared slices of such a shape
        // are in its fragment layout, so that path has no fallback.
        const bool dma = (ctx->conv_dma & 1) && dma_applies(n, cin, h, w, cout);
        const bool aligned = ((uintptr_t)in & 15) == 0 && ((uintptr_t)out & 7) == 0;
        if (dma && (aligned || prepared)) {
            const bf16_t* wpp = prepared;
            // a forward whose data gradient takes the DMA kernel too: both
            // layouts from one prep launch
            const bool pair = !DGRAD && !wpp && dg_out && dma_applies(n, cout, h, w, cin);
            if (!wpp) {
                bf16_t* ws = static_cast<bf16_t*>(workspace(ctx, sizeof(T) * (size_t)dma_prep_elems(cin, cout)));
                if (!ws) return NOTT_ERR_ALLOC;
                const int st = pair ? dma_prep_pair(ctx, wsrc, ws, dg_out, cin, cout)
                                    : dma_prep<DGRAD>(ctx, wsrc, ws, cin, cout);
                if (st != NOTT_OK) return st;
                wpp = ws;
            }
            if (dg_out && !pair) {
                // the data gradient's pass is cout → cin over the same weight
                if ((ctx->conv_dma & 1) && dma_applies(n, cout, h, w, cin)) {
                    const int st = dma_prep<true>(ctx, wsrc, dg_out, cout, cin);
                    if (st != NOTT_OK) return st;
                } else {
                    hipLaunchKernelGGL((conv3x3_wprep_kernel<T, true>),
                                       dim3((unsigned)ceil_div(9 * kTileCo * CC, 256), (unsigned)(cout / CC),
                                            (unsigned)ceil_div(cin, kTileCo)),
                                       dim3(256), 0, ctx->stream, wsrc, dg_out, cin, cout);
                }
            }
            return dma_run(ctx, n, cin, h, w, cout, in, wpp, bias, out, relu);
        }
    }
    const int64_t cbc = ceil_div(cout, kTileCo);                 // 64-channel blocks (the last may be partial)
    const size_t wbytes = sizeof(T) * (size_t)cbc * kTileCo * cin * 9;
    const int32_t in_rows = (in_rows_bound(h, w) + 15) & ~15;   // whole 16-row LDS groups
    if (same_lds_bytes(h, w, sizeof(T)) > kSameLdsMax)
        return fail(ctx, NOTT_ERR_UNSUPPORTED, "conv3x3: tile does not fit in LDS");
    // Split the channel chunks over blockIdx.z when the grid leaves
    // workgroup slots (two per CU) idle (small images, many channels); split
    // only the tiles of a last, partly filled round when the grid has more
    // tiles than slots (one channel block).
    const int64_t tiles = ceil_div((int64_t)n * h * w, kTilePix);
    const int64_t blocks = tiles * cbc;
    const int64_t slots = 2 * (int64_t)ctx->num_cu;
    const int32_t nchunks = cin / CC;
    int32_t splits = 1, tail = 1;
    const int64_t npix64 = (int64_t)n * h * w;
    if (blocks < slots && nchunks > 1 && npix64 % 4 == 0)
        splits = pick_chunk_splits(blocks, nchunks, slots, sizeof(T));
    else if (cbc == 1 && nchunks > 1 && npix64 % 4 == 0)
        tail = pick_tail_splits(blocks, nchunks, slots, sizeof(T));
    const int32_t cc_per_split = (int32_t)ceil_div(nchunks, std::max(splits, tail));
    if (tail > 1)
        tail = (int32_t)ceil_div(nchunks, cc_per_split);
    else
        splits = (int32_t)ceil_div(nchunks, cc_per_split);
    const int64_t tail_tiles = tail > 1 ? blocks % slots : 0;
    const int64_t tail_first = tiles - tail_tiles;
    const int64_t part_m0 = tail > 1 ? tail_first * kTilePix : 0;
    const int64_t part_npix = npix64 - part_m0;
    const int32_t nsplit = std::max(splits, tail);      // partial planes
    const size_t wbytes_al = (wbytes + 255) & ~(size_t)255;
    const size_t pbytes = nsplit > 1 ? sizeof(float) * (size_t)nsplit * cout * (size_t)part_npix : 0;
    char* ws = static_cast<char*>(workspace(ctx, wbytes_al + pbytes));
    if (!ws) return NOTT_ERR_ALLOC;
    T* wp = reinterpret_cast<T*>(ws);
    if (prepared) {
        wp = const_cast<T*>(prepared);
    } else if (dg_out && sizeof(T) == 2 && (ctx->conv_dma & 1) && dma_applies(n, cout, h, w, cin)) {
        hipLaunchKernelGGL((conv3x3_wprep_kernel<T, DGRAD>), dim3((unsigned)ceil_div(9 * kTileCo * CC, 256),
                           (unsigned)(cin / CC), (unsigned)cbc), dim3(256), 0, ctx->stream, wsrc, wp, cout, cin);
        if constexpr (sizeof(T) == 2) {
            const int st = dma_prep<true>(ctx, wsrc, dg_out, cout, cin);
            if (st != NOTT_OK) return st;
        }
    } else if (dg_out && cout % kTileCo == 0 && cin % kTileCo == 0 && ((uintptr_t)wsrc & 15) == 0 &&
               ((uintptr_t)dg_out & 15) == 0) {
        const int64_t threads = 2 * (int64_t)cout * (cin / Chunk<T>::SUB);
        hipLaunchKernelGGL(conv3x3_wprep2v_kernel<T>, dim3((unsigned)ceil_div(threads, 256)), dim3(256), 0, ctx->stream,
                           wsrc, wp, dg_out, cout, cin);
    } else if (dg_out) {
        const int64_t cbd = ceil_div(cin, kTileCo);
        hipLaunchKernelGGL(conv3x3_wprep2_kernel<T>, dim3((unsigned)ceil_div(9 * kTileCo * CC, 256),
                           (unsigned)(std::max(cin, cout) / CC), (unsigned)(cbc + cbd)), dim3(256), 0, ctx->stream,
                           wsrc, wp, dg_out, cout, cin, (int32_t)cbc);
    } else {
        hipLaunchKernelGGL((conv3x3_wprep_kernel<T, DGRAD>), dim3((unsigned)ceil_div(9 * kTileCo * CC, 256),
                           (unsigned)(cin / CC), (unsigned)cbc), dim3(256), 0, ctx->stream, wsrc, wp, cout, cin);
    }
    SameParams p;
    p.n = n; p.cin = cin; p.h = h; p.w = w; p.cout = cout;
    p.hw = h * w; p.w2 = row_pitch(w); p.npix = n * h * w; p.in_rows = in_rows;
    p.fd_hw = FastDiv((uint32_t)(h * w));
    p.fd_w = FastDiv((uint32_t)w);
    p.fd_w2 = FastDiv((uint32_t)row_pitch(w));
    p.fd_h2 = FastDiv((uint32_t)(h + 2));
    p.cc_per_split = cc_per_split;
    p.relu = relu;
    p.partial = nsplit > 1 ? reinterpret_cast<float*>(ws + wbytes_al) : nullptr;
    p.tail_splits = tail > 1 ? tail : 0;
    p.tail_first = (int32_t)tail_first;
    p.part_m0 = (int32_t)part_m0;
    p.part_npix = (int32_t)part_npix;
    p.remap_n = (int32_t)tail_first;        // whole tiles (all of them without a tail split)
    p.remap = (tail_first % 8 == 0) ? 1 : 0;
    p.vec_store = ((h * w) % (16 / (int)sizeof(T)) == 0 && ((uintptr_t)out % 16) == 0) ? 1 : 0;
    // Vector fill when the input is 16-byte aligned and image rows split into
    // 16- or 8-byte pieces (narrower pieces measured slower than the element
    // fill).
    const int lw = wgrad_load_width(w, sizeof(T));
    const bool vec = ((uintptr_t)in % 16) == 0 && lw >= 8;
    const size_t lds = same_lds_bytes(h, w, sizeof(T));
    const void* fn = !vec      ? reinterpret_cast<const void*>(&conv3x3_same_kernel<T, false, 16>)
                     : lw == 16 ? reinterpret_cast<const void*>(&conv3x3_same_kernel<T, true, 16>)
                     : lw == 8  ? reinterpret_cast<const void*>(&conv3x3_same_kernel<T, true, 8>)
                     : lw == 4  ? reinterpret_cast<const void*>(&conv3x3_same_kernel<T, true, 4>)
                                : reinterpret_cast<const void*>(&conv3x3_same_kernel<T, true, sizeof(T) == 2 ? 2 : 4>);
    (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, 80 * 1024);
    const dim3 grid = tail > 1 ? dim3((unsigned)(tail_first + tail_tiles * tail), 1u, 1u)
                               : dim3((unsigned)tiles, (unsigned)cbc, (unsigned)splits);
    if (!vec)
        hipLaunchKernelGGL((conv3x3_same_kernel<T, false, 16>), grid, dim3(kThreads), lds, ctx->stream, in, wp, bias, out, p);
    else if (lw == 16)
        hipLaunchKernelGGL((conv3x3_same_kernel<T, true, 16>), grid, dim3(kThreads), lds, ctx->stream, in, wp, bias, out, p);
    else if (lw == 8)
        hipLaunchKernelGGL((conv3x3_same_kernel<T, true, 8>), grid, dim3(kThreads), lds, ctx->stream, in, wp, bias, out, p);
    else if (lw == 4)
        hipLaunchKernelGGL((conv3x3_same_kernel<T, true, 4>), grid, dim3(kThreads), lds, ctx->stream, in, wp, bias, out, p);
    else
        hipLaunchKernelGGL((conv3x3_same_kernel<T, true, sizeof(T) == 2 ? 2 : 4>), grid, dim3(kThreads), lds, ctx->stream,
                           in, wp, bias, out, p);
    if (nsplit > 1)
        hipLaunchKernelGGL(conv3x3_split_reduce_kernel<T>, dim3((unsigned)ceil_div(part_npix / 4 * cout, 256)), dim3(256),
                           0, ctx->stream, p.partial, nsplit, cout, p.part_m0, p.part_npix, p.fd_hw, p.hw, bias, out,
                           p.relu);
    return launch_status(ctx, "conv3x3_same");
}


// ---------------------------------------------------------------------------
// wgrad: dw[k, c, r, s] = Σ_{n,h,w} dy[n,k,h,w] · x[n, c, h−1+r, w−1+s]
//
// GEMM with M = 64 output channels k, N = 64 input channels c × 9 taps and
// the reduction over pixels.  Pixels live in "slots": image row h occupies
// slots [h·P, h·P + W) and slots [h·P + W, (h+1)·P) stay zero (P = W + 1
// rounded up to a power of two).  dy and x share the slot numbering, so a
// tap (r, s) is the slot offset (r−1)·P + (s−1) into x, and every pixel that
// falls off the image reads a zero slot.  The reduction runs over all slots
// of a band of TH rows (padding slots carry dy = 0).
//
// Per band, LDS holds dy[64 k][TH·P slots] and x[64 c][(TH+2)·P slots] (one
// halo row above and below) as 16-byte chunks of slots, stored chunk-major
// in groups of 16 channels: chunk j of channel ch sits in the 256-byte block
// (ch / 16, j) at slot (ch ^ 4·(j % 4)) % 16.  The 16 lanes that read one
// chunk of 16 channels, and the 16 lanes that fill 4 consecutive chunks of 4
// channels, both touch 16 distinct slots (conflict-free ds_read/ds_write_b128),
// and a lane's read slots depend on j % 4 only, which its k-slice fixes, so
// every read address is a per-lane base plus a compile-time offset.  x has
// one zero guard block before and after each channel group, read by the
// s = 0 / s = 2 shifts at the band edges.  A lane's
// MFMA k-slice is 8 (bf16) / 4 (fp32) consecutive slots: s = 1 is an aligned
// 16-byte LDS read, s = 0 and s = 2 realign it with one dword of each
// neighbouring chunk in registers.  Wave w owns channels 16w..16w+15 for all
// 9 taps and 32 of the 64 k: 18 accumulator tiles per 2 + 3 chunk reads
// (+ 6 dword reads); the next k-step's operands are read while the current
// one's 18 MFMAs run.
//
// The pixel range is split across workgroups (whole bands each); partial
// sums go to ws[split][tap][k][c] and conv3x3_wgrad_reduce_kernel adds them
// in split order (deterministic).
// ---------------------------------------------------------------------------
// 8 waves: wave w owns x channels 16·(w % 4)..+15 and dy channels
// 32·(w / 4)..+31, i.e. 2 × 9 accumulator tiles, so a wave fits in 256
// registers and two waves share each SIMD (one wave per SIMD cannot keep the
// matrix core busy).
constexpr int kWgThreads = 512;
template <typename T> struct WgCfg;
template <> struct WgCfg<bf16_t> { static constexpr int TH = 4, E = 8, KSTEP = 32; };
template <> struct WgCfg<float> { static constexpr int TH = 2, E = 4, KSTEP = 16; };
// Image rows per band.  bf16 slot rows of at most 16 elements (images up to
// 15 wide) take bands of 256 slots (8 k-steps) over the images stacked
// vertically with one zero row after each: a band's fill and barriers are
// then paid for by 8 k-steps instead of 1–2, and rows past an image's end
// are that zero row.  Other shapes keep one image per band (at 28×28,
// 8-row stacked bands measured slower than 4-row bands).
template <typename T, int P>
constexpr int wg_rows() {
    return (sizeof(T) == 2 && P <= 16) ? 256 / P : WgCfg<T>::TH;
}
template <typename T, int P>
constexpr bool wg_stacked() {
    return wg_rows<T, P>() != WgCfg<T>::TH;
}

struct WgradParams {
    int32_t n, c, k, h, w;
    int32_t bands_per_img, total_bands, bands_per_split;
    int32_t kblocks;
    FastDiv fd_h1;             // h + 1: stacked rows per image (stacked bands)
};

// Chunk j (16 bytes) of channel ch in a region of nch chunks per channel.
__device__ __forceinline__ int wg_off(int ch, int j, int nch) {
    return (ch >> 4) * (nch << 8) + (j << 8) + (((ch ^ ((j & 3) << 2)) & 15) << 4);
}

// Shift a 16-byte chunk by one element toward lower slots (s = 2: slots base+1..)
// or toward higher slots (s = 0: slots base−1..).
template <typename T>
__device__ __forceinline__ u32x4 shift_lo(const u32x4& cur, const u32x4& next);  // elements [1..E] of cur:next
template <typename T>
__device__ __forceinline__ u32x4 shift_hi(const u32x4& prev, const u32x4& cur);  // elements [E-1] of prev, [0..E-2] of cur
template <>
__device__ __forceinline__ u32x4 shift_lo<bf16_t>(const u32x4& c, const u32x4& n) {
    return u32x4{__builtin_amdgcn_alignbit(c.y, c.x, 16), __builtin_amdgcn_alignbit(c.z, c.y, 16),
                 __builtin_amdgcn_alignbit(c.w, c.z, 16), __builtin_amdgcn_alignbit(n.x, c.w, 16)};
}
template <>
__device__ __forceinline__ u32x4 shift_hi<bf16_t>(const u32x4& p, const u32x4& c) {
    return u32x4{__builtin_amdgcn_alignbit(c.x, p.w, 16), __builtin_amdgcn_alignbit(c.y, c.x, 16),
                 __builtin_amdgcn_alignbit(c.z, c.y, 16), __builtin_amdgcn_alignbit(c.w, c.z, 16)};
}
template <>
__device__ __forceinline__ u32x4 shift_lo<float>(const u32x4& c, const u32x4& n) { return u32x4{c.y, c.z, c.w, n.x}; }
template <>
__device__ __forceinline__ u32x4 shift_hi<float>(const u32x4& p, const u32x4& c) { return u32x4{p.w, c.x, c.y, c.z}; }

template <typename T, int P, int LW>
__global__ __launch_bounds__(kWgThreads, 1) void conv3x3_wgrad_kernel(const T* __restrict__ x, const T* __restrict__ dy,
                                                                   float* __restrict__ ws, WgradParams p) {
    constexpr int TH = wg_rows<T, P>(), E = WgCfg<T>::E, KSTEP = WgCfg<T>::KSTEP;
    constexpr bool STACK = wg_stacked<T, P>();
    constexpr int CPR = P / E;                          // 16-byte chunks per slot row
    constexpr int A_TOTAL = 64 * TH * CPR, B_TOTAL = 64 * (TH + 2) * CPR;   // 16-byte chunks per band
    constexpr int A_TASKS = (A_TOTAL + kWgThreads - 1) / kWgThreads;             // per thread
    constexpr int RB = P * (int)sizeof(T);              // bytes per slot row
    constexpr int KSTEPS = TH * P / KSTEP;
    constexpr int NA = TH * CPR;                        // dy chunks per channel
    constexpr int NB = (TH + 2) * CPR + 2;              // x chunks per channel, with the two guards
    extern __shared__ __attribute__((aligned(16))) char smem[];
    char* lds_a = smem;
    char* lds_b = smem + 64 * NA * 16;

    const int kb = blockIdx.y % p.kblocks, cb = blockIdx.y / p.kblocks;
    const int32_t b0 = blockIdx.x * p.bands_per_split;
    const int32_t b1 = min(p.total_bands, b0 + p.bands_per_split);
    const int wid = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r16 = lane & 15, kq = lane >> 4;
    const int cg = wid & 3, kh = wid >> 2;               // x channel group, dy channel half
    const int64_t plane = (int64_t)p.h * p.w;

    // Zero the guard chunks of x (never written by the fill).
    for (int i = threadIdx.x; i < 64 * 2; i += kWgThreads) {
        const int ch = i >> 1, j = (i & 1) ? NB - 1 : 0;
        *reinterpret_cast<u32x4*>(lds_b + wg_off(ch, j, NB)) = u32x4{0u, 0u, 0u, 0u};
    }

    f32x4 acc[2][9];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 9; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Fill task t: chunk j = 4·jh + t%4 of channel ch = 4·chh + (t/4)%4, with
    // (jh, chh) = t/16 split over the chunk quads of a channel: 16 lanes fill
    // 4 consecutive chunks of 4 channels (64-byte global runs).
    constexpr int NBF = (TH + 2) * CPR;                  // filled x chunks per channel
    constexpr int QA = NA / 4, QB = (NBF + 3) / 4;       // chunk quads per channel
    constexpr int A_TOTAL4 = 64 * QA * 16 / 4, B_TOTAL4 = 64 * QB * 16 / 4;
    static_assert(NA % 4 == 0, "dy chunks per channel must be a multiple of 4");
    static_assert(A_TOTAL4 == A_TOTAL, "task count");
    auto task = [](int t, int nq, int& ch, int& j) {
        const int rest = t >> 4;
        j = (rest % nq) * 4 + (t & 3);
        ch = (rest / nq) * 4 + ((t >> 2) & 3);
    };
    u32x4 ra[A_TASKS], rb[(B_TOTAL4 + kWgThreads - 1) / kWgThreads];
    // Rows of odd bf16 width (2-byte aligned) are read with the realigning
    // 16-byte loads, except in a band that reads the last image's last row
    // (whose loads would reach past the tensor): element loads there.  (At
    // 4-byte alignment the realigning loads measured slower than 4-byte
    // pieces.)
    auto fetch_rows = [&](int32_t band, auto fast_tag) __attribute__((always_inline)) {
        constexpr bool FAST = decltype(fast_tag)::value;
        auto load_row_chunk = [&](const T* row, int ch) __attribute__((always_inline)) -> u32x4 {
            if constexpr (FAST) return load_chunk_narrow(row, ch, p.w);
            else return load_chunk<T, LW>(row, ch, p.w);
        };
        // Band rows: image rows h0 .. h0 + TH − 1 of image img0, or stacked
        // rows h0 .. (row R = image R / (h + 1), row R % (h + 1); row h of
        // every image and rows past the last image are zero).
        int32_t img0 = 0, h0;
        if constexpr (STACK) {
            h0 = band * TH;
        } else {
            img0 = band / p.bands_per_img;
            h0 = (band - img0 * p.bands_per_img) * TH;
        }
        auto locate = [&](int32_t R, int32_t& img, int32_t& h) __attribute__((always_inline)) -> bool {
            if constexpr (STACK) {
                if (R < 0) return false;
                uint32_t q, r;
                p.fd_h1.divmod((uint32_t)R, q, r);
                img = (int32_t)q;
                h = (int32_t)r;
                return h < p.h && img < p.n;
            } else {
                img = img0;
                h = R;
                return R >= 0 && R < p.h;
            }
        };
#pragma unroll
        for (int i = 0; i < A_TASKS; ++i) {
            const int t = threadIdx.x + i * kWgThreads;
            int kk, j;
            task(t, QA, kk, j);
            const int ch = j % CPR;
            int32_t img, h;
            u32x4 v = u32x4{0u, 0u, 0u, 0u};
            if ((A_TOTAL % kWgThreads == 0 || t < A_TOTAL) && ch * E < p.w && locate(h0 + j / CPR, img, h))
                v = load_row_chunk(dy + ((int64_t)img * p.k + kb * 64 + kk) * plane + (int64_t)h * p.w, ch);
            ra[i] = v;
        }
#pragma unroll
        for (int i = 0; i < (B_TOTAL4 + kWgThreads - 1) / kWgThreads; ++i) {
            const int t = threadIdx.x + i * kWgThreads;
            int cc, j;
            task(t, QB, cc, j);
            const int ch = j % CPR;
            int32_t img, h;
            u32x4 v = u32x4{0u, 0u, 0u, 0u};
            if ((B_TOTAL4 % kWgThreads == 0 || t < B_TOTAL4) && j < NBF && ch * E < p.w && cb * 64 + cc < p.c &&
                locate(h0 - 1 + j / CPR, img, h))
                v = load_row_chunk(x + ((int64_t)img * p.c + cb * 64 + cc) * plane + (int64_t)h * p.w, ch);
            rb[i] = v;
        }
    };
    auto fetch = [&](int32_t band) __attribute__((always_inline)) {
        if constexpr (sizeof(T) == 2 && LW == 2) {
            // the last valid row of the last image: stacked row n(h+1) − 2,
            // or the last band of one-image bands
            const bool fast = STACK ? (int64_t)band * TH + TH < (int64_t)p.n * (p.h + 1) - 2
                                    : band + 1 < p.total_bands;
            if (fast) {
                fetch_rows(band, std::true_type{});
                return;
            }
        }
        fetch_rows(band, std::false_type{});
    };
    auto stash = [&]() {
#pragma unroll
        for (int i = 0; i < A_TASKS; ++i) {
            const int t = threadIdx.x + i * kWgThreads;
            int kk, j;
            task(t, QA, kk, j);
            if (A_TOTAL % kWgThreads == 0 || t < A_TOTAL)
                *reinterpret_cast<u32x4*>(lds_a + wg_off(kk, j, NA)) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < (B_TOTAL4 + kWgThreads - 1) / kWgThreads; ++i) {
            const int t = threadIdx.x + i * kWgThreads;
            int cc, j;
            task(t, QB, cc, j);
            if ((B_TOTAL4 % kWgThreads == 0 || t < B_TOTAL4) && j < NBF)
                *reinterpret_cast<u32x4*>(lds_b + wg_off(cc, 1 + j, NB)) = rb[i];
        }
    };

    // Per-lane LDS bases.  dy: chunk ja = 4·t + kq of channel (2·kh + mt)·16 + r16
    // is at a_base + mt·NA·256 + t·1024.  x: chunk j = 1 + 4·t + kq + r·CPR + d of
    // channel cl is at b_base[c] + (1 + 4·t + r·CPR + d)·256 with
    // c = (1 + r·CPR + d) % 4 (the slot depends on j % 4 = (kq + c) % 4).
    const int cl = cg * 16 + r16;                               // this lane's x channel
    const int a_base = kh * 2 * NA * 256 + kq * 256 + ((r16 ^ (kq << 2)) & 15) * 16;
    int b_base[4];
#pragma unroll
    for (int c = 0; c < 4; ++c)
        b_base[c] = (cl >> 4) * (NB << 8) + kq * 256 + (((cl ^ (((kq + c) & 3) << 2)) & 15) << 4);
    struct Ops {
        u32x4 a[2], cur[3];
        uint32_t prev_w[3], next_x[3];
    };
    auto load_ops = [&](int t, Ops& o) {
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
            o.a[mt] = *reinterpret_cast<const u32x4*>(lds_a + a_base + mt * NA * 256 + t * 1024);
#pragma unroll
        for (int r = 0; r < 3; ++r) {
            const int jc = 1 + 4 * t + r * CPR;                 // chunk of s = 1, less kq
            o.cur[r] = *reinterpret_cast<const u32x4*>(lds_b + b_base[(jc) & 3] + jc * 256);
            o.prev_w[r] = *reinterpret_cast<const uint32_t*>(lds_b + b_base[(jc + 3) & 3] + (jc - 1) * 256 + 12);
            o.next_x[r] = *reinterpret_cast<const uint32_t*>(lds_b + b_base[(jc + 1) & 3] + (jc + 1) * 256);
        }
    };
    if (b0 < b1) fetch(b0);
    for (int32_t band = b0; band < b1; ++band) {
        __syncthreads();
        stash();
        __syncthreads();
        if (band + 1 < b1) fetch(band + 1);
        Ops ops[2];
        load_ops(0, ops[0]);
#pragma unroll
        for (int t = 0; t < KSTEPS; ++t) {
            Ops& o = ops[t & 1];
            if (t + 1 < KSTEPS) load_ops(t + 1, ops[(t + 1) & 1]);
#pragma unroll
            for (int r = 0; r < 3; ++r) {
                const u32x4 pv = u32x4{0u, 0u, 0u, o.prev_w[r]}, nx = u32x4{o.next_x[r], 0u, 0u, 0u};
                const u32x4 b_s0 = shift_hi<T>(pv, o.cur[r]);
                const u32x4 b_s2 = shift_lo<T>(o.cur[r], nx);
#pragma unroll
                for (int mt = 0; mt < 2; ++mt) {
                    mfma_chunk<T>(o.a[mt], b_s0, acc[mt][r * 3 + 0]);
                    mfma_chunk<T>(o.a[mt], o.cur[r], acc[mt][r * 3 + 1]);
                    mfma_chunk<T>(o.a[mt], b_s2, acc[mt][r * 3 + 2]);
                }
            }
        }
    }
    // Partials in dw's own layout, ws[split][k][c][tap].  For each (mt, e) a
    // wave holds 4 k rows (one per 16-lane group) × its 16 channels × 9 taps,
    // i.e. 4 runs of 144 consecutive floats; they pass through the wave's own
    // LDS slice so that the global stores are whole 16-byte pieces.
    const int32_t c0 = cb * 64 + cg * 16;        // this wave's first channel
    float* wsp = ws + (int64_t)blockIdx.x * 9 * p.k * p.c;
    float* slice = reinterpret_cast<float*>(smem) + wid * (4 * 16 * 9);
    __syncthreads();                             // every wave is done with the band operands
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
#pragma unroll
            for (int tap = 0; tap < 9; ++tap) slice[(kq * 16 + r16) * 9 + tap] = acc[mt][tap][e];
            // the slice is this wave's own: wave-scope ordering suffices
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            __builtin_amdgcn_wave_barrier();
            // float4 piece i of run g (k = kb·64 + (kh·2 + mt)·16 + 4g + e): 36 per run
            for (int i = lane; i < 4 * 36; i += 64) {
                const int g = i / 36, j = i - g * 36;
                const int32_t k = kb * 64 + (kh * 2 + mt) * 16 + g * 4 + e;
                const int32_t cw = min(16, p.c - c0);   // channels of this wave inside c (whole groups of 16 or fewer)
                if (4 * j < cw * 9)
                    *reinterpret_cast<f32x4*>(wsp + ((int64_t)k * p.c + c0) * 9 + 4 * j) =
                        *reinterpret_cast<const f32x4*>(slice + g * 144 + 4 * j);
            }
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            __builtin_amdgcn_wave_barrier();
        }
}

// dw[k][c][tap] (+)= Σ_split ws[split][k][c][tap] (the partials share dw's
// layout, so reads and writes are contiguous float4 runs).  A block owns
// 256 / ZL float4 groups; thread t takes group t % G and the splits
// z ≡ t / G (mod ZL) in order, 8 loads in flight, and the ZL lane sums of a
// group combine in LDS in lane order, so the summation order is fixed.
// ZL = 4 (1 KB coalesced runs) for few splits, 16 for many (more loads in
// flight per group, four times the workgroups).  Requires 9·k·c % 4 == 0.
template <int ZL>
__global__ __launch_bounds__(256) void conv3x3_wgrad_reduce_kernel(const float* __restrict__ ws, int32_t splits,
                                                                   int32_t k, int32_t c, float* __restrict__ dw,
                                                                   int accumulate) {
    constexpr int G = 256 / ZL;
    __shared__ f32x4 red[ZL][G];
    const int gl = threadIdx.x % G, zl = threadIdx.x / G;
    const int64_t per = (int64_t)9 * k * c;
    const int64_t q = (int64_t)blockIdx.x * G + gl;   // float4 group: i = 4q = (tap·k + kk)·c + cc
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
    if (4 * q < per && zl < splits) {
        const int32_t n = (splits - zl + ZL - 1) / ZL;   // splits zl, zl + ZL, ...
        s = ordered_sum4(ws + 4 * q + (int64_t)zl * per, (int64_t)ZL * per, n);
    }
    red[zl][gl] = s;
    __syncthreads();
    if (zl != 0 || 4 * q >= per) return;
    f32x4 t = red[0][gl];
#pragma unroll
    for (int u = 1; u < ZL; ++u) t += red[u][gl];
    float* o = dw + 4 * q;
    if (((uintptr_t)dw & 15) == 0) {
        f32x4* o4 = reinterpret_cast<f32x4*>(o);
        *o4 = accumulate ? *o4 + t : t;
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = accumulate ? o[e] + t[e] : t[e];
    }
}


template <typename T, int P, int LW>
int run_wgrad(nott_ctx ctx, const nott_conv2d_desc* d, const T* x, const T* dy, float* dw, int accumulate) {
    constexpr int TH = wg_rows<T, P>();
    constexpr int RB = P * (int)sizeof(T);
    WgradParams p;
    p.n = (int32_t)d->n; p.c = (int32_t)d->c; p.k = (int32_t)d->k; p.h = (int32_t)d->h; p.w = (int32_t)d->w;
    p.bands_per_img = (p.h + TH - 1) / TH;
    p.total_bands = wg_stacked<T, P>() ? (int32_t)ceil_div((int64_t)p.n * (p.h + 1), TH) : p.n * p.bands_per_img;
    p.fd_h1 = FastDiv((uint32_t)(p.h + 1));
    p.kblocks = p.k / 64;
    constexpr int CPR = P * (int)sizeof(T) / 16;
    const int tiles = p.kblocks * (int)ceil_div(p.c, 64);
    // About one workgroup per CU in total.
    int64_t splits = std::max<int64_t>(1, std::min<int64_t>(p.total_bands, ceil_div((int64_t)ctx->num_cu, tiles)));
    p.bands_per_split = (int32_t)ceil_div(p.total_bands, splits);
    splits = ceil_div(p.total_bands, p.bands_per_split);
    // band operands, or the epilogue's 8 wave slices of 4·16·9 floats if larger
    const size_t lds = std::max<size_t>((size_t)64 * 16 * (TH * CPR + (TH + 2) * CPR + 2), 8 * 4 * 16 * 9 * sizeof(float));
    if (lds > 160 * 1024) return fail(ctx, NOTT_ERR_UNSUPPORTED, "conv3x3 wgrad: band does not fit in LDS");
    float* ws = static_cast<float*>(workspace(ctx, sizeof(float) * (size_t)splits * 9 * p.k * p.c));
    if (!ws) return NOTT_ERR_ALLOC;
    static bool attr_set = false;
    if (!attr_set) {
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&conv3x3_wgrad_kernel<T, P, LW>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        attr_set = true;
    }
    hipLaunchKernelGGL((conv3x3_wgrad_kernel<T, P, LW>), dim3((unsigned)splits, (unsigned)tiles), dim3(kWgThreads), lds,
                       ctx->stream, x, dy, ws, p);
    const int64_t per = (int64_t)9 * p.k * p.c;
    if (splits >= 32)
        hipLaunchKernelGGL(conv3x3_wgrad_reduce_kernel<16>, dim3((unsigned)ceil_div(per / 4, 16)), dim3(256), 0,
                           ctx->stream, ws, (int32_t)splits, p.k, p.c, dw, accumulate);
    else
        hipLaunchKernelGGL(conv3x3_wgrad_reduce_kernel<4>, dim3((unsigned)ceil_div(per / 4, 64)), dim3(256), 0,
                           ctx->stream, ws, (int32_t)splits, p.k, p.c, dw, accumulate);
    return launch_status(ctx, "conv3x3_wgrad");
}

int wgrad_slot_pitch(int64_t w) {
    int P = 8;
    while (P < w + 1) P <<= 1;
    return P;
}

}  // namespace

// Widest load (bytes) that keeps every image row's pieces aligned.
int wgrad_load_width(int64_t w, size_t elem) {
    for (int lw = 16; lw > (int)elem; lw >>= 1)
        if ((w * (int64_t)elem) % lw == 0) return lw;
    return (int)elem;
}

bool fwd_applies(const nott_conv2d_desc* d, size_t elem) {
    const int cc = elem == 2 ? Chunk<bf16_t>::CC : Chunk<float>::CC;
    // Output channels: whole 16-channel MFMA columns (the last 64-channel
    // block may be partial; its missing channels are zero weights).
    return same_shape(d) && d->c % cc == 0 && d->k % 16 == 0 &&
           same_lds_bytes((int32_t)d->h, (int32_t)d->w, elem) <= kSameLdsMax;
}

bool dgrad_applies(const nott_conv2d_desc* d, size_t elem) {
    const int cc = elem == 2 ? Chunk<bf16_t>::CC : Chunk<float>::CC;
    // dgrad's input channels are the conv's outputs (k), its outputs the conv's inputs (c).
    return same_shape(d) && d->k % cc == 0 && d->c % 16 == 0 &&
           same_lds_bytes((int32_t)d->h, (int32_t)d->w, elem) <= kSameLdsMax;
}

bool wgrad_applies(const nott_conv2d_desc* d, size_t elem) {
    // A slot row of at most 64, whole 64-channel blocks of dy and 16-channel
    // groups of x (a partial last x block loads zeros past c), image rows of
    // any width (narrower loads when rows are not whole 16-byte chunks).
    (void)elem;
    return same_shape(d) && wgrad_slot_pitch(d->w) <= 64 && d->k % 64 == 0 && d->c % 16 == 0;
}


template <typename T>
int fwd(nott_ctx ctx, const nott_conv2d_desc* d, const T* x, const T* w, const float* b, T* y, int relu) {
    return run_same<T, false>(ctx, (int32_t)d->n, (int32_t)d->c, (int32_t)d->h, (int32_t)d->w, (int32_t)d->k, x, w, b, y,
                              relu);
}

template <typename T>
int dgrad(nott_ctx ctx, const nott_conv2d_desc* d, const T* dy, const T* w, T* dx) {
    return run_same<T, true>(ctx, (int32_t)d->n, (int32_t)d->k, (int32_t)d->h, (int32_t)d->w, (int32_t)d->c, dy, w,
                             nullptr, dx);
}

// The forward with the data gradient's weight slices written by the same
// prep launch, and the data gradient from such slices.
template <typename T>
int fwd_prep(nott_ctx ctx, const nott_conv2d_desc* d, const T* x, const T* w, const float* b, T* y, int relu, T* wd) {
    return run_same<T, false>(ctx, (int32_t)d->n, (int32_t)d->c, (int32_t)d->h, (int32_t)d->w, (int32_t)d->k, x, w, b, y,
                              relu, nullptr, wd);
}

template <typename T>
int dgrad_prepared(nott_ctx ctx, const nott_conv2d_desc* d, const T* dy, const T* wd, T* dx) {
    return run_same<T, true>(ctx, (int32_t)d->n, (int32_t)d->k, (int32_t)d->h, (int32_t)d->w, (int32_t)d->c, dy, nullptr,
                             nullptr, dx, 0, wd);
}

int64_t dgrad_prep_elems(const nott_conv2d_desc* d) { return prep_elems(d->k, d->c); }

template <typename T, int LW>
int wgrad_p(nott_ctx ctx, const nott_conv2d_desc* d, const T* x, const T* dy, float* dw, int accumulate) {
    switch (wgrad_slot_pitch(d->w)) {
        case 8: return run_wgrad<T, 8, LW>(ctx, d, x, dy, dw, accumulate);
        case 16: return run_wgrad<T, 16, LW>(ctx, d, x, dy, dw, accumulate);
        case 32: return run_wgrad<T, 32, LW>(ctx, d, x, dy, dw, accumulate);
        default: return run_wgrad<T, 64, LW>(ctx, d, x, dy, dw, accumulate);
    }
}

template <typename T>
int wgrad(nott_ctx ctx, const nott_conv2d_desc* d, const T* x, const T* dy, float* dw, int accumulate) {
    if constexpr (sizeof(T) == 2) {
        const int32_t n = (int32_t)d->n, c = (int32_t)d->c, h = (int32_t)d->h, w = (int32_t)d->w, k = (int32_t)d->k;
        if ((ctx->conv_dma & 2) && wdma_applies(n, c, h, w, k) && ((uintptr_t)x & 15) == 0 && ((uintptr_t)dy & 15) == 0) {
            float* ws = nullptr;
            int32_t splits = 0;
            const int st = wdma_partials(ctx, n, c, h, w, k, x, dy, &ws, &splits);
            if (st != NOTT_OK) return st;
            const int64_t per = (int64_t)9 * k * c;
            if (splits >= 32)
                hipLaunchKernelGGL(conv3x3_wgrad_reduce_kernel<16>, dim3((unsigned)ceil_div(per / 4, 16)), dim3(256),
                                   0, ctx->stream, ws, splits, k, c, dw, accumulate);
            else
                hipLaunchKernelGGL(conv3x3_wgrad_reduce_kernel<4>, dim3((unsigned)ceil_div(per / 4, 64)), dim3(256),
                                   0, ctx->stream, ws, splits, k, c, dw, accumulate);
            return launch_status(ctx, "conv3x3_wgrad_reduce");
        }
    }
    switch (wgrad_load_width(d->w, sizeof(T))) {
        case 16: return wgrad_p<T, 16>(ctx, d, x, dy, dw, accumulate);
        case 8: return wgrad_p<T, 8>(ctx, d, x, dy, dw, accumulate);
        case 4: return wgrad_p<T, 4>(ctx, d, x, dy, dw, accumulate);
        default:
            if constexpr (sizeof(T) == 2) return wgrad_p<T, 2>(ctx, d, x, dy, dw, accumulate);
            else return wgrad_p<T, 4>(ctx, d, x, dy, dw, accumulate);
    }
}

template int fwd<float>(nott_ctx, const nott_conv2d_desc*, const float*, const float*, const float*, float*, int);
template int fwd<bf16_t>(nott_ctx, const nott_conv2d_desc*, const bf16_t*, const bf16_t*, const float*, bf16_t*, int);
template int dgrad<float>(nott_ctx, const nott_conv2d_desc*, const float*, const float*, float*);
template int dgrad<bf16_t>(nott_ctx, const nott_conv2d_desc*, const bf16_t*, const bf16_t*, bf16_t*);
template int fwd_prep<float>(nott_ctx, const nott_conv2d_desc*, const float*, const float*, const float*, float*, int,
                             float*);
template int fwd_prep<bf16_t>(nott_ctx, const nott_conv2d_desc*, const bf16_t*, const bf16_t*, const float*, bf16_t*,
                              int, bf16_t*);
template int dgrad_prepared<float>(nott_ctx, const nott_conv2d_desc*, const float*, const float*, float*);
template int dgrad_prepared<bf16_t>(nott_ctx, const nott_conv2d_desc*, const bf16_t*, const bf16_t*, bf16_t*);
template int wgrad<float>(nott_ctx, const nott_conv2d_desc*, const float*, const float*, float*, int);
template int wgrad<bf16_t>(nott_ctx, const nott_conv2d_desc*, const bf16_t*, const bf16_t*, float*, int);

}  // namespace conv_fast
}  // namespace nott
