// bf16 3x3 / stride 1 / pad 1 NCHW forward and data gradient with
// direct-to-LDS fills (gfx950).
//
//   out[n, co, p] = b[co] + Σ_{ci, r, s} wt[co, ci, r, s] · in[n, ci, p + (r−1)·W + (s−1)]
//
// with zeros outside the image: the forward (in = x, wt = w) and the data
// gradient (in = dy, wt[c, k, r, s] = w[k, c, 2−r, 2−s]) of reference
// conv.hpp:177 (ATen convolution / convolution_backward, input grad).
//
// Horizontal taps as output shifts.  With
//   Z_s[co, p] = Σ_{ci, r} wt[co, ci, r, s] · in[ci, p + (r−1)·W]
// (tap column s applied without its horizontal offset),
//   out[p] = Z_1[p] + Z_0[p−1]·[w(p) > 0] + Z_2[p+1]·[w(p) < W−1].
// The MFMA operands then read input pixels only at multiples of W from a
// 4-aligned pixel, so the raw NCHW rows can sit in LDS exactly as they lie in
// memory (copied by global_load_lds_dwordx4: no VGPR staging, no register
// transpose, no ds_write) and every fragment is an aligned transposing read
// (ds_read_b64_tr_b16: within each 16-lane group, lane i receives the 4
// channel-consecutive values of pixel i from a [channel][pixel] block).  The
// two shifts are applied once per tile to the accumulators: inside a lane's 4
// consecutive pixels they are a choice of register, across lane groups one
// ds_bpermute rotation per block.
//
// Work decomposition.  A tile is 448 pixels of whole image rows (W divides
// 112) × 32 output channels.  A workgroup is 8 waves: 4 pixel waves (112
// pixels = 7 blocks of 16 each) × 2 channel waves (16 channels each), so a
// wave holds 3 (taps s) × 7 (blocks) accumulator tiles of
// v_mfma_f32_16x16x32_bf16 with M = pixels, N = output channels and K = 32
// input channels per stage.  One workgroup per CU, persistent: workgroup b
// serves output block b / gpc and a contiguous range of that block's tiles,
// so the block's weight fragments (all input chunks, pre-arranged by
// dma_wprep_kernel in B-operand order) are copied into LDS once and stay
// resident; the blocks of one row band run at the same time on workgroups
// of the same XCD, which share the band's input rows through L2.
//
// Stages.  One stage = one 32-channel input chunk of one tile: the chunk's
// rows h0−1 .. h0+rows, a contiguous pixel range of each channel plane
// rounded out to 16-byte pieces (pieces off the image load from a zero
// block), in a 2-slot LDS ring ordered only by s_waitcnt vmcnt and a
// fence-free s_barrier.  The next stage's DMA instructions are issued
// between the MFMA blocks of the current one, so the vector memory queue
// drains while the matrix core works.  A tile's output is formed during the
// next tile's first stage, block by block, just before that block's
// accumulators restart, so the epilogue's shuffles, adds and stores overlap
// matrix work in flight rather than draining the matrix core.
#include "conv_fast.hpp"
#include "lds_dma.hpp"

#include <type_traits>

namespace nott {
namespace conv_fast {

using lds::barrier;
using lds::dma16;
using lds::lds_addr;
using lds::wait_vm_lgkm0;

namespace {

typedef short v4i16 __attribute__((ext_vector_type(4)));

constexpr int kPxWaves = 4;                 // pixel waves per workgroup
constexpr int kCoWaves = 2;                 // channel waves per workgroup (16 output channels each)
constexpr int kDWaves = kPxWaves * kCoWaves;
constexpr int kDThreads = 64 * kDWaves;
constexpr int kWavePx = 112;                // pixels per pixel wave: 7 blocks of 16
constexpr int kBlk = 7;
constexpr int kTilePxD = kPxWaves * kWavePx;   // pixels per tile
constexpr int kCoTile = 16 * kCoWaves;      // output channels per tile
constexpr int kCK = 32;                     // input channels per stage
constexpr int kWSlice = 9 * kCoWaves * 1024;   // weight bytes per input chunk: 9 taps × 2 channel waves × 1 KB
constexpr int kMaxIn = 6;                   // input DMA instructions per wave per stage (at most)
constexpr int kMaxLds = 160 * 1024;

// Read by the DMA lanes whose 16-byte piece lies above or below the image.
__device__ __attribute__((aligned(16))) uint32_t g_dma_zero[4];

struct DmaParams {
    int32_t n, cin, h, w, cout, hw;
    int32_t trows;       // image rows per tile (448 / w)
    int32_t tpi;         // tiles per image
    int32_t nchunks;     // 32-channel input chunks
    int32_t tiles_cb;    // tiles per output block: n · tpi
    int32_t gpc;         // workgroups per output block
    int32_t pb;          // LDS bytes per input channel row (≡ 32 mod 64)
    int32_t blk;         // LDS bytes per block of 8 channel rows: 8·pb + 128
    int32_t in_bytes;    // LDS bytes of a stage's input: 4·blk
    int32_t fbytes;      // bytes of each channel's pixel range that are loaded (≤ pb)
    int32_t in_instr;    // input DMA instructions per stage (in_bytes / 1024, rounded up)
    int32_t w_bytes;     // LDS bytes of the workgroup's resident weights: nchunks · kWSlice
};

struct TileInfo {
    int32_t img, h0, fs;   // image, first row, first loaded pixel (a multiple of 8, may be < 0)
};

__device__ __forceinline__ TileInfo decode_tile(int32_t t, const DmaParams& p) {
    TileInfo ti;
    ti.img = t / p.tpi;
    ti.h0 = (t - ti.img * p.tpi) * p.trows;
    ti.fs = ((ti.h0 - 1) * p.w) & ~7;      // rounds toward −∞
    return ti;
}

// Weight fragments: for output block cb (32 channels), input chunk c (32
// channels), tap t = 3r + s and channel wave cw, 1 KB in B-operand order:
// lane l's 16 bytes hold wt[co = 32cb + 16cw + l%16][ci = 32c + 8(l/16) + e],
// e = 0..7, at byte ((((cb·nch + c)·9 + t)·2 + cw)·64 + l)·16.
// Forward: w is [cout][cin][3][3]; data gradient: w is the conv weight
// [cin][cout][3][3] of this pass's terms, flipped.
// Source element of destination element i of a pass cin → cout.
template <bool DGRAD>
__device__ __forceinline__ int64_t dma_wprep_src(int64_t i, int32_t cin, int32_t cout) {
    const int32_t nch = cin / kCK;
    const int e = (int)(i & 7);
    const int64_t g = i >> 3;
    const int l = (int)(g & 63);
    int64_t q = g >> 6;
    const int cw = (int)(q % kCoWaves);
    q /= kCoWaves;
    const int t = (int)(q % 9);
    q /= 9;
    const int c = (int)(q % nch);
    const int cb = (int)(q / nch);
    const int32_t co = cb * kCoTile + cw * 16 + (l & 15);
    const int32_t ci = c * kCK + 8 * (l >> 4) + e;
    return DGRAD ? (((int64_t)ci * cout + co) * 9 + (8 - t)) : (((int64_t)co * cin + ci) * 9 + t);
}
template <bool DGRAD>
__global__ __launch_bounds__(256) void dma_wprep_kernel(const bf16_t* __restrict__ w, bf16_t* __restrict__ wp,
                                                        int32_t cin, int32_t cout) {
    // one element per thread (destination order, so stores are contiguous)
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)cout * cin * 9) return;
    wp[i] = w[dma_wprep_src<DGRAD>(i, cin, cout)];
}
// Both passes of one conv weight w [cout][cin][3][3] in one launch: the
// forward's slices (cin → cout) into wf and the data gradient's (cout → cin,
// flipped) into wd.
__global__ __launch_bounds__(256) void dma_wprep_pair_kernel(const bf16_t* __restrict__ w, bf16_t* __restrict__ wf,
                                                             bf16_t* __restrict__ wd, int32_t cin, int32_t cout) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)cout * cin * 9) return;
    wf[i] = w[dma_wprep_src<false>(i, cin, cout)];
    wd[i] = w[dma_wprep_src<true>(i, cout, cin)];
}

// LDS: [weights of the workgroup's output block, all input chunks][input
// slot 0][input slot 1].  Workgroup b serves output block b / gpc and a
// contiguous range of that block's tiles, so its weights are loaded once.
template <bool RELU>
__global__ __launch_bounds__(kDThreads, 1) void conv3x3_dma_kernel(const bf16_t* __restrict__ in,
                                                                   const bf16_t* __restrict__ wp,
                                                                   const float* __restrict__ bias,
                                                                   bf16_t* __restrict__ out, DmaParams p) {
    extern __shared__ __attribute__((aligned(1024))) char smem_raw[];
    char NOTT_LDS* smem = (char NOTT_LDS*)smem_raw;
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int pw = wid / kCoWaves, cw = wid % kCoWaves;
    const int G = lane >> 4, jl = lane & 15;

    const int32_t cb = (int32_t)blockIdx.x / p.gpc, gi = (int32_t)blockIdx.x - cb * p.gpc;
    const int32_t t0 = (int32_t)(((int64_t)gi * p.tiles_cb) / p.gpc);
    const int32_t t1 = (int32_t)(((int64_t)(gi + 1) * p.tiles_cb) / p.gpc);
    const int32_t nst = (t1 - t0) * p.nchunks;
    const int32_t co = cb * kCoTile + cw * 16 + jl;          // this lane's output channel
    const float bv = bias ? bias[co] : 0.f;

    // The block's weights, once: 1 KB per instruction.
    {
        const bf16_t* wsl = wp + (int64_t)cb * p.nchunks * (kWSlice / 2);
        const int32_t nw = p.nchunks * (kWSlice / 1024);
        for (int32_t wi = wid; wi < nw; wi += kDWaves)
            dma16(wsl + (int64_t)wi * 512 + lane * 8, lds_addr(smem) + (uint32_t)wi * 1024u);
    }

    // This lane's input pieces: instruction ii = wid + 8k moves LDS bytes
    // [1024·ii, 1024·ii + 1024) of a slot; lane piece s = 64·ii + lane lies
    // in channel block s / (blk/16), row (s % (blk/16)) / (pb/16) of it (rows
    // 8.. are the block's 128-byte gap), piece s % (pb/16) of that row.
    int32_t rel[kMaxIn], gpx[kMaxIn];
    {
        const int32_t ppc = p.pb >> 4, ppb = p.blk >> 4;
#pragma unroll
        for (int k = 0; k < kMaxIn; ++k) {
            const int32_t ii = wid + kDWaves * k;
            const int32_t s = ii * 64 + lane;
            const int32_t bi = s / ppb, rem = s - bi * ppb;
            const int32_t row = rem / ppc, g = rem - row * ppc;
            rel[k] = (8 * bi + row) * p.hw + 8 * g;
            gpx[k] = (row < 8 && 16 * g < p.fbytes) ? 8 * g : -(1 << 30);
        }
    }
    const void* zero = g_dma_zero;
    // Input DMA of stage sj into `slot`, instructions k in [k0, k1).
    struct Pending {
        const bf16_t* base;
        int32_t fs;
        uint32_t st;
    };
    auto prepare = [&](const TileInfo& ti, int32_t ch, int slot) -> Pending {
        Pending q;
        q.base = in + ((int64_t)ti.img * p.cin + (int64_t)ch * kCK) * p.hw + ti.fs;
        q.fs = ti.fs;
        q.st = lds_addr(smem) + (uint32_t)(p.w_bytes + slot * p.in_bytes);
        return q;
    };
    auto issue = [&](const Pending& q, int k0, int k1) {
#pragma unroll
        for (int k = k0; k < k1; ++k) {
            const int32_t ii = wid + kDWaves * k;
            if (ii < p.in_instr) {
                const int32_t px = q.fs + gpx[k];
                const void* src = (px >= 0 && px < p.hw) ? (const void*)(q.base + rel[k]) : zero;
                // the last instruction may reach past the slot: those lanes
                // (a bound on lane ids) do not load
                if (ii * 1024 + 1024 <= p.in_bytes || lane * 16 < p.in_bytes - ii * 1024)
                    dma16(src, q.st + (uint32_t)ii * 1024u);
            }
        }
    };

    // Row-edge masks of this lane's pixel groups (the same for every tile: a
    // pixel wave starts at a row start, since W divides 112): bit b of m0 /
    // m3 says the group of block b starts / ends a row.
    uint32_t m0 = 0, m3 = 0;
#pragma unroll
    for (int b = 0; b < kBlk; ++b) {
        const int32_t wq = (16 * b + 4 * G) % p.w;
        if (wq == 0) m0 |= 1u << b;
        if (wq + 4 == p.w) m3 |= 1u << b;
    }

    f32x4 z[3][kBlk];
    const int32_t rw2 = 2 * p.w;       // bytes per image row in LDS
    const int32_t hi = 4 * p.pb;       // the fragment's upper 4 channels
    const char NOTT_LDS* wb = smem + cw * 1024 + 16 * lane;
    // A tile's output is formed during the next tile's first stage, block by
    // block, just before that block's first MFMAs restart its accumulators:
    // the epilogue's shuffles, adds and stores then overlap matrix work
    // already in flight instead of draining the matrix core.
    bf16_t* pend_op = nullptr;      // this lane's first output pixel of the tile being written
    uint32_t pend_mask = 0;         // blocks of that tile that lie in the image
    // Epilogue pieces for the tile held in z (tile `et`).  Lane holds, for
    // output channel co, pixels 4G..4G+3 of each block; out = Z_1 (which
    // started from the bias) + Z_0 shifted right + Z_2 shifted left.
    // r0[b] = Z_0 at pixel 4G−1 (lane l−16's last pixel), r2[b] = Z_2 at
    // pixel 4G+4 (lane l+16's first).  (Elements are taken from the whole
    // vector's bit pattern: bit-casting z[.][b][3] alone compiled to a read
    // of element 0.)
    const int up = ((lane - 16) & 63) << 2, dn = ((lane + 16) & 63) << 2;
    float r0[kBlk], r2[kBlk];
    auto shuffle0 = [&](int b) {
        const u32x4 v = __builtin_bit_cast(u32x4, z[0][b]);
        r0[b] = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(up, (int)v.w));
    };
    auto shuffle2 = [&](int b) {
        const u32x4 v = __builtin_bit_cast(u32x4, z[2][b]);
        r2[b] = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(dn, (int)v.x));
    };
    auto epi_begin = [&](const TileInfo& et) {
        const int32_t qw = et.h0 * p.w + pw * kWavePx;
        pend_op = out + ((int64_t)et.img * p.cout + co) * p.hw + qw + 4 * G;
        // blocks whose group of this lane lies in the image (rows past the
        // image end in the last band are not stored)
        pend_mask = 0;
        const int32_t left = p.hw - (qw + 4 * G);
#pragma unroll
        for (int b = 0; b < kBlk; ++b)
            if (16 * b < left) pend_mask |= 1u << b;
    };
    auto epi_block = [&](int b) {
        // group 0 takes its left neighbour from the previous block's
        // group 3; group 3 its right neighbour from the next block's group 0
        const float left = G == 0 ? (b > 0 ? r0[b - 1] : 0.f) : r0[b];
        const float right = G == 3 ? (b + 1 < kBlk ? r2[b + 1] : 0.f) : r2[b];
        float o[4];
        o[0] = z[1][b][0] + ((m0 >> b) & 1 ? 0.f : left) + z[2][b][1];
        o[1] = z[1][b][1] + z[0][b][0] + z[2][b][2];
        o[2] = z[1][b][2] + z[0][b][1] + z[2][b][3];
        o[3] = z[1][b][3] + z[0][b][2] + ((m3 >> b) & 1 ? 0.f : right);
        if constexpr (RELU) {
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = relu_out(o[e]);
        }
        // stored right away: the rest of the stage's matrix work covers the
        // write acknowledgements that the next ring wait includes
        if ((pend_mask >> b) & 1)
            *reinterpret_cast<u32x2*>(pend_op + 16 * b) = u32x2{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
    };
    // Stage sj is chunk ch of tile cur; (nt, nch) is the stage after it.
    // Tiles advance by counters (no divisions in the loop).
    TileInfo cur = decode_tile(t0, p), prev = cur;
    if (nst > 0) issue(prepare(cur, 0, 0), 0, kMaxIn);
    int32_t ch = 0, sj = 0;
    // Accumulators start from the bias (Z_1) and zero (Z_0, Z_2).
    auto init_block = [&](int b) {
        z[0][b] = f32x4{0.f, 0.f, 0.f, 0.f};
        z[1][b] = f32x4{bv, bv, bv, bv};
        z[2][b] = f32x4{0.f, 0.f, 0.f, 0.f};
    };
#pragma unroll
    for (int b = 0; b < kBlk; ++b) init_block(b);
    // One stage.  EPI (the first chunk of a tile after the workgroup's
    // first): block by block, before the block's first MFMAs, it forms the
    // previous tile's output from the block's accumulators and restarts them.
    auto stage = [&](auto epi_tag) {
        constexpr bool EPI = decltype(epi_tag)::value;
        wait_vm_lgkm0<0>();
        barrier();
        const bool more = sj + 1 < nst;
        const bool last_chunk = ch + 1 == p.nchunks;
        TileInfo nt = cur;
        if (last_chunk) {
            nt.h0 += p.trows;
            if (nt.h0 >= p.h) {
                nt.h0 = 0;
                ++nt.img;
            }
            nt.fs = ((nt.h0 - 1) * p.w) & ~7;
        }
        const Pending nx = prepare(nt, last_chunk ? 0 : ch + 1, (sj + 1) & 1);

        const char NOTT_LDS* st = smem + p.w_bytes + (sj & 1) * p.in_bytes;
        // Transposing-read offset of this lane for block 0, tap row 0, low
        // channel half: channel row 8G + jl/4 (block G, row jl/4), pixel
        // (wave start − W) + 4·(jl % 4).  Blocks of 8 rows are 8·pb + 128
        // bytes apart, so the two 16-lane groups of a half-wave (rows k and
        // k + 8, 8·pb ≡ 0 mod 256) land on disjoint banks.
        const char NOTT_LDS* a0 =
            st + G * p.blk + (jl >> 2) * p.pb + 2 * (cur.h0 * p.w + pw * kWavePx - p.w - cur.fs + 4 * (jl & 3));
        const char NOTT_LDS* b0 = wb + ch * kWSlice;
        // Fragments: one set of A (7 blocks of this tap row) and two of B.
        // MFMAs go block by block (3 per block, one per tap column), and a
        // block's A registers are refilled with the next tap row as soon as
        // its 3 MFMAs are issued, 6 blocks of matrix work ahead of their use.
        v4i16 alo[kBlk], ahi[kBlk];
        u32x4 bw[2][3];
        auto load_a = [&](int r, int b) {
            const char NOTT_LDS* ar = a0 + r * rw2 + 32 * b;
            alo[b] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((v4i16 NOTT_LDS*)ar);
            ahi[b] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((v4i16 NOTT_LDS*)(ar + hi));
        };
        auto load_b = [&](int r, int buf) {
#pragma unroll
            for (int s = 0; s < 3; ++s) bw[buf][s] = *(const u32x4 NOTT_LDS*)(b0 + (r * 3 + s) * 2 * 1024);
        };
        // One tap row: 21 MFMAs.  The next stage's input DMA goes out two
        // instructions per tap row, between blocks, so the vector memory
        // queue drains while the matrix core works.
        auto taps = [&](int r) {
            if (r + 1 < 3) load_b(r + 1, (r + 1) & 1);
#pragma unroll
            for (int b = 0; b < kBlk; ++b) {
                if constexpr (EPI) {
                    if (r == 0) {
                        // shuffles one block ahead (their reads precede this
                        // block's overwrite), then this block's output
                        if (b + 1 < kBlk) {
                            shuffle0(b + 1);
                            if (b + 2 < kBlk) shuffle2(b + 2);
                        }
                        epi_block(b);
                        init_block(b);
                    }
                }
                const v4i16 av[2] = {alo[b], ahi[b]};
                const bf16x8 a = __builtin_bit_cast(bf16x8, av);
#pragma unroll
                for (int s = 0; s < 3; ++s)
                    z[s][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, __builtin_bit_cast(bf16x8, bw[r & 1][s]),
                                                                      z[s][b], 0, 0, 0);
                if (r + 1 < 3) load_a(r + 1, b);
                if (b == 1 && more) issue(nx, 2 * r, 2 * r + 1);
                if (b == 4 && more) issue(nx, 2 * r + 1, 2 * r + 2);
                // keeps the scheduler from hoisting later blocks' loads (and
                // their registers) above this block's MFMAs
                __builtin_amdgcn_sched_barrier(0);
            }
        };
#pragma unroll
        for (int b = 0; b < kBlk; ++b) load_a(0, b);
        load_b(0, 0);
        if constexpr (EPI) {
            epi_begin(prev);
            shuffle0(0);
            shuffle2(0);
            shuffle2(1);
        }
        taps(0);
        taps(1);
        taps(2);
        if (last_chunk) prev = cur;
        cur = nt;
        ch = last_chunk ? 0 : ch + 1;
        ++sj;
    };
    if (sj < nst) {
        for (int32_t c = 0; c < p.nchunks; ++c) stage(std::false_type{});
    }
    while (sj < nst) {
        stage(std::true_type{});
        for (int32_t c = 1; c < p.nchunks; ++c) stage(std::false_type{});
    }
    // the last tile's output, on its own
    if (nst > 0) {
        epi_begin(prev);
#pragma unroll
        for (int b = 0; b < kBlk; ++b) {
            shuffle0(b);
            shuffle2(b);
        }
#pragma unroll
        for (int b = 0; b < kBlk; ++b) epi_block(b);
    }
}

struct DmaPlan {
    DmaParams p;
    size_t lds;
    int64_t grid;
};

bool dma_plan(int32_t n, int32_t cin, int32_t h, int32_t w, int32_t cout, int num_cu, DmaPlan& pl) {
    if (w <= 0 || w % 4 != 0 || kWavePx % w != 0 || (int64_t)h * w % 8 != 0) return false;
    if (cin % kCK != 0 || cout % kCoTile != 0 || n <= 0 || h <= 0) return false;
    if ((int64_t)n * cin * h * w >= (int64_t(1) << 31) || (int64_t)n * cout * h * w >= (int64_t(1) << 31)) return false;
    DmaParams& p = pl.p;
    p.n = n; p.cin = cin; p.h = h; p.w = w; p.cout = cout; p.hw = h * w;
    p.trows = kTilePxD / w;
    p.tpi = (int32_t)ceil_div(h, p.trows);
    p.nchunks = cin / kCK;
    const int64_t tiles_cb = (int64_t)n * p.tpi;
    if (tiles_cb >= (int64_t(1) << 30)) return false;
    p.tiles_cb = (int32_t)tiles_cb;
    const int32_t cbs = cout / kCoTile;
    // rows h0−1 .. h0+trows, rounded out to 8-pixel pieces (exact when
    // rows are whole pieces; otherwise up to 4 pixels more at each end)
    const int32_t fpx = (p.trows + 2) * w + (w % 8 == 0 ? 0 : 8);
    p.fbytes = 2 * fpx;
    int32_t pb = p.fbytes;
    while (pb % 64 != 32) pb += 16;
    p.pb = pb;
    p.blk = 8 * pb + 128;
    p.in_bytes = 4 * p.blk;
    p.in_instr = (p.in_bytes + 1023) / 1024;
    if (p.in_instr > kDWaves * kMaxIn) return false;
    p.w_bytes = p.nchunks * kWSlice;
    pl.lds = (size_t)p.w_bytes + 2 * (size_t)p.in_bytes;
    if (pl.lds > (size_t)kMaxLds) return false;
    // one workgroup per CU; each output block gets an equal share
    p.gpc = (int32_t)std::max<int64_t>(1, std::min<int64_t>(tiles_cb, num_cu / std::max(1, cbs)));
    pl.grid = (int64_t)cbs * p.gpc;
    return true;
}

// ---------------------------------------------------------------------------
// Weight gradient, bf16: dw[k, c, r, s] = Σ_{n,h,w} dy[n,k,h,w] · x[n, c, h−1+r, w−1+s]
// (reference conv.hpp:177, ATen convolution_backward weight grad).
//
// GEMM with M = 64 dy channels k, N = 64 x channels c × 9 taps and the
// reduction over pixels, which lie contiguously in both NCHW operands, so
// fragments are plain 16-byte reads of 8 consecutive pixels.  A band is 224
// pixels of whole image rows (W divides 224, W a multiple of 8): dy rows
// h0 .. h0+th−1 and x rows h0−1 .. h0+th, copied untouched into LDS by
// global_load_lds_dwordx4 (each x row between a zero 16-byte guard on each
// side).  The reduction runs over the band's flattened pixels: tap (r, s)
// reads x at pixel p + r·W + s − 1 of the band's x rows; s = 1 is an aligned
// read, s = 0 and s = 2 realign it with one dword of each neighbour.  Where
// p starts (s = 0) or ends (s = 2) an image row, the shifted x element is
// the row padding and is set to zero, so a dy value meets exactly the zero
// that the reference's padded input puts there.  No pixel slot is spent on
// padding.
//
// 8 waves: wave w owns x channels 16·(w % 4).. +15 and dy channels
// 32·(w / 4).. +31 for all 9 taps (18 accumulator tiles of
// v_mfma_f32_16x16x32_bf16, M = k, N = c, K = 32 pixels).  Bands go through a
// 2-slot LDS ring; the next band's DMA is issued between the current one's
// k-steps.  One workgroup per CU: the pixel range is split into `splits`
// contiguous band ranges per (k, c) tile, and partial sums go to
// ws[split][k][c][tap] (dw's own layout) for the ordered reduce.
constexpr int kWdWaves = 8;
constexpr int kWdThreads = 64 * kWdWaves;
constexpr int kWdPix = 224;                 // pixels per band: 7 k-steps of 32
constexpr int kWdSteps = kWdPix / 32;
constexpr int kWdMaxI = 10;                 // DMA instructions per wave per band (at most)

struct WdParams {
    int32_t n, c, k, h, w, hw;
    int32_t th, bpi, bands;       // image rows per band, bands per image, n·bpi
    int32_t kblocks, cblocks, tiles, splits;
    int32_t xcd_map;              // grid grouped by XCD (see tile_split)
    int32_t pa, pbx;              // LDS bytes per dy row and per x row (both 16·odd)
    int32_t a_bytes, slot_bytes;  // 64·pa, 64·(pa + pbx)
    int32_t a_instr, instr;       // DMA instructions per band: dy, all
    int32_t xdata;                // 16-byte x data pieces per row: (th + 2)·w / 8
};

__device__ __forceinline__ u32x4 wd_shift_s0(uint32_t prev, const u32x4& c) {   // elements p−1 .. p+6
    return u32x4{__builtin_amdgcn_alignbit(c.x, prev, 16), __builtin_amdgcn_alignbit(c.y, c.x, 16),
                 __builtin_amdgcn_alignbit(c.z, c.y, 16), __builtin_amdgcn_alignbit(c.w, c.z, 16)};
}
__device__ __forceinline__ u32x4 wd_shift_s2(const u32x4& c, uint32_t next) {   // elements p+1 .. p+8
    return u32x4{__builtin_amdgcn_alignbit(c.y, c.x, 16), __builtin_amdgcn_alignbit(c.z, c.y, 16),
                 __builtin_amdgcn_alignbit(c.w, c.z, 16), __builtin_amdgcn_alignbit(next, c.w, 16)};
}

__global__ __launch_bounds__(kWdThreads, 1) void conv3x3_wgrad_dma_kernel(const bf16_t* __restrict__ x,
                                                                           const bf16_t* __restrict__ dy,
                                                                           float* __restrict__ ws, WdParams p) {
    extern __shared__ __attribute__((aligned(1024))) char smem_raw[];
    char NOTT_LDS* smem = (char NOTT_LDS*)smem_raw;
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int cg = wid & 3, kh = wid >> 2;
    const int G = lane >> 4, jl = lane & 15;

    // Tile and split.  With the XCD map, workgroups b and b + 8 (the same
    // XCD) take different tiles of the same split, so the x rows that the
    // k tiles share come from that XCD's L2.
    int32_t tile, split;
    {
        const int32_t b = (int32_t)blockIdx.x;
        if (p.xcd_map) {
            const int32_t slot = b >> 3, xcd = b & 7;
            tile = slot % p.tiles;
            split = (slot / p.tiles) * 8 + xcd;
        } else {
            tile = b % p.tiles;
            split = b / p.tiles;
        }
    }
    const int32_t kb = tile % p.kblocks, cb = tile / p.kblocks;
    const int32_t b0 = (int32_t)(((int64_t)split * p.bands) / p.splits);
    const int32_t b1 = (int32_t)(((int64_t)(split + 1) * p.bands) / p.splits);
    const void* zero = g_dma_zero;

    // This lane's DMA pieces: instruction ii = wid + 8k moves LDS bytes
    // [1024·ii, 1024·ii + 1024) of a slot (dy rows first, then x rows).
    // rel: element offset from (row 0 of the tile's channel block, band
    // start pixel); gpx: pixel offset from the band start, or invalid.
    int32_t rel[kWdMaxI], gpx[kWdMaxI];
#pragma unroll
    for (int k = 0; k < kWdMaxI; ++k) {
        const int32_t ii = wid + kWdWaves * k;
        const int32_t s = ii * 64 + lane;
        int32_t row, px;
        bool ok;
        if (ii < p.a_instr) {
            const int32_t ppr = p.pa >> 4;
            row = s / ppr;
            const int32_t g = s - row * ppr;
            px = 8 * g;
            ok = 8 * g < p.th * p.w;
        } else {
            const int32_t ppr = p.pbx >> 4, s2 = s - p.a_instr * 64;
            row = s2 / ppr;
            const int32_t g = s2 - row * ppr;
            px = 8 * (g - 1) - p.w;
            ok = g >= 1 && g <= p.xdata && cb * 64 + row < p.c;
        }
        rel[k] = row * p.hw + px;
        gpx[k] = ok ? px : -(1 << 30);
    }
    auto issue = [&](int32_t band, int slot, int k) {
        const int32_t ii = wid + kWdWaves * k;
        if (ii >= p.instr) return;
        const int32_t img = band / p.bpi, q0 = (band - img * p.bpi) * p.th * p.w;
        const bf16_t* base = ii < p.a_instr ? dy + ((int64_t)img * p.k + kb * 64) * p.hw + q0
                                            : x + ((int64_t)img * p.c + cb * 64) * p.hw + q0;
        const int32_t px = q0 + gpx[k];
        const void* src = (px >= 0 && px < p.hw) ? (const void*)(base + rel[k]) : zero;
        dma16(src, lds_addr(smem) + (uint32_t)(slot * p.slot_bytes + ii * 1024));
    };

    // Row-edge masks of this lane's 8-pixel groups, the same for every band
    // (a band starts at a row start): bit t of rs / re says the group of
    // k-step t starts / ends an image row.
    uint32_t rs = 0, re = 0;
#pragma unroll
    for (int t = 0; t < kWdSteps; ++t) {
        const int32_t q = 32 * t + 8 * G;
        if (q % p.w == 0) rs |= 1u << t;
        if ((q + 8) % p.w == 0) re |= 1u << t;
    }

    f32x4 acc[2][9];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 9; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    struct Ops {
        u32x4 a[2], cur[3];
        uint32_t prev[3], next[3];
    };
    const int32_t nb = b1 - b0;
    if (nb > 0) {
#pragma unroll
        for (int k = 0; k < kWdMaxI; ++k) issue(b0, 0, k);
    }
    for (int32_t i = 0; i < nb; ++i) {
        wait_vm_lgkm0<0>();
        barrier();
        const bool more = i + 1 < nb;
        const char NOTT_LDS* sa = smem + (i & 1) * p.slot_bytes + (kh * 32 + jl) * p.pa + 16 * G;
        const char NOTT_LDS* sx = smem + (i & 1) * p.slot_bytes + p.a_bytes + (cg * 16 + jl) * p.pbx + 16 + 16 * G;
        auto load_ops = [&](int t, Ops& o) {
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) o.a[mt] = *(const u32x4 NOTT_LDS*)(sa + mt * 16 * p.pa + 64 * t);
#pragma unroll
            for (int r = 0; r < 3; ++r) {
                const char NOTT_LDS* q = sx + 64 * t + 2 * r * p.w;
                o.cur[r] = *(const u32x4 NOTT_LDS*)q;
                o.prev[r] = *(const uint32_t NOTT_LDS*)(q - 4);
                o.next[r] = *(const uint32_t NOTT_LDS*)(q + 16);
            }
        };
        Ops ops[2];
        load_ops(0, ops[0]);
#pragma unroll
        for (int t = 0; t < kWdSteps; ++t) {
            Ops& o = ops[t & 1];
            if (t + 1 < kWdSteps) load_ops(t + 1, ops[(t + 1) & 1]);
            // the next band's DMA: instructions t and t + 7
            if (more) {
                issue(b0 + i + 1, (i + 1) & 1, t);
                if (t + kWdSteps < kWdMaxI) issue(b0 + i + 1, (i + 1) & 1, t + kWdSteps);
            }
            __builtin_amdgcn_sched_barrier(0);
            const uint32_t m0 = (rs >> t) & 1 ? 0xffff0000u : 0xffffffffu;
            const uint32_t m7 = (re >> t) & 1 ? 0x0000ffffu : 0xffffffffu;
#pragma unroll
            for (int r = 0; r < 3; ++r) {
                u32x4 bs0 = wd_shift_s0(o.prev[r], o.cur[r]);
                u32x4 bs2 = wd_shift_s2(o.cur[r], o.next[r]);
                bs0.x &= m0;
                bs2.w &= m7;
#pragma unroll
                for (int mt = 0; mt < 2; ++mt) {
                    const bf16x8 av = __builtin_bit_cast(bf16x8, o.a[mt]);
                    acc[mt][3 * r + 0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, __builtin_bit_cast(bf16x8, bs0),
                                                                                 acc[mt][3 * r + 0], 0, 0, 0);
                    acc[mt][3 * r + 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        av, __builtin_bit_cast(bf16x8, o.cur[r]), acc[mt][3 * r + 1], 0, 0, 0);
                    acc[mt][3 * r + 2] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, __builtin_bit_cast(bf16x8, bs2),
                                                                                 acc[mt][3 * r + 2], 0, 0, 0);
                }
            }
        }
    }

    // Partials in dw's layout, ws[split][k][c][tap].  For each (mt, e) a wave
    // holds 4 k rows (one per 16-lane group) × its 16 channels × 9 taps, i.e.
    // 4 runs of 144 consecutive floats; they pass through the wave's own LDS
    // slice so the global stores are whole 16-byte pieces.
    const int32_t c0 = cb * 64 + cg * 16;
    float* wsp = ws + (int64_t)split * 9 * p.k * p.c;
    float NOTT_LDS* slice = (float NOTT_LDS*)smem + wid * (4 * 16 * 9);
    wait_vm_lgkm0<0>();
    barrier();                                    // every wave is done with the band operands
    const int32_t cw = min(16, p.c - c0);         // channels of this wave inside c
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
#pragma unroll
            for (int tap = 0; tap < 9; ++tap) slice[(G * 16 + jl) * 9 + tap] = acc[mt][tap][e];
            // the slice is this wave's own: wave-scope ordering suffices
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            __builtin_amdgcn_wave_barrier();
            for (int q = lane; q < 4 * 36; q += 64) {
                const int g = q / 36, j = q - g * 36;
                const int32_t kk = kb * 64 + kh * 32 + mt * 16 + g * 4 + e;
                if (4 * j < cw * 9)
                    *reinterpret_cast<f32x4*>(wsp + ((int64_t)kk * p.c + c0) * 9 + 4 * j) =
                        *(const f32x4 NOTT_LDS*)(slice + g * 144 + 4 * j);
            }
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            __builtin_amdgcn_wave_barrier();
        }
}

bool wd_plan(int32_t n, int32_t c, int32_t h, int32_t w, int32_t k, int num_cu, WdParams& p, size_t& lds) {
    if (w <= 0 || w % 8 != 0 || kWdPix % w != 0 || k % 64 != 0 || c % 16 != 0 || n <= 0 || h <= 0) return false;
    if ((int64_t)n * std::max(c, k) * h * w >= (int64_t(1) << 31)) return false;
    p.n = n; p.c = c; p.k = k; p.h = h; p.w = w; p.hw = h * w;
    p.th = kWdPix / w;
    p.bpi = (int32_t)ceil_div(h, p.th);
    p.bands = n * p.bpi;
    p.kblocks = k / 64;
    p.cblocks = (int32_t)ceil_div(c, 64);
    p.tiles = p.kblocks * p.cblocks;
    // pitches that are 16·odd bytes: 16 lanes reading 16 rows at one column
    // touch 16 distinct 16-byte slots
    auto odd16 = [](int32_t b) {
        b = (b + 15) & ~15;
        return ((b >> 4) & 1) ? b : b + 16;
    };
    p.pa = odd16(p.th * w * 2);
    p.pbx = odd16((p.th + 2) * w * 2 + 32);
    p.xdata = (p.th + 2) * w / 8;
    p.a_bytes = 64 * p.pa;
    p.slot_bytes = 64 * (p.pa + p.pbx);
    p.a_instr = p.pa / 16;
    p.instr = (p.pa + p.pbx) / 16;
    if (p.instr > kWdWaves * kWdMaxI) return false;
    lds = std::max<size_t>(2 * (size_t)p.slot_bytes, (size_t)kWdWaves * 4 * 16 * 9 * sizeof(float));
    if (lds > (size_t)kMaxLds) return false;
    // one workgroup per CU
    if (num_cu >= 8 * p.tiles) {
        p.xcd_map = 1;
        p.splits = 8 * (num_cu / (8 * p.tiles));
    } else {
        p.xcd_map = 0;
        p.splits = std::max(1, num_cu / p.tiles);
    }
    p.splits = std::min(p.splits, p.bands);
    if (p.xcd_map && p.splits % 8 != 0) p.xcd_map = 0;
    return true;
}

}  // namespace

bool dma_applies(int32_t n, int32_t cin, int32_t h, int32_t w, int32_t cout) {
    DmaPlan pl;
    return dma_plan(n, cin, h, w, cout, 256, pl);
}

int64_t dma_prep_elems(int32_t cin, int32_t cout) { return (int64_t)cout * cin * 9; }

template <bool DGRAD>
int dma_prep(nott_ctx ctx, const bf16_t* w, bf16_t* wp, int32_t cin, int32_t cout) {
    const int64_t elems = (int64_t)cout * cin * 9;
    hipLaunchKernelGGL(dma_wprep_kernel<DGRAD>, dim3((unsigned)ceil_div(elems, 256)), dim3(256), 0, ctx->stream, w,
                       wp, cin, cout);
    return launch_status(ctx, "conv3x3_dma_wprep");
}

int dma_prep_pair(nott_ctx ctx, const bf16_t* w, bf16_t* wf, bf16_t* wd, int32_t cin, int32_t cout) {
    const int64_t elems = (int64_t)cout * cin * 9;
    hipLaunchKernelGGL(dma_wprep_pair_kernel, dim3((unsigned)ceil_div(elems, 256)), dim3(256), 0, ctx->stream, w, wf,
                       wd, cin, cout);
    return launch_status(ctx, "conv3x3_dma_wprep_pair");
}

int dma_run(nott_ctx ctx, int32_t n, int32_t cin, int32_t h, int32_t w, int32_t cout, const bf16_t* in,
            const bf16_t* wp, const float* bias, bf16_t* out, int relu) {
    DmaPlan pl;
    if (!dma_plan(n, cin, h, w, cout, ctx->num_cu, pl))
        return fail(ctx, NOTT_ERR_UNSUPPORTED, "conv3x3_dma: shape not supported");
    if (((uintptr_t)in & 15) != 0 || ((uintptr_t)out & 7) != 0 || ((uintptr_t)wp & 15) != 0)
        return fail(ctx, NOTT_ERR_UNSUPPORTED, "conv3x3_dma: operands must be 16-byte (input, weights) / 8-byte (output) aligned");
    static bool attr_set = false;
    if (!attr_set) {
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&conv3x3_dma_kernel<false>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLds);
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&conv3x3_dma_kernel<true>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLds);
        attr_set = true;
    }
    if (relu)
        hipLaunchKernelGGL(conv3x3_dma_kernel<true>, dim3((unsigned)pl.grid), dim3(kDThreads), pl.lds, ctx->stream, in,
                           wp, bias, out, pl.p);
    else
        hipLaunchKernelGGL(conv3x3_dma_kernel<false>, dim3((unsigned)pl.grid), dim3(kDThreads), pl.lds, ctx->stream,
                           in, wp, bias, out, pl.p);
    return launch_status(ctx, "conv3x3_dma");
}

bool wdma_applies(int32_t n, int32_t c, int32_t h, int32_t w, int32_t k) {
    WdParams p;
    size_t lds;
    return wd_plan(n, c, h, w, k, 256, p, lds);
}

int wdma_partials(nott_ctx ctx, int32_t n, int32_t c, int32_t h, int32_t w, int32_t k, const bf16_t* x,
                  const bf16_t* dy, float** ws_out, int32_t* splits_out) {
    WdParams p;
    size_t lds;
    if (!wd_plan(n, c, h, w, k, ctx->num_cu, p, lds))
        return fail(ctx, NOTT_ERR_UNSUPPORTED, "conv3x3 wgrad (dma): shape not supported");
    if (((uintptr_t)x & 15) != 0 || ((uintptr_t)dy & 15) != 0)
        return fail(ctx, NOTT_ERR_UNSUPPORTED, "conv3x3 wgrad (dma): operands must be 16-byte aligned");
    float* ws = static_cast<float*>(workspace(ctx, sizeof(float) * (size_t)p.splits * 9 * k * c));
    if (!ws) return NOTT_ERR_ALLOC;
    static bool attr_set = false;
    if (!attr_set) {
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&conv3x3_wgrad_dma_kernel),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLds);
        attr_set = true;
    }
    hipLaunchKernelGGL(conv3x3_wgrad_dma_kernel, dim3((unsigned)(p.tiles * p.splits)), dim3(kWdThreads), lds,
                       ctx->stream, x, dy, ws, p);
    *ws_out = ws;
    *splits_out = p.splits;
    return launch_status(ctx, "conv3x3_wgrad_dma");
}

template int dma_prep<false>(nott_ctx, const bf16_t*, bf16_t*, int32_t, int32_t);
template int dma_prep<true>(nott_ctx, const bf16_t*, bf16_t*, int32_t, int32_t);

}  // namespace conv_fast
}  // namespace nott
