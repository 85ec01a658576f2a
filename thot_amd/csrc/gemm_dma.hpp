// bf16 MFMA GEMM with direct-to-LDS operand fills (gfx950).
//
//   C[M×N] = Σ_k A(m, k)·B(n, k),  fp32 accumulate, bf16 operands:
//   A(m, k) = A[m·lda + k]  (AT = false)   or   A[k·lda + m]  (AT = true)
//   B(n, k) = B[n·ldb + k]  (BT = false)   or   B[k·ldb + n]  (BT = true)
//
// Work decomposition.  A workgroup owns a BM×BN output tile and walks K in
// 64-deep stages; its WM×WN waves each own a (BM/WM)×(BN/WN) sub-tile made
// of 32×32 v_mfma_f32_32x32x16_bf16 blocks (one 32×32×16 product per issue).
//
// Fills.  Operands go from global memory straight into LDS with
// global_load_lds_dwordx4: one instruction moves 1 KB (16 bytes per lane,
// lane i to byte 16·i of a wave-uniform LDS base), so no VGPRs, no VALU
// repacking and no ds_write are spent on staging.  The lane→global mapping
// is chosen so that the 1 KB blocks land in a swizzled layout:
//   k-contiguous operand (AT/BT false), tile [row][k] (128 bytes per row):
//     16-byte chunk c (k = 8c..8c+7) of row r at r·128 + ((c ^ ((r>>1)&7))·16);
//     a 32×32×16 operand read (rows r0..r0+31, chunk 2s + lane/32) hits 16
//     distinct 16-byte slots in every quarter-wave.
//   row-contiguous operand (AT/BT true), tile [k][row] (2·R bytes per k):
//     chunk cr (rows 8cr..8cr+7) of k-row k at k·2R + ((cr ^ 4·(k&3))·16);
//     operands are read with ds_read_b64_tr_b16, which hands lane i of each
//     16-lane group the 4 k-consecutive values of row i from a [k][row]
//     block, i.e. the MFMA operand layout, so no transpose is ever stored.
// Stages form an S-deep ring: the loads of stage t+S are issued right after
// the barrier that follows every wave's last read of stage t, so S-1 stages
// are in flight while one is multiplied.  Only s_waitcnt vmcnt (how many of
// this wave's loads may still be outstanding) and s_barrier order the ring;
// the compiler's workgroup fence (which would wait for every load) is not
// used, and the DMA is issued as inline assembly (see dma16).  Within a
// stage the four 16-deep slices are software-pipelined: the fragments of
// slice s+1 are read while slice s is multiplied.
//
// Tile order.  Workgroups are dispatched round-robin over the 8 XCDs (each
// with its own L2); the linear tile index is remapped so that each XCD gets
// a contiguous band of tiles (grouped `gm` tile-rows at a time) and its L2
// holds the A rows and B columns that band shares.
#pragma once

#include "gemm.hpp"
#include "lds_dma.hpp"

namespace nott {
namespace gemm {
namespace dma {

constexpr int BK = 64;

using lds::barrier;
using lds::dma16;
using lds::lds_addr;
using lds::wait_vm_lgkm0;

// Issues this wave's share of one operand tile (R rows × 64 k) of stage k0.
// Rows past `rows` are clamped to the last row (their results are never
// stored); row-contiguous operands need rows % 8 == 0 and rows >= 8.
template <bool TR, int R, int NW>
__device__ __forceinline__ void fill(const bf16_t* __restrict__ p, int64_t ld, int64_t row0, int64_t rows, int64_t k0,
                                     char NOTT_LDS* dst, int wid, int lane) {
    constexpr int NB = R / 8;   // 1 KB blocks per tile
    static_assert(NB % NW == 0, "tile blocks must split evenly over the waves");
#pragma unroll
    for (int qq = 0; qq < NB / NW; ++qq) {
        const int q = qq * NW + wid;
        const bf16_t* src;
        if constexpr (!TR) {
            const int r = 8 * q + (lane >> 3);
            const int c = (lane & 7) ^ ((r >> 1) & 7);
            int64_t gr = row0 + r;
            gr = gr < rows ? gr : rows - 1;
            src = p + gr * ld + k0 + 8 * c;
        } else {
            static_assert(R >= 128, "row-contiguous tiles need at least 128 rows");
            constexpr int KPB = 1024 / (2 * R);   // k-rows per block
            const int b = 16 * lane;
            const int k = q * KPB + b / (2 * R);
            const int cr = ((b % (2 * R)) >> 4) ^ ((k & 3) << 2);
            int64_t gc = row0 + 8 * cr;
            gc = gc <= rows - 8 ? gc : rows - 8;
            src = p + (k0 + k) * ld + gc;
        }
        dma16(src, lds_addr(dst) + 1024 * q);
    }
}

// A 32×16 MFMA operand (lane l: row l % 32, k = 8·(l/32) + 0..7): one
// 16-byte read from a [row][k] tile, or two transposing 8-byte reads from a
// [k][row] tile.
typedef short v4i16 __attribute__((ext_vector_type(4)));
template <bool TR> struct Frag;
template <> struct Frag<false> {
    u32x4 v;
    __device__ __forceinline__ bf16x8 get() const { return __builtin_bit_cast(bf16x8, v); }
    __device__ __forceinline__ void ld(const char NOTT_LDS* p) { v = *reinterpret_cast<const u32x4 NOTT_LDS*>(p); }
};
template <> struct Frag<true> {
    v4i16 lo, hi;
    __device__ __forceinline__ bf16x8 get() const {
        const v4i16 w[2] = {lo, hi};
        return __builtin_bit_cast(bf16x8, w);
    }
    __device__ __forceinline__ void ld(const char NOTT_LDS* p, int hi_off) {
        lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((v4i16 NOTT_LDS*)p);
        hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((v4i16 NOTT_LDS*)(p + hi_off));
    }
};

// Per-lane LDS byte offsets of one operand's fragments inside a stage tile
// (R rows; this wave's rows start at w0; F fragments of 32 rows).
//   [row][k] tile: fragment f, slice s at off[s] + 4096·f, where
//     off[s] = (w0 + l%32)·128 + ((2s + l/32) ^ ((l>>1)&7))·16
//     (w0 + 32f is a multiple of 16, so the swizzle depends on l only).
//   [k][row] tile: fragment f, slice s, half h at off[f] + (16s + 4h)·2R, where
//     off[f] = k·2R + (((r>>3) ^ 4·(k&3))·16) + (r&7)·2 with
//     r = w0 + 32f + 16·((l>>4)&1) + 4·(l&3), k = 8·(l/32) + ((l&15)>>2).
template <bool TR, int R, int F>
struct FragAddr {
    uint32_t off[TR ? F : 4];
    __device__ __forceinline__ void init(int w0, int lane) {
        if constexpr (!TR) {
#pragma unroll
            for (int s = 0; s < 4; ++s)
                off[s] = (uint32_t)((w0 + (lane & 31)) * 128 + ((((2 * s) | (lane >> 5)) ^ ((lane >> 1) & 7)) << 4));
        } else {
            const int k = 8 * (lane >> 5) + ((lane & 15) >> 2);
#pragma unroll
            for (int f = 0; f < F; ++f) {
                const int r = w0 + 32 * f + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
                off[f] = (uint32_t)(k * (2 * R) + (((r >> 3) ^ ((k & 3) << 2)) << 4) + (r & 7) * 2);
            }
        }
    }
    // Reads fragment FI of slice S of the tile at `base`.
    template <int S, int FI>
    __device__ __forceinline__ void read(Frag<TR>& d, const char NOTT_LDS* base) const {
        if constexpr (!TR) d.ld(base + off[S] + 4096 * FI);
        else d.ld(base + off[FI] + 16 * S * 2 * R, 4 * 2 * R);
    }
};

template <int S, bool TR, int R, int F, int I = 0>
__device__ __forceinline__ void read_all(Frag<TR> (&d)[F], const FragAddr<TR, R, F>& a, const char NOTT_LDS* base) {
    if constexpr (I < F) {
        a.template read<S, I>(d[I], base);
        read_all<S, TR, R, F, I + 1>(d, a, base);
    }
}

// Maps the linear tile index to (tile row, tile column): XCD-contiguous bands
// (when the tile count is a multiple of 8), grouped `gm` tile-rows at a time.
__device__ __forceinline__ void tile_of(int id, int tm, int tn, int gm, int& pm, int& pn) {
    const int nt = tm * tn;
    if ((nt & 7) == 0) id = (id & 7) * (nt >> 3) + (id >> 3);
    const int per_group = gm * tn;
    const int g = id / per_group;
    const int first = g * gm;
    const int gsz = min(tm - first, gm);
    const int in = id - g * per_group;
    pm = first + in % gsz;
    pn = in / gsz;
}

// Sum of the 8 bf16 values of an operand fragment, in k order.
__device__ __forceinline__ void add_bf16x2(float& s, uint32_t w) {
    s += __builtin_bit_cast(float, w << 16);
    s += __builtin_bit_cast(float, w & 0xffff0000u);
}
__device__ __forceinline__ void add_frag(float& s, const Frag<false>& f) {
    add_bf16x2(s, f.v.x);
    add_bf16x2(s, f.v.y);
    add_bf16x2(s, f.v.z);
    add_bf16x2(s, f.v.w);
}
__device__ __forceinline__ void add_frag(float& s, const Frag<true>& f) {
    const u32x4 w = __builtin_bit_cast(u32x4, f.get());
    add_bf16x2(s, w.x);
    add_bf16x2(s, w.y);
    add_bf16x2(s, w.z);
    add_bf16x2(s, w.w);
}

// grid: x = tiles (tm·tn), z = k splits of kps (a multiple of BK) each.
// ROWSUM: also Σ_k A(m, k) for every row m of the tile (the bias gradient
// when A is the output gradient of a Linear), summed in fp32 from the A
// fragments already in registers: only the tiles of tile column 0 sum, and
// there fragment f's sum is kept by wave column f % WN, so each row is
// summed once; the two k-halves of a row are held by lanes l and l+32 and
// combined at the end; the epilogue receives it via ep.rowsum(m, v).
template <bool AT, bool BT, int BM, int BN, int WM, int WN, int S, bool ROWSUM, class EP>
__global__ __launch_bounds__(64 * WM * WN) void gemm_kernel(const bf16_t* __restrict__ A, int64_t lda,
                                                             const bf16_t* __restrict__ B, int64_t ldb, EP ep,
                                                             int64_t M, int64_t N, int64_t K, int64_t kps, int gm) {
    constexpr int NW = WM * WN;
    constexpr int TM = BM / WM, TN = BN / WN;
    constexpr int FM = TM / 32, FN = TN / 32;
    constexpr int A_BYTES = BM * 128, B_BYTES = BN * 128, STAGE = A_BYTES + B_BYTES;
    constexpr int LOADS = (BM / 8 + BN / 8) / NW;   // global_load_lds per wave per stage
    static_assert(TM % 32 == 0 && TN % 32 == 0, "wave tiles are whole 32x32 blocks");
    static_assert(S >= 2 && (S - 2) * LOADS < 64, "ring depth");
    extern __shared__ __attribute__((aligned(1024))) char smem_raw[];
    char NOTT_LDS* smem = (char NOTT_LDS*)smem_raw;

    const int tm = (int)((M + BM - 1) / BM), tn = (int)((N + BN - 1) / BN);
    int pm, pn;
    tile_of((int)blockIdx.x, tm, tn, gm, pm, pn);
    const int64_t m0 = (int64_t)pm * BM, n0 = (int64_t)pn * BN;
    const int64_t kb = (int64_t)blockIdx.z * kps;
    const int64_t ke = kb + kps < K ? kb + kps : K;
    const int nk = ke > kb ? (int)((ke - kb) / BK) : 0;
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int wm = wid / WN, wn = wid % WN;

    f32x16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

    auto issue = [&](int t, int slot) {
        char NOTT_LDS* st = smem + slot * STAGE;
        const int64_t k0 = kb + (int64_t)t * BK;
        fill<AT, BM, NW>(A, lda, m0, M, k0, st, wid, lane);
        fill<BT, BN, NW>(B, ldb, n0, N, k0, st + A_BYTES, wid, lane);
    };
    FragAddr<AT, BM, FM> fa;
    FragAddr<BT, BN, FN> fb;
    fa.init(wm * TM, lane);
    fb.init(wn * TN, lane);

    Frag<AT> a[2][FM];
    Frag<BT> b[2][FN];
    float rs[FM];
#pragma unroll
    for (int i = 0; i < FM; ++i) rs[i] = 0.f;
    auto mma = [&](int p) {
        if constexpr (ROWSUM) {
            if (pn == 0) {
#pragma unroll
                for (int i = 0; i < FM; ++i)
                    if (i % WN == wn) add_frag(rs[i], a[p][i]);
            }
        }
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[p][i].get(), b[p][j].get(), acc[i][j], 0, 0, 0);
    };

    // Stages 0..S-2 are in flight before the loop.  The loads of stage t+S
    // go into slot t % S once every wave has passed the barrier that follows
    // its last read of stage t.
#pragma unroll
    for (int s = 0; s < S - 1; ++s)
        if (s < nk) issue(s, s);
    if (nk > 0) {
        if (nk >= S - 1) wait_vm_lgkm0<(S - 2) * LOADS>();
        else wait_vm_lgkm0<0>();
        barrier();
        if (S - 1 < nk) issue(S - 1, S - 1);
        read_all<0>(a[0], fa, smem);
        read_all<0>(b[0], fb, smem + A_BYTES);
    }
    int slot = 0;   // ring slot of stage t
    for (int t = 0; t < nk; ++t) {
        const char NOTT_LDS* sa = smem + slot * STAGE;
        const char NOTT_LDS* sb = sa + A_BYTES;
        read_all<1>(a[1], fa, sa);
        read_all<1>(b[1], fb, sb);
        mma(0);
        read_all<2>(a[0], fa, sa);
        read_all<2>(b[0], fb, sb);
        mma(1);
        read_all<3>(a[1], fa, sa);
        read_all<3>(b[1], fb, sb);
        mma(0);
        const int nslot = slot + 1 == S ? 0 : slot + 1;
        if (t + 1 < nk) {
            // Stage t+1 must have landed; stages t+2 .. t+S-1 may be in flight.
            if (t + S - 1 < nk) wait_vm_lgkm0<(S - 2) * LOADS>();
            else wait_vm_lgkm0<0>();
            barrier();
            if (t + S < nk) issue(t + S, slot);
            const char NOTT_LDS* na = smem + nslot * STAGE;
            read_all<0>(a[0], fa, na);
            read_all<0>(b[0], fb, na + A_BYTES);
        }
        mma(1);
        slot = nslot;
    }
    if constexpr (ROWSUM) {
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            if (pn != 0 || i % WN != wn) continue;
            const float v = rs[i] + __shfl_xor(rs[i], 32);
            if (lane < 32) ep.rowsum(m0 + wm * TM + 32 * i + lane, v);
        }
    }
    // Accumulator layout of a 32×32 block: lane l holds column l % 32 and,
    // in register 4q + e, row 8q + 4·(l/32) + e.
    const int col = lane & 31, rh = (lane >> 5) * 4;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    ep.store(m0 + wm * TM + 32 * i + 8 * q + rh + e, n0 + wn * TN + 32 * j + col, acc[i][j][4 * q + e]);
}

template <bool AT, bool BT, int BM, int BN, int WM, int WN, int S>
struct Config {
    static constexpr bool kAT = AT, kBT = BT;
    static constexpr int kBM = BM, kBN = BN, kWM = WM, kWN = WN, kS = S;
    static constexpr int kThreads = 64 * WM * WN;
    static constexpr size_t kLds = (size_t)S * (BM + BN) * 128;
};

// Tile shapes the dispatcher picks from (measured on the configs[3]
// projection shapes and on large square products): 256×256 with 8 waves of
// 128×64 and a 2-deep ring for long-K products, unsplit when they fill the
// chip and split over K when they have few tiles; 256×128 with 8 waves of
// 64×64 and a 3-deep ring for other grids that fill the chip on their own;
// 128×128 with 4 waves and a 3-deep ring for the rest.
enum class Shape { T256x128, T256x256, T128x128 };

struct Plan {
    Shape shape;
    int64_t splits, kps;
};

inline Plan plan(nott_ctx ctx, int64_t M, int64_t N, int64_t K, int64_t splits) {
    const int64_t cu = ctx->num_cu;
    const int64_t nkb = K / BK;
    auto tiles = [&](int bm, int bn) { return ceil_div(M, bm) * ceil_div(N, bn); };
    Plan p{Shape::T128x128, 1, K};
    int64_t want = 1, min_stages = 4;
    // Split counts keep the grid within one round of workgroups (one per CU:
    // the 256x256 and 128x128 shapes hold 128 and 96 KB of LDS), so that a
    // few leftover splits do not cost a second round.
    if (tiles(256, 256) >= cu && nkb >= 32) {
        // long-K products that fill the chip with the larger tile: 8192^3
        // 890 -> 974 TFLOP/s, 16384x4096x4096 938 -> 1070 (at K = 1024 the
        // 256x128 tile's 3-deep ring wins)
        p.shape = Shape::T256x256;
    } else if (tiles(256, 128) >= cu) {
        p.shape = Shape::T256x128;
    } else if (tiles(256, 256) >= cu / 8 && nkb >= 16) {
        p.shape = Shape::T256x256;
        want = std::max<int64_t>(1, cu / tiles(256, 256));
        min_stages = 8;
    } else {
        want = std::max<int64_t>(1, cu / tiles(128, 128));
    }
    if (splits <= 0) splits = std::min<int64_t>(want, std::max<int64_t>(1, nkb / min_stages));
    splits = std::max<int64_t>(1, std::min<int64_t>(splits, std::min<int64_t>(nkb, 65535)));
    p.kps = ceil_div(nkb, splits) * BK;
    p.splits = ceil_div(K, p.kps);
    return p;
}

// Whether the operands qualify: K a multiple of 64, 16-byte aligned bases
// and leading dimensions, row-contiguous operands in whole 8-row groups, and
// at least 128 rows and columns (narrower products waste most of a tile).
template <bool AT, bool BT>
inline bool applies(const bf16_t* A, int64_t lda, const bf16_t* B, int64_t ldb, int64_t M, int64_t N, int64_t K) {
    auto ok16 = [](const void* p, int64_t ld) { return ((uintptr_t)p % 16) == 0 && (ld % 8) == 0; };
    if (K <= 0 || K % BK != 0 || !ok16(A, lda) || !ok16(B, ldb)) return false;
    if (M < 128 || N < 128) return false;
    if ((AT && M % 8 != 0) || (BT && N % 8 != 0)) return false;
    return ceil_div(M, 128) * ceil_div(N, 128) < (int64_t)1 << 31;
}

// fp32 scratch the split-K partials of an M×N×K product need (0 if unsplit).
inline size_t partial_floats(nott_ctx ctx, int64_t M, int64_t N, int64_t K) {
    const Plan p = plan(ctx, M, N, K, 0);
    return p.splits > 1 ? (size_t)(p.splits * M * N) : 0;
}

template <class Cfg, bool ROWSUM, class EP>
int launch(nott_ctx ctx, const bf16_t* A, int64_t lda, const bf16_t* B, int64_t ldb, const EP& ep, int64_t M,
           int64_t N, int64_t K, int64_t splits, int64_t kps) {
    auto fn = gemm_kernel<Cfg::kAT, Cfg::kBT, Cfg::kBM, Cfg::kBN, Cfg::kWM, Cfg::kWN, Cfg::kS, ROWSUM, EP>;
    static bool attr = false;   // one setting per kernel instantiation
    if (!attr) {
        if (hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)Cfg::kLds) != hipSuccess)
            return fail(ctx, NOTT_ERR_HIP, "gemm_dma: cannot reserve LDS");
        attr = true;
    }
    const int64_t tiles = ceil_div(M, Cfg::kBM) * ceil_div(N, Cfg::kBN);
    hipLaunchKernelGGL(fn, dim3((unsigned)tiles, 1, (unsigned)splits), dim3(Cfg::kThreads), Cfg::kLds, ctx->stream, A,
                       lda, B, ldb, ep, M, N, K, kps, 4);
    return launch_status(ctx, "gemm_dma");
}

template <bool AT, bool BT, bool ROWSUM, class EP>
int launch_shape(nott_ctx ctx, Shape sh, const bf16_t* A, int64_t lda, const bf16_t* B, int64_t ldb, const EP& ep,
                 int64_t M, int64_t N, int64_t K, int64_t splits, int64_t kps) {
    switch (sh) {
        case Shape::T256x128:
            return launch<Config<AT, BT, 256, 128, 4, 2, 3>, ROWSUM>(ctx, A, lda, B, ldb, ep, M, N, K, splits, kps);
        case Shape::T256x256:
            return launch<Config<AT, BT, 256, 256, 2, 4, 2>, ROWSUM>(ctx, A, lda, B, ldb, ep, M, N, K, splits, kps);
        default:
            return launch<Config<AT, BT, 128, 128, 2, 2, 3>, ROWSUM>(ctx, A, lda, B, ldb, ep, M, N, K, splits, kps);
    }
}

// Split-K partial store with per-split row sums: ws[split][m][n] and
// rows[split][m].
struct PartialRowStore {
    float* ws;
    float* rows;
    int64_t M, N;
    __device__ __forceinline__ void store(int64_t m, int64_t n, float v) const {
        if (m < M && n < N) ws[((int64_t)blockIdx.z * M + m) * N + n] = v;
    }
    __device__ __forceinline__ void rowsum(int64_t m, float v) const {
        if (m < M) rows[(int64_t)blockIdx.z * M + m] = v;
    }
};


// C = A·B, or NOTT_ERR_UNSUPPORTED when the operands do not qualify (the
// caller then uses another engine).  Split-K partials go to `partial` when
// given (partial_floats() of them), else to the workspace, and are summed in
// split order by the reduce kernel, which applies the epilogue.  ROWSUM also
// hands ep.rowsum(m, Σ_k A(m, k)) for every row (see gemm_kernel).
template <bool AT, bool BT, bool ROWSUM = false, class EP>
int run(nott_ctx ctx, const bf16_t* A, int64_t lda, const bf16_t* B, int64_t ldb, const EP& ep, int64_t M, int64_t N,
        int64_t K, int64_t splits = 0, float* partial = nullptr) {
    if (M <= 0 || N <= 0) return NOTT_OK;
    if (!applies<AT, BT>(A, lda, B, ldb, M, N, K)) return NOTT_ERR_UNSUPPORTED;
    // The split reduce that also sums rows works on 4-column groups.
    if (ROWSUM && N % 4 != 0) splits = 1;
    const Plan p = plan(ctx, M, N, K, splits);
    if (p.splits == 1) return launch_shape<AT, BT, ROWSUM>(ctx, p.shape, A, lda, B, ldb, ep, M, N, K, 1, p.kps);
    const size_t body = (size_t)(p.splits * M * N), rows = ROWSUM ? (size_t)(p.splits * M) : 0;
    float* ws = partial && !ROWSUM ? partial : static_cast<float*>(workspace(ctx, sizeof(float) * (body + rows)));
    if (!ws) return NOTT_ERR_ALLOC;
    int st;
    if constexpr (ROWSUM)
        st = launch_shape<AT, BT, true>(ctx, p.shape, A, lda, B, ldb, PartialRowStore{ws, ws + body, M, N}, M, N, K,
                                        p.splits, p.kps);
    else
        st = launch_shape<AT, BT, false>(ctx, p.shape, A, lda, B, ldb, PartialStore{ws, M, N}, M, N, K, p.splits,
                                         p.kps);
    if (st != NOTT_OK) return st;
    if constexpr (ROWSUM) launch_splitk_reduce(ctx, ws, p.splits, M, N, ep, ws + body);
    else launch_splitk_reduce(ctx, ws, p.splits, M, N, ep);
    return launch_status(ctx, "gemm_dma_splitk");
}

}  // namespace dma
}  // namespace gemm
}  // namespace nott
