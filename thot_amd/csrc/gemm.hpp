// Generic MFMA GEMM engine for gfx950: C[M×N] = Σ_k A(m,k)·B(k,n), fp32
// accumulate, operands fp32 or bf16.
//
// The engine owns tiling, LDS staging, the MFMA inner loop and split-K; the
// caller supplies two loaders (how to read A(m,k) and B(k,n) from memory,
// including implicit-im2col gathers for convolutions) and an epilogue (how
// to write C(m,n)).  Specialised kernels (conv3x3.hip) handle the hot shapes;
// this engine covers every shape, stride, padding and transpose correctly.
//
// Tile: BM×BN = 128×128 per 256-thread workgroup (4 waves as 2×2, each wave
// 64×64 = 4×4 MFMA 16×16 tiles).  The k-step holds 64 bytes of k per row:
// 32 bf16 (one v_mfma_f32_16x16x32_bf16) or 16 fp32 (four
// v_mfma_f32_16x16x4f32).  LDS keeps both operands k-contiguous per row
// ([row][k], 80-byte padded rows), double-buffered with register prefetch.
//
// MFMA operand layout (16×16 output tile): lane l supplies row (l % 16) of A
// and column (l % 16) of B, each as the 16 bytes at k-byte-offset 16·(l/16).
// A and B use the same lane→k assignment, so the product is exact whatever
// order the instruction sums the 64-byte k-slice in.  Accumulator: lane l
// holds column l % 16, rows 4·(l/16) + {0,1,2,3}.
#pragma once

#include "common.hpp"

namespace nott {
namespace gemm {

constexpr int BM = 128;
constexpr int BN = 128;
constexpr int kThreads = 256;
constexpr int kRowBytes = 64;        // k extent of one LDS row
constexpr int kLdsStride = 80;       // padded LDS row pitch (bytes)
constexpr int kChunksPerRow = kRowBytes / 16;

template <typename T> struct KTraits;
template <> struct KTraits<float> {
    static constexpr int kElemsPerChunk = 4;
    static constexpr int BK = 16;
};
template <> struct KTraits<bf16_t> {
    static constexpr int kElemsPerChunk = 8;
    static constexpr int BK = 32;
};

// Packs elements into a 16-byte chunk.
template <typename T> struct Pack;
template <> struct Pack<float> {
    static __device__ __forceinline__ u32x4 make(const float (&v)[4]) {
        u32x4 r;
        r.x = __builtin_bit_cast(uint32_t, v[0]);
        r.y = __builtin_bit_cast(uint32_t, v[1]);
        r.z = __builtin_bit_cast(uint32_t, v[2]);
        r.w = __builtin_bit_cast(uint32_t, v[3]);
        return r;
    }
};
template <> struct Pack<bf16_t> {
    static __device__ __forceinline__ u32x4 make(const bf16_t (&v)[8]) {
        u32x4 r;
        r.x = (uint32_t)v[0] | ((uint32_t)v[1] << 16);
        r.y = (uint32_t)v[2] | ((uint32_t)v[3] << 16);
        r.z = (uint32_t)v[4] | ((uint32_t)v[5] << 16);
        r.w = (uint32_t)v[6] | ((uint32_t)v[7] << 16);
        return r;
    }
};

// Raw element access in storage type (no conversion).
template <typename T>
__device__ __forceinline__ T raw_ld(const T* p, int64_t i) { return p[i]; }

// ---------------------------------------------------------------------------
// Loaders.  A loader describes an operand as R(row, k) for row in [0, rows)
// and k in [0, K): for A, row = m; for B, row = n.  Out-of-range elements
// read as zero.  Each loader provides
//   static constexpr bool kRowFast   lane mapping: true -> consecutive lanes
//                                    take consecutive rows (k-strided memory);
//                                    false -> consecutive lanes walk k.
//   u32x4 chunk(row, k0)             the 16-byte chunk of k0 .. k0+E-1.
// ---------------------------------------------------------------------------

// Row-major, k contiguous: R(row, k) = p[row·ld + k].
template <typename T>
struct RowKLoader {
    static constexpr bool kRowFast = false;
    static constexpr int E = KTraits<T>::kElemsPerChunk;
    const T* p;
    int64_t ld, rows, K;
    bool vec;  // p and ld allow aligned 16-byte loads
    __device__ __forceinline__ u32x4 chunk(int64_t row, int64_t k0) const {
        if (row < rows && vec && k0 + E <= K) return *reinterpret_cast<const u32x4*>(p + row * ld + k0);
        T v[E];
#pragma unroll
        for (int e = 0; e < E; ++e) v[e] = (row < rows && k0 + e < K) ? p[row * ld + k0 + e] : T(0);
        return Pack<T>::make(v);
    }
};

// k-strided, row contiguous: R(row, k) = p[k·ld + row]  (a transposed operand).
template <typename T>
struct ColKLoader {
    static constexpr bool kRowFast = true;
    static constexpr int E = KTraits<T>::kElemsPerChunk;
    const T* p;
    int64_t ld, rows, K;
    __device__ __forceinline__ u32x4 chunk(int64_t row, int64_t k0) const {
        T v[E];
#pragma unroll
        for (int e = 0; e < E; ++e) v[e] = (row < rows && k0 + e < K) ? p[(k0 + e) * ld + row] : T(0);
        return Pack<T>::make(v);
    }
};

// Epilogue: row-major C[m·ldc + n] (fp32 or T), optional bias[n], optional
// accumulate into existing fp32 values; relu: a fused ReLU on the result
// (NaN passes); mask (nullable, C's shape): the backward of a ReLU whose
// output is mask, zero where mask <= 0.
template <typename TC>
struct RowMajorStore {
    TC* c;
    int64_t ldc, M, N;
    const float* bias;   // per column, nullable
    int accumulate;
    int relu = 0;
    const TC* mask = nullptr;
    __device__ __forceinline__ void store(int64_t m, int64_t n, float v) const {
        if (m >= M || n >= N) return;
        if (bias) v += bias[n];
        if (accumulate) v += Io<TC>::ld(c, m * ldc + n);
        if (relu && !(v > 0.f || v != v)) v = 0.f;
        if (mask && Io<TC>::ld(mask, m * ldc + n) <= 0.f) v = 0.f;
        Io<TC>::st(c, m * ldc + n, v);
    }
};

// Split-K partial store: ws[split][m][n] fp32 (dense M×N).
struct PartialStore {
    float* ws;
    int64_t M, N;
    __device__ __forceinline__ void store(int64_t m, int64_t n, float v) const {
        if (m < M && n < N) ws[((int64_t)blockIdx.z * M + m) * N + n] = v;
    }
};

// ---------------------------------------------------------------------------
// LDS fill: each of the 256 threads moves (BM·4)/256 = 2 chunks per operand.
// ---------------------------------------------------------------------------
template <class L>
__device__ __forceinline__ void map_chunk(int i, int& row, int& ch) {
    // i in [0, 512): chunk index inside the 128-row × 4-chunk tile.
    if (L::kRowFast) {
        row = i & 127;
        ch = i >> 7;
    } else {
        row = i >> 2;
        ch = i & 3;
    }
}

template <class L>
__device__ __forceinline__ void fetch(const L& ld, int64_t row0, int64_t k0, u32x4 (&r)[2]) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        int row, ch;
        map_chunk<L>(threadIdx.x + j * kThreads, row, ch);
        r[j] = ld.chunk(row0 + row, k0 + ch * L::E);
    }
}

template <class L>
__device__ __forceinline__ void stash(char* lds, const u32x4 (&r)[2]) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        int row, ch;
        map_chunk<L>(threadIdx.x + j * kThreads, row, ch);
        *reinterpret_cast<u32x4*>(lds + row * kLdsStride + ch * 16) = r[j];
    }
}

// One 64-byte k-slice of MFMAs for this wave's 64×64 sub-tile.
template <typename T>
__device__ __forceinline__ void mma_slice(const char* la, const char* lb, int wm, int wn, f32x4 (&acc)[4][4]) {
    const int lane = threadIdx.x & 63;
    const int r16 = lane & 15, kq = lane >> 4;
    u32x4 a[4], b[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
        a[i] = *reinterpret_cast<const u32x4*>(la + (wm * 64 + i * 16 + r16) * kLdsStride + kq * 16);
#pragma unroll
    for (int j = 0; j < 4; ++j)
        b[j] = *reinterpret_cast<const u32x4*>(lb + (wn * 64 + j * 16 + r16) * kLdsStride + kq * 16);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if constexpr (sizeof(T) == 2) {
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a[i]),
                                                                    __builtin_bit_cast(bf16x8, b[j]), acc[i][j], 0, 0, 0);
            } else {
                const f32x4 af = __builtin_bit_cast(f32x4, a[i]);
                const f32x4 bf = __builtin_bit_cast(f32x4, b[j]);
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af.x, bf.x, acc[i][j], 0, 0, 0);
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af.y, bf.y, acc[i][j], 0, 0, 0);
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af.z, bf.z, acc[i][j], 0, 0, 0);
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af.w, bf.w, acc[i][j], 0, 0, 0);
            }
        }
}

// grid: x = ceil(N/BN), y = ceil(M/BM), z = splits (k range per split = k_per_split).
template <typename T, class LA, class LB, class EP>
__global__ __launch_bounds__(kThreads) void gemm_kernel(LA la, LB lb, EP ep, int64_t M, int64_t N, int64_t K,
                                                        int64_t k_per_split) {
    __shared__ __attribute__((aligned(16))) char lds[2][2][BM * kLdsStride];
    constexpr int BK = KTraits<T>::BK;
    const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;
    const int64_t kb = (int64_t)blockIdx.z * k_per_split;
    const int64_t ke = std::min<int64_t>(K, kb + k_per_split);
    const int wid = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int wm = wid >> 1, wn = wid & 1;

    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int64_t nk = ke > kb ? (ke - kb + BK - 1) / BK : 0;
    u32x4 ra[2], rb[2];
    if (nk > 0) {
        fetch(la, m0, kb, ra);
        fetch(lb, n0, kb, rb);
        stash<LA>(lds[0][0], ra);
        stash<LB>(lds[0][1], rb);
    }
    __syncthreads();
    for (int64_t t = 0; t < nk; ++t) {
        const int cur = (int)(t & 1);
        const bool more = t + 1 < nk;
        if (more) {
            // Loaders zero-fill past K; the split's own end is enforced by
            // clamping through a bounded view of K.
            const int64_t k1 = kb + (t + 1) * BK;
            fetch(la, m0, k1, ra);
            fetch(lb, n0, k1, rb);
        }
        mma_slice<T>(lds[cur][0], lds[cur][1], wm, wn, acc);
        if (more) {
            stash<LA>(lds[cur ^ 1][0], ra);
            stash<LB>(lds[cur ^ 1][1], rb);
        }
        __syncthreads();
    }
    // Epilogue: lane holds column (lane % 16), rows 4·(lane/16)+e of each 16×16 tile.
    const int col = lane & 15, rq = (lane >> 4) * 4;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                ep.store(m0 + wm * 64 + i * 16 + rq + e, n0 + wn * 64 + j * 16 + col, acc[i][j][e]);
}

// Sums split-K partials ws[s][m][n] and hands each total to the epilogue.  A
// block owns 64 consecutive outputs (lane = output, coalesced); its 4 waves
// take the splits round-robin with 8 loads in flight each and combine in LDS
// in wave order, so the summation order is fixed (deterministic).
template <class EP>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ ws, int64_t splits, int64_t M,
                                                            int64_t N, EP ep) {
    __shared__ float red[4][64];
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int64_t i = (int64_t)blockIdx.x * 64 + lane;
    const int64_t MN = M * N;
    float s = 0.f;
    if (i < MN) {
        for (int64_t z = wid; z < splits; z += 32) {
            float t[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int64_t zz = z + 4 * u;
                t[u] = ws[(zz < splits ? zz : splits - 1) * MN + i];
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) s += (z + 4 * u < splits) ? t[u] : 0.f;
        }
    }
    red[wid][lane] = s;
    __syncthreads();
    if (wid == 0 && i < MN) ep.store(i / N, i % N, (red[0][lane] + red[1][lane]) + (red[2][lane] + red[3][lane]));
}

// Vector form of splitk_reduce_kernel for N % 4 == 0: a thread owns 4
// consecutive outputs of one row, loads them as one 16-byte word per split
// (8 splits' loads in flight) and adds the splits in order 0, 1, 2, ...
// With `rows` (per-split row sums rows[z][m], the bias gradient of a Linear),
// the thread that owns column 0 of row m also hands ep.rowsum(m, Σ_z rows).
template <class EP, bool ROWS>
__global__ __launch_bounds__(256) void splitk_reduce4_kernel(const float* __restrict__ ws, int64_t splits, int64_t M,
                                                             int64_t N, EP ep, const float* __restrict__ rows) {
    const int64_t MN = M * N;
    const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i >= MN) return;
    if constexpr (ROWS) {
        if (i % N == 0) {
            const int64_t m = i / N;
            float r = 0.f;
            for (int64_t z = 0; z < splits; ++z) r += rows[z * M + m];
            ep.rowsum(m, r);
        }
    }
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
    int64_t z = 0;
    for (; z + 8 <= splits; z += 8) {
        f32x4 t[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) t[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(ws + (z + u) * MN + i));
#pragma unroll
        for (int u = 0; u < 8; ++u) s += t[u];
    }
    for (; z < splits; ++z) s += __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(ws + z * MN + i));
    const int64_t m = i / N, n = i - m * N;
#pragma unroll
    for (int e = 0; e < 4; ++e) ep.store(m, n + e, s[e]);
}

// Sums split-K partials ws[splits][M][N] (fp32, 16-byte aligned) through
// the epilogue, in split order.
template <class EP>
void launch_splitk_reduce(nott_ctx ctx, const float* ws, int64_t splits, int64_t M, int64_t N, const EP& ep) {
    if (N % 4 == 0 && ((uintptr_t)ws % 16) == 0)
        hipLaunchKernelGGL((splitk_reduce4_kernel<EP, false>), dim3((unsigned)ceil_div(M * N, 1024)), dim3(256), 0,
                           ctx->stream, ws, splits, M, N, ep, nullptr);
    else
        hipLaunchKernelGGL((splitk_reduce_kernel<EP>), dim3((unsigned)ceil_div(M * N, 64)), dim3(256), 0, ctx->stream,
                           ws, splits, M, N, ep);
}

// The same, also reducing per-split row sums rows[splits][M] into
// ep.rowsum (N % 4 == 0 and a 16-byte aligned ws required).
template <class EP>
void launch_splitk_reduce(nott_ctx ctx, const float* ws, int64_t splits, int64_t M, int64_t N, const EP& ep,
                          const float* rows) {
    hipLaunchKernelGGL((splitk_reduce4_kernel<EP, true>), dim3((unsigned)ceil_div(M * N, 1024)), dim3(256), 0,
                       ctx->stream, ws, splits, M, N, ep, rows);
}

// Picks a split count that gives the grid at least ~2 workgroups per CU
// while keeping each split at least `min_k` long.
inline int64_t pick_splits(int64_t tiles, int64_t K, int64_t num_cu, int64_t bk) {
    int64_t want = std::max<int64_t>(1, (2 * num_cu + tiles - 1) / tiles);
    const int64_t max_by_k = std::max<int64_t>(1, K / (8 * bk));
    return std::min<int64_t>(want, max_by_k);
}

// Runs C = A·B with loaders la, lb and epilogue ep.  When the k range is
// split, partials go to the context workspace and the reduce kernel applies
// ep; otherwise the GEMM kernel applies ep directly.  Loaders must report
// their true K (they zero-fill past it); splits cut K into equal ranges.
template <typename T, class LA, class LB, class EP>
int run(nott_ctx ctx, const LA& la, const LB& lb, const EP& ep, int64_t M, int64_t N, int64_t K, int64_t splits = 0) {
    if (M <= 0 || N <= 0) return NOTT_OK;
    constexpr int BK = KTraits<T>::BK;
    const int64_t tn = ceil_div(N, BN), tm = ceil_div(M, BM);
    if (tn > 0x7fffffff || tm > 65535) return fail(ctx, NOTT_ERR_UNSUPPORTED, "gemm: grid too large");
    if (splits <= 0) splits = pick_splits(tn * tm, K, ctx->num_cu, BK);
    splits = std::max<int64_t>(1, std::min<int64_t>(splits, 65535));
    // Split boundaries on BK multiples so that a chunk never straddles two splits.
    int64_t kps = ceil_div(ceil_div(K, splits), BK) * BK;
    splits = std::max<int64_t>(1, ceil_div(K, kps));
    if (K <= 0) {
        kps = 0;
        splits = 1;
    }
    if (splits == 1) {
        hipLaunchKernelGGL((gemm_kernel<T, LA, LB, EP>), dim3((unsigned)tn, (unsigned)tm, 1), dim3(kThreads), 0,
                           ctx->stream, la, lb, ep, M, N, K, std::max<int64_t>(kps, 1));
        return launch_status(ctx, "gemm_kernel");
    }
    float* ws = static_cast<float*>(workspace(ctx, sizeof(float) * (size_t)(splits * M * N)));
    if (!ws) return NOTT_ERR_ALLOC;
    PartialStore ps{ws, M, N};
    hipLaunchKernelGGL((gemm_kernel<T, LA, LB, PartialStore>), dim3((unsigned)tn, (unsigned)tm, (unsigned)splits),
                       dim3(kThreads), 0, ctx->stream, la, lb, ps, M, N, K, kps);
    launch_splitk_reduce(ctx, ws, splits, M, N, ep);
    return launch_status(ctx, "gemm_splitk");
}

// ---------------------------------------------------------------------------
// Small-grid variant for products whose 128×128 grid would leave most CUs
// idle (a Linear layer at a small batch: M = 64 rows, or a 10-column output).
// Tile 64×64 per 256-thread workgroup (4 waves as 2×2, 32×32 each = 2×2
// MFMA 16×16 tiles); a stage holds 256 bytes of k per row (64 fp32 / 128
// bf16), all of it loaded at once (4 chunks per operand per thread), so a
// one-stage workgroup has a single load round trip.  Split-K cuts the k range
// into whole stages to give the grid ~2 workgroups per CU once a tile would
// take more than two stages; the partials are summed in split order by the
// same reduce kernel as above.  Operand and epilogue interfaces as gemm_kernel.
// ---------------------------------------------------------------------------
constexpr int kSmallTile = 64;
constexpr int kSmallPitch = 272;   // 256 bytes of k + 16: a quarter-wave's 16 rows hit distinct 16-byte slots

template <class L>
__device__ __forceinline__ void small_map(int i, int& row, int& ch) {
    // i in [0, 1024): chunk index inside the 64-row × 16-chunk stage.
    if (L::kRowFast) {
        row = i & 63;
        ch = i >> 6;
    } else {
        row = i >> 4;
        ch = i & 15;
    }
}

template <typename T, class LA, class LB, class EP>
__global__ __launch_bounds__(kThreads) void gemm64_kernel(LA la, LB lb, EP ep, int64_t M, int64_t N, int64_t K,
                                                          int64_t k_per_split) {
    __shared__ __attribute__((aligned(16))) char lds[2][kSmallTile * kSmallPitch];
    constexpr int E = KTraits<T>::kElemsPerChunk;
    constexpr int KC = 16 * E;   // k elements per stage
    const int64_t m0 = (int64_t)blockIdx.y * kSmallTile, n0 = (int64_t)blockIdx.x * kSmallTile;
    const int64_t kb = (int64_t)blockIdx.z * k_per_split;
    const int64_t ke = std::min<int64_t>(K, kb + k_per_split);
    const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63;
    const int wm = wid >> 1, wn = wid & 1;
    const int r16 = lane & 15, kq = lane >> 4;

    f32x4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int64_t ns = ke > kb ? (ke - kb + KC - 1) / KC : 0;
    u32x4 ra[4], rb[4];
    auto fetch = [&](int64_t k0) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            int row, ch;
            small_map<LA>(tid + j * kThreads, row, ch);
            ra[j] = la.chunk(m0 + row, k0 + ch * E);
            small_map<LB>(tid + j * kThreads, row, ch);
            rb[j] = lb.chunk(n0 + row, k0 + ch * E);
        }
    };
    if (ns > 0) fetch(kb);
    for (int64_t t = 0; t < ns; ++t) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            int row, ch;
            small_map<LA>(tid + j * kThreads, row, ch);
            *reinterpret_cast<u32x4*>(lds[0] + row * kSmallPitch + ch * 16) = ra[j];
            small_map<LB>(tid + j * kThreads, row, ch);
            *reinterpret_cast<u32x4*>(lds[1] + row * kSmallPitch + ch * 16) = rb[j];
        }
        __syncthreads();
        if (t + 1 < ns) fetch(kb + (t + 1) * KC);
#pragma unroll
        for (int s = 0; s < 4; ++s) {   // four 64-byte k slices
            u32x4 a[2], b[2];
#pragma unroll
            for (int i = 0; i < 2; ++i)
                a[i] = *reinterpret_cast<const u32x4*>(lds[0] + (wm * 32 + i * 16 + r16) * kSmallPitch + s * 64 +
                                                       kq * 16);
#pragma unroll
            for (int j = 0; j < 2; ++j)
                b[j] = *reinterpret_cast<const u32x4*>(lds[1] + (wn * 32 + j * 16 + r16) * kSmallPitch + s * 64 +
                                                       kq * 16);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    if constexpr (sizeof(T) == 2) {
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                            __builtin_bit_cast(bf16x8, a[i]), __builtin_bit_cast(bf16x8, b[j]), acc[i][j], 0, 0, 0);
                    } else {
                        const f32x4 af = __builtin_bit_cast(f32x4, a[i]);
                        const f32x4 bf = __builtin_bit_cast(f32x4, b[j]);
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af.x, bf.x, acc[i][j], 0, 0, 0);
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af.y, bf.y, acc[i][j], 0, 0, 0);
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af.z, bf.z, acc[i][j], 0, 0, 0);
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af.w, bf.w, acc[i][j], 0, 0, 0);
                    }
                }
        }
        __syncthreads();
    }
    const int rq = kq * 4;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                ep.store(m0 + wm * 32 + i * 16 + rq + e, n0 + wn * 32 + j * 16 + r16, acc[i][j][e]);
}

// True when the 128×128 grid of `run` would have fewer workgroups than CUs.
inline bool small_grid(nott_ctx ctx, int64_t M, int64_t N) {
    return ceil_div(M, BM) * ceil_div(N, BN) < ctx->num_cu;
}

// C = A·B on the 64×64 tiles, as run().
template <typename T, class LA, class LB, class EP>
int run_small(nott_ctx ctx, const LA& la, const LB& lb, const EP& ep, int64_t M, int64_t N, int64_t K) {
    if (M <= 0 || N <= 0) return NOTT_OK;
    constexpr int KC = 16 * KTraits<T>::kElemsPerChunk;
    const int64_t tn = ceil_div(N, kSmallTile), tm = ceil_div(M, kSmallTile);
    if (tn > 0x7fffffff || tm > 65535) return fail(ctx, NOTT_ERR_UNSUPPORTED, "gemm: grid too large");
    const int64_t stages = std::max<int64_t>(1, ceil_div(K, KC));
    int64_t splits = 1;
    if (stages > 2) splits = std::min<int64_t>({stages, std::max<int64_t>(1, ceil_div(2 * ctx->num_cu, tn * tm)), 65535});
    const int64_t kps = ceil_div(stages, splits) * KC;   // whole stages per split
    splits = std::max<int64_t>(1, ceil_div(K, kps));
    if (splits == 1) {
        hipLaunchKernelGGL((gemm64_kernel<T, LA, LB, EP>), dim3((unsigned)tn, (unsigned)tm, 1), dim3(kThreads), 0,
                           ctx->stream, la, lb, ep, M, N, K, std::max<int64_t>(K, 1));
        return launch_status(ctx, "gemm64_kernel");
    }
    float* ws = static_cast<float*>(workspace(ctx, sizeof(float) * (size_t)(splits * M * N)));
    if (!ws) return NOTT_ERR_ALLOC;
    PartialStore ps{ws, M, N};
    hipLaunchKernelGGL((gemm64_kernel<T, LA, LB, PartialStore>), dim3((unsigned)tn, (unsigned)tm, (unsigned)splits),
                       dim3(kThreads), 0, ctx->stream, la, lb, ps, M, N, K, kps);
    launch_splitk_reduce(ctx, ws, splits, M, N, ep);
    return launch_status(ctx, "gemm64_splitk");
}

}  // namespace gemm
}  // namespace nott

// ===========================================================================
// Fast bf16 path: plain strided operands (no gathers), K a multiple of 64.
//
//   A(m, k) = A[m·lda + k]   (AT = false)   or   A[k·lda + m]   (AT = true)
//   B(n, k) = B[n·ldb + k]   (BT = false)   or   B[k·ldb + n]   (BT = true)
//
// 128×128 tile per 256-thread workgroup (4 waves as 2×2, each 64×64 = 4×4
// tiles of v_mfma_f32_16x16x32_bf16); a k-stage is 64 deep (two 32-wide
// MFMA slices) and the LDS stages are double-buffered, so a wave runs 32
// MFMAs per barrier and the next stage's global loads are in flight while it
// does.  Both operands sit in LDS as [row][k] 16-byte chunks (row = m or n);
// a transposed operand is transposed in registers on its way in (8×8 bf16
// blocks).  Chunk (row, c) of slice s is at
//   s·8 KiB + (row/16)·1 KiB + c·256 + ((row%16) ^ ((row/16)%8))·16,
// which keeps every 16-row MFMA fragment read, every plain fill (16 rows per
// quarter-wave) and every transposed fill (rows 8j+i of 16 consecutive j)
// on 16 distinct 16-byte slots.
// ===========================================================================
namespace nott {
namespace gemm {
namespace fast {

constexpr int BM = 128, BN = 128, BK = 64;
constexpr int kThreads = 256;
constexpr int kStageBytes = 2 * BM * BK * 2;   // A and B, one stage (32 KiB)

__device__ __forceinline__ int off(int row, int c) {
    const int s = c >> 2, sub = c & 3;
    return (s << 13) + ((row >> 4) << 10) + (sub << 8) + ((((row & 15) ^ ((row >> 4) & 7))) << 4);
}

// One operand tile (128 rows × 64 k) of stage `k0`, staged through registers.
template <bool TR>
struct Fill {
    u32x4 r[TR ? 8 : 4];
    // Plain: chunk c = j·256 + tid -> row = 16·(c / 128) + c % 16, k-chunk (c / 16) % 8.
    // Transposed: threads 0..127 each own an 8k × 8row block
    // (k-block kb = t % 8, row block rb = t / 8).
    __device__ __forceinline__ void load(const bf16_t* __restrict__ p, int64_t ld, int64_t row0, int64_t rows,
                                         int64_t k0, int tid, bool active) {
        if constexpr (!TR) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int c = j * kThreads + tid;
                const int64_t row = row0 + 16 * (c >> 7) + (c & 15);
                const int kc = (c >> 4) & 7;
                const int64_t rr = row < rows ? row : rows - 1;
                r[j] = *reinterpret_cast<const u32x4*>(p + rr * ld + k0 + kc * 8);
            }
        } else {
            if (!active) return;
            const int kb = tid & 7, rb = tid >> 3;
            int64_t col = row0 + rb * 8;
            col = col + 8 <= rows ? col : (rows >= 8 ? rows - 8 : 0);   // clamped reads; masked at the store
#pragma unroll
            for (int e = 0; e < 8; ++e) r[e] = *reinterpret_cast<const u32x4*>(p + (k0 + kb * 8 + e) * ld + col);
        }
    }
    __device__ __forceinline__ void store(char* lds, int tid, bool active) const {
        if constexpr (!TR) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int c = j * kThreads + tid;
                *reinterpret_cast<u32x4*>(lds + off(16 * (c >> 7) + (c & 15), (c >> 4) & 7)) = r[j];
            }
        } else {
            if (!active) return;
            const int kb = tid & 7, rb = tid >> 3;
            // r[e] holds rows rb·8 + 0..7 of k = kb·8 + e; out[i] holds k = kb·8 + 0..7 of row rb·8 + i.
#pragma unroll
            for (int i = 0; i < 8; i += 2) {
                u32x4 o0, o1;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint32_t a = r[2 * e][i >> 1], b = r[2 * e + 1][i >> 1];
                    o0[e] = (a & 0xffffu) | (b << 16);
                    o1[e] = (a >> 16) | (b & 0xffff0000u);
                }
                *reinterpret_cast<u32x4*>(lds + off(rb * 8 + i, kb)) = o0;
                *reinterpret_cast<u32x4*>(lds + off(rb * 8 + i + 1, kb)) = o1;
            }
        }
    }
};

template <bool AT, bool BT, class EP>
__global__ __launch_bounds__(kThreads, 2) void gemm_bf16_kernel(const bf16_t* __restrict__ A, int64_t lda,
                                                                const bf16_t* __restrict__ B, int64_t ldb, EP ep,
                                                                int64_t M, int64_t N, int64_t K, int64_t k_per_split) {
    extern __shared__ __attribute__((aligned(16))) char smem[];
    const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;
    const int64_t kb0 = (int64_t)blockIdx.z * k_per_split;
    const int nk = (int)((std::min<int64_t>(K, kb0 + k_per_split) - kb0) / BK);
    const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63;
    const int wm = wid >> 1, wn = wid & 1, r16 = lane & 15, kq = lane >> 4;
    // Transposed fills: A on threads 0..127, B on 128..255 (one 8×8 block each).
    const bool act_a = !AT || tid < 128, act_b = !BT || tid >= 128;
    const int tid_a = AT ? (tid & 127) : tid, tid_b = BT ? (tid & 127) : tid;

    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    Fill<AT> fa;
    Fill<BT> fb;
    fa.load(A, lda, m0, M, kb0, tid_a, act_a);
    fb.load(B, ldb, n0, N, kb0, tid_b, act_b);
    fa.store(smem, tid_a, act_a);
    fb.store(smem + kStageBytes / 2, tid_b, act_b);
    __syncthreads();
    for (int t = 0; t < nk; ++t) {
        const char* la = smem + (t & 1) * kStageBytes;
        const char* lb = la + kStageBytes / 2;
        const bool more = t + 1 < nk;
        if (more) {
            fa.load(A, lda, m0, M, kb0 + (t + 1) * BK, tid_a, act_a);
            fb.load(B, ldb, n0, N, kb0 + (t + 1) * BK, tid_b, act_b);
        }
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            u32x4 a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) a[i] = *reinterpret_cast<const u32x4*>(la + off(wm * 64 + i * 16 + r16, 4 * s + kq));
#pragma unroll
            for (int j = 0; j < 4; ++j) b[j] = *reinterpret_cast<const u32x4*>(lb + off(wn * 64 + j * 16 + r16, 4 * s + kq));
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a[i]),
                                                                        __builtin_bit_cast(bf16x8, b[j]), acc[i][j], 0, 0, 0);
        }
        if (more) {
            char* na = smem + ((t + 1) & 1) * kStageBytes;
            fa.store(na, tid_a, act_a);
            fb.store(na + kStageBytes / 2, tid_b, act_b);
        }
        __syncthreads();
    }
    const int col = lane & 15, rq = (lane >> 4) * 4;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                ep.store(m0 + wm * 64 + i * 16 + rq + e, n0 + wn * 64 + j * 16 + col, acc[i][j][e]);
}

// Split-K plan: `splits` k-ranges of `kps` (a multiple of BK) each.
inline void plan(nott_ctx ctx, int64_t M, int64_t N, int64_t K, int64_t& splits, int64_t& kps) {
    const int64_t tn = ceil_div(N, BN), tm = ceil_div(M, BM);
    const int64_t nkb = K / BK;
    if (splits <= 0) {
        splits = std::max<int64_t>(1, (2 * (int64_t)ctx->num_cu + tn * tm - 1) / (tn * tm));
        splits = std::min<int64_t>(splits, std::max<int64_t>(1, nkb / 4));   // at least 4 stages per split
    }
    splits = std::max<int64_t>(1, std::min<int64_t>(splits, std::min<int64_t>(nkb, 65535)));
    kps = ceil_div(nkb, splits) * BK;
    splits = ceil_div(K, kps);
}

// fp32 scratch the split-K partials of an M×N product need (0 if unsplit).
inline size_t partial_floats(nott_ctx ctx, int64_t M, int64_t N, int64_t K) {
    int64_t splits = 0, kps = 0;
    plan(ctx, M, N, K, splits, kps);
    return splits > 1 ? (size_t)(splits * M * N) : 0;
}

// C = A·B through the fast path, or NOTT_ERR_UNSUPPORTED when the operands do
// not qualify (then the caller uses the generic engine).  Split-K partials go
// to `partial` when given (partial_floats() of them), else to the workspace.
template <bool AT, bool BT, class EP>
int run(nott_ctx ctx, const bf16_t* A, int64_t lda, const bf16_t* B, int64_t ldb, const EP& ep, int64_t M, int64_t N,
        int64_t K, int64_t splits = 0, float* partial = nullptr) {
    if (M <= 0 || N <= 0) return NOTT_OK;
    auto ok16 = [](const void* p, int64_t ld) { return ((uintptr_t)p % 16) == 0 && (ld % 8) == 0; };
    if (K <= 0 || K % BK != 0 || !ok16(A, lda) || !ok16(B, ldb)) return NOTT_ERR_UNSUPPORTED;
    // transposed operands are read in whole 8-row blocks
    if ((AT && M % 8 != 0) || (BT && N % 8 != 0)) return NOTT_ERR_UNSUPPORTED;
    const int64_t tn = ceil_div(N, BN), tm = ceil_div(M, BM);
    if (tn > 0x7fffffff || tm > 65535) return NOTT_ERR_UNSUPPORTED;
    int64_t kps = 0;
    plan(ctx, M, N, K, splits, kps);
    const size_t lds = 2 * kStageBytes;
    if (splits == 1) {
        hipLaunchKernelGGL((gemm_bf16_kernel<AT, BT, EP>), dim3((unsigned)tn, (unsigned)tm, 1), dim3(kThreads), lds,
                           ctx->stream, A, lda, B, ldb, ep, M, N, K, K);
        return launch_status(ctx, "gemm_bf16");
    }
    float* ws = partial ? partial : static_cast<float*>(workspace(ctx, sizeof(float) * (size_t)(splits * M * N)));
    if (!ws) return NOTT_ERR_ALLOC;
    PartialStore ps{ws, M, N};
    hipLaunchKernelGGL((gemm_bf16_kernel<AT, BT, PartialStore>), dim3((unsigned)tn, (unsigned)tm, (unsigned)splits),
                       dim3(kThreads), lds, ctx->stream, A, lda, B, ldb, ps, M, N, K, kps);
    launch_splitk_reduce(ctx, ws, splits, M, N, ep);
    return launch_status(ctx, "gemm_bf16_splitk");
}

}  // namespace fast
}  // namespace gemm
}  // namespace nott
