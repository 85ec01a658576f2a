// LayerNorm forward (saves mean / rstd) and backward.
//
// Replaces torch::nn::LayerNorm as TransformerEncoderLayerImpl builds it
// (reference block/details/transformers/classic.hpp:399-404, final norm :495;
// eps 1e-5, elementwise affine), i.e. ATen native_layer_norm and
// native_layer_norm_backward.
//   forward : x̂ = (x − μ)·rstd, rstd = 1/sqrt(var_biased + eps), y = x̂·γ + β
//   backward: g = dy·γ; dx = rstd·(g − Σg/d − x̂·Σ(g·x̂)/d)
//             dγ = Σ_rows dy·x̂, dβ = Σ_rows dy
// One wavefront owns one row: the row's x and dy stay in VGPRs, the two row
// sums are DPP/shuffle wave reductions, and every lane keeps running dγ / dβ
// sums for its columns.  Blocks write per-block column partials; a second
// kernel reduces them (deterministic order).
#include "common.hpp"

#include <mutex>

#include <initializer_list>

namespace {

constexpr int kThreads = 256;  // 4 waves
constexpr int kWaves = kThreads / 64;
constexpr int kReduceThreads = 1024;   // column reduction: 16 waves split the partial rows
constexpr int kReduceWaves = kReduceThreads / 64;
constexpr int kReduceUnroll = 32;  // 16 waves x 32 loads cover 512 partial rows in one round

// Element e of a lane's DPL row values is column col(g, e) with g = e / G:
// group g of lane `lane` covers the 16 bytes at columns [(g*64 + lane)*G, +G),
// G = 4 (fp32) or 8 (bf16), so every wave access is a 1 KB coalesced run.
template <typename T>
__device__ __forceinline__ int64_t row_col(int lane, int e) {
    constexpr int G = Pack16<T>::N;
    return ((int64_t)(e / G) * 64 + lane) * G + e % G;
}

// Every lane issues all of its loads unconditionally (columns past d read
// column 0 and are zeroed afterwards), so a row's loads stay in flight
// together.
template <typename T, int DPL, bool NT>
__device__ __forceinline__ void load_row(const T* __restrict__ p, int64_t d, int lane, float (&v)[DPL]) {
    constexpr int G = Pack16<T>::N;
    typename Pack16<T>::Raw raw[DPL / G > 0 ? DPL / G : 1];
#pragma unroll
    for (int g = 0; g < DPL / G; ++g) {
        const int64_t c0 = ((int64_t)g * 64 + lane) * G;
        raw[g] = Pack16<T>::template raw<NT>(p + (c0 < d ? c0 : 0));
    }
#pragma unroll
    for (int g = 0; g < DPL / G; ++g) {
        const int64_t c0 = ((int64_t)g * 64 + lane) * G;
        float t[G];
        Pack16<T>::unpack(raw[g], t);
#pragma unroll
        for (int e = 0; e < G; ++e) v[G * g + e] = c0 < d ? t[e] : 0.f;
    }
}

// load_row split in two: the raw 16-byte loads, and their conversion to
// floats (columns past d read column 0 and become zero).
template <typename T>
__host__ __device__ constexpr int raw_groups(int dpl) { return dpl / Pack16<T>::N > 0 ? dpl / Pack16<T>::N : 1; }
template <typename T, int DPL, bool NT>
__device__ __forceinline__ void load_raw(const T* __restrict__ p, int64_t d, int lane,
                                         typename Pack16<T>::Raw (&raw)[raw_groups<T>(DPL)]) {
    constexpr int G = Pack16<T>::N;
#pragma unroll
    for (int g = 0; g < DPL / G; ++g) {
        const int64_t c0 = ((int64_t)g * 64 + lane) * G;
        raw[g] = Pack16<T>::template raw<NT>(p + (c0 < d ? c0 : 0));
    }
}
template <typename T, int DPL>
__device__ __forceinline__ void unpack_row(const typename Pack16<T>::Raw (&raw)[raw_groups<T>(DPL)], int64_t d,
                                           int lane, float (&v)[DPL]) {
    constexpr int G = Pack16<T>::N;
#pragma unroll
    for (int g = 0; g < DPL / G; ++g) {
        const int64_t c0 = ((int64_t)g * 64 + lane) * G;
        float t[G];
        Pack16<T>::unpack(raw[g], t);
#pragma unroll
        for (int e = 0; e < G; ++e) v[G * g + e] = c0 < d ? t[e] : 0.f;
    }
}

template <typename T, int DPL, bool NT>
__device__ __forceinline__ void store_row(T* __restrict__ p, int64_t d, int lane, const float (&v)[DPL]) {
    constexpr int G = Pack16<T>::N;
#pragma unroll
    for (int g = 0; g < DPL / G; ++g) {
        const int64_t c0 = ((int64_t)g * 64 + lane) * G;
        float t[G];
#pragma unroll
        for (int e = 0; e < G; ++e) t[e] = v[G * g + e];
        if (c0 < d) Pack16<T>::template st<NT>(p + c0, t);
    }
}

template <typename T, int DPL>
__global__ __launch_bounds__(kThreads) void ln_fwd_kernel(const T* __restrict__ x, const T* __restrict__ gamma,
                                                          const T* __restrict__ beta, float eps, T* __restrict__ y,
                                                          float* __restrict__ mean, float* __restrict__ rstd,
                                                          int64_t rows, int64_t d) {
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    float gm[DPL], bt[DPL];
    load_row<T, DPL, false>(gamma, d, lane, gm);
    load_row<T, DPL, false>(beta, d, lane, bt);
    const float inv_d = 1.f / (float)d;
    for (int64_t r = (int64_t)blockIdx.x * kWaves + wid; r < rows; r += (int64_t)gridDim.x * kWaves) {
        float v[DPL];
        load_row<T, DPL, true>(x + r * d, d, lane, v);
        float s = 0.f;
#pragma unroll
        for (int e = 0; e < DPL; ++e) s += v[e];
        const float mu = wave_sum(s) * inv_d;
        float ss = 0.f;
#pragma unroll
        for (int e = 0; e < DPL; ++e) {
            const float t = row_col<T>(lane, e) < d ? v[e] - mu : 0.f;
            ss += t * t;
        }
        const float rs = 1.f / sqrtf(wave_sum(ss) * inv_d + eps);
#pragma unroll
        for (int e = 0; e < DPL; ++e) v[e] = (v[e] - mu) * rs * gm[e] + bt[e];
        store_row<T, DPL, false>(y + r * d, d, lane, v);
        if (lane == 0) {
            mean[r] = mu;
            rstd[r] = rs;
        }
    }
}

// WAVES waves per block, one block per CU (measured best for configs[2]a:
// 8 waves of one row each, ordinary loads and stores, with the next row's
// loads in flight while the current row is reduced).
template <typename T, int DPL, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void ln_bwd_kernel(const T* __restrict__ x, const T* __restrict__ dy,
                                                            const float* __restrict__ mean,
                                                            const float* __restrict__ rstd,
                                                            const T* __restrict__ gamma, T* __restrict__ dx,
                                                            float* __restrict__ partial, int64_t rows, int64_t d) {
    extern __shared__ float lds[];  // [WAVES][2][d]
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    float gm[DPL];
    load_row<T, DPL, false>(gamma, d, lane, gm);
    float dg[DPL], db[DPL];
#pragma unroll
    for (int e = 0; e < DPL; ++e) dg[e] = db[e] = 0.f;
    const float inv_d = 1.f / (float)d;
    constexpr int kRowsInFlight = 1;
    constexpr int NG = raw_groups<T>(DPL);
    const int64_t stride = (int64_t)gridDim.x * WAVES * kRowsInFlight;
    // The next group of rows is loaded (raw) while the current one is
    // reduced and stored: two groups' loads per wave stay in flight.
    typename Pack16<T>::Raw rx[kRowsInFlight][NG], rd[kRowsInFlight][NG];
    float nmu[kRowsInFlight], nrs[kRowsInFlight];
    auto fetch = [&](int64_t r0) {
#pragma unroll
        for (int i = 0; i < kRowsInFlight; ++i) {
            // Rows past the end re-read the last row (unconditional loads keep
            // every row's loads in flight together); they are not stored.
            const int64_t r = r0 + i < rows ? r0 + i : rows - 1;
            load_raw<T, DPL, false>(x + r * d, d, lane, rx[i]);
            load_raw<T, DPL, false>(dy + r * d, d, lane, rd[i]);
            nmu[i] = mean[r];
            nrs[i] = rstd[r];
        }
    };
    const int64_t first = ((int64_t)blockIdx.x * WAVES + wid) * kRowsInFlight;
    if (first < rows) fetch(first);
    for (int64_t r0 = first; r0 < rows; r0 += stride) {
        float xv[kRowsInFlight][DPL], gv[kRowsInFlight][DPL];
        float mu[kRowsInFlight], rs[kRowsInFlight];
#pragma unroll
        for (int i = 0; i < kRowsInFlight; ++i) {
            unpack_row<T, DPL>(rx[i], d, lane, xv[i]);
            unpack_row<T, DPL>(rd[i], d, lane, gv[i]);
            mu[i] = nmu[i];
            rs[i] = nrs[i];
        }
        if (r0 + stride < rows) fetch(r0 + stride);
#pragma unroll
        for (int i = 0; i < kRowsInFlight; ++i) {
            const int64_t r = r0 + i;
            if (r >= rows) break;
            float sg = 0.f, sgx = 0.f;
#pragma unroll
            for (int e = 0; e < DPL; ++e) {
                const float xh = (xv[i][e] - mu[i]) * rs[i];
                const float dyv = gv[i][e];
                dg[e] += dyv * xh;
                db[e] += dyv;
                const float g = dyv * gm[e];
                sg += g;
                sgx += g * xh;
                xv[i][e] = xh;
                gv[i][e] = g;
            }
            sg = wave_sum(sg) * inv_d;
            sgx = wave_sum(sgx) * inv_d;
#pragma unroll
            for (int e = 0; e < DPL; ++e) xv[i][e] = rs[i] * (gv[i][e] - sg - xv[i][e] * sgx);
            store_row<T, DPL, false>(dx + r * d, d, lane, xv[i]);
        }
    }
    // Combine the waves' column sums and write this block's partial row.
#pragma unroll
    for (int e = 0; e < DPL; ++e) {
        const int64_t col = row_col<T>(lane, e);
        if (col < d) {
            lds[(wid * 2 + 0) * d + col] = dg[e];
            lds[(wid * 2 + 1) * d + col] = db[e];
        }
    }
    __syncthreads();
    // Partial layout [which][16-column group][block][16]: the reduction reads
    // each group's partials as one contiguous run.
    const int64_t ngroups = (d + 15) / 16;
    for (int64_t j = threadIdx.x; j < 2 * d; j += 64 * WAVES) {
        const int which = j >= d;
        const int64_t col = j - which * d;
        float s = 0.f;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) s += lds[(w * 2 + which) * d + col];
        partial[((which * ngroups + col / 16) * gridDim.x + blockIdx.x) * 16 + col % 16] = s;
    }
}

// dgamma / dbeta from ln_bwd_kernel's grouped partials.  One 4-wave block
// per 16-column group of one output: thread = (block row b = tid / 4 mod 64,
// column quad tid % 4), 16-byte loads, kGroupUnroll of them in flight (512
// partial rows in one round), so each wave load reads 1 KB of consecutive
// partials.  Each thread adds its rows in order, the 16 row slots of a wave
// combine by a fixed butterfly and the 4 waves in wave order: the summation
// order does not depend on timing.
constexpr int kGroupUnroll = 8;
__global__ __launch_bounds__(256) void col_reduce_grouped_kernel(const float* __restrict__ partial, int64_t nparts,
                                                                 int64_t d, float* __restrict__ dgamma,
                                                                 float* __restrict__ dbeta, int accumulate) {
    __shared__ f32x4 red[4][4];
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int64_t ngroups = (d + 15) / 16;
    const int64_t gi = blockIdx.x;                  // which · ngroups + group
    const int which = gi >= ngroups;
    const int64_t cg = gi - which * ngroups;
    const int q = tid & 3, br = tid >> 2;
    const f32x4* src = reinterpret_cast<const f32x4*>(partial + gi * nparts * 16) + q;
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
    for (int64_t b0 = 0; b0 < nparts; b0 += 64 * kGroupUnroll) {
        f32x4 t[kGroupUnroll];
#pragma unroll
        for (int u = 0; u < kGroupUnroll; ++u) {
            const int64_t b = b0 + u * 64 + br;
            t[u] = b < nparts ? src[b * 4] : f32x4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int u = 0; u < kGroupUnroll; ++u) s += t[u];
    }
#pragma unroll
    for (int off = 4; off < 64; off <<= 1) {
        s.x += __shfl_xor(s.x, off);
        s.y += __shfl_xor(s.y, off);
        s.z += __shfl_xor(s.z, off);
        s.w += __shfl_xor(s.w, off);
    }
    if (lane < 4) red[wid][lane] = s;
    __syncthreads();
    if (tid >= 4) return;
    s = red[0][q] + red[1][q] + red[2][q] + red[3][q];
    float* out = which ? dbeta : dgamma;
    if (out) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int64_t col = cg * 16 + q * 4 + e;
            if (col < d) out[col] = accumulate ? out[col] + s[e] : s[e];
        }
    }
}

// Sums `nparts` partial rows of 2·d floats into dgamma / dbeta.  A block owns
// 64 columns of one output (lane = column, so every load is a 256-byte
// coalesced run); its 16 waves take the partial rows round-robin, each with
// kReduceUnroll independent loads in flight, and combine in LDS in wave order,
// so the summation order is fixed.
__global__ __launch_bounds__(kReduceThreads) void col_reduce_kernel(const float* __restrict__ partial, int64_t nparts,
                                                                    int64_t d, float* __restrict__ dgamma,
                                                                    float* __restrict__ dbeta, int accumulate) {
    __shared__ float red[kReduceWaves][64];
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int which = blockIdx.y;
    const int64_t col = (int64_t)blockIdx.x * 64 + lane;
    float s = 0.f;
    if (col < d) {
        const float* src = partial + (int64_t)which * d + col;
        for (int64_t b = wid; b < nparts; b += kReduceUnroll * kReduceWaves) {
            // all kReduceUnroll loads in flight at once (indices past the end
            // re-read the last partial row and are not added)
            float t[kReduceUnroll];
#pragma unroll
            for (int u = 0; u < kReduceUnroll; ++u) {
                const int64_t i = b + u * kReduceWaves;
                t[u] = src[(i < nparts ? i : nparts - 1) * 2 * d];
            }
#pragma unroll
            for (int u = 0; u < kReduceUnroll; ++u) s += (b + u * kReduceWaves < nparts) ? t[u] : 0.f;
        }
    }
    red[wid][lane] = s;
    __syncthreads();
    if (wid == 0 && col < d) {
        float t = 0.f;
#pragma unroll
        for (int w = 0; w < kReduceWaves; ++w) t += red[w][lane];
        float* out = which ? dbeta : dgamma;
        if (out) out[col] = accumulate ? out[col] + t : t;
    }
}

// Generic row kernels (any d): one block per row, three passes over the row.
template <typename T>
__global__ __launch_bounds__(kThreads) void ln_fwd_generic(const T* __restrict__ x, const T* __restrict__ gamma,
                                                           const T* __restrict__ beta, float eps, T* __restrict__ y,
                                                           float* __restrict__ mean, float* __restrict__ rstd,
                                                           int64_t d) {
    __shared__ float red[kWaves];
    const int64_t r = blockIdx.x;
    const T* xr = x + r * d;
    float s = 0.f;
    for (int64_t j = threadIdx.x; j < d; j += kThreads) s += Io<T>::ld(xr, j);
    const float mu = block_sum<kWaves>(s, red) / (float)d;
    float ss = 0.f;
    for (int64_t j = threadIdx.x; j < d; j += kThreads) {
        const float t = Io<T>::ld(xr, j) - mu;
        ss += t * t;
    }
    const float rs = 1.f / sqrtf(block_sum<kWaves>(ss, red) / (float)d + eps);
    for (int64_t j = threadIdx.x; j < d; j += kThreads)
        Io<T>::st(y + r * d, j, (Io<T>::ld(xr, j) - mu) * rs * Io<T>::ld(gamma, j) + Io<T>::ld(beta, j));
    if (threadIdx.x == 0) {
        mean[r] = mu;
        rstd[r] = rs;
    }
}

template <typename T>
__global__ __launch_bounds__(kThreads) void ln_bwd_generic(const T* __restrict__ x, const T* __restrict__ dy,
                                                           const float* __restrict__ mean,
                                                           const float* __restrict__ rstd, const T* __restrict__ gamma,
                                                           T* __restrict__ dx, float* __restrict__ partial, int64_t d) {
    __shared__ float red[kWaves];
    const int64_t r = blockIdx.x;
    const float mu = mean[r], rs = rstd[r];
    float sg = 0.f, sgx = 0.f;
    for (int64_t j = threadIdx.x; j < d; j += kThreads) {
        const float xh = (Io<T>::ld(x, r * d + j) - mu) * rs;
        const float dyv = Io<T>::ld(dy, r * d + j);
        const float g = dyv * Io<T>::ld(gamma, j);
        sg += g;
        sgx += g * xh;
        partial[(r * 2 + 0) * d + j] = dyv * xh;
        partial[(r * 2 + 1) * d + j] = dyv;
    }
    sg = block_sum<kWaves>(sg, red) / (float)d;
    sgx = block_sum<kWaves>(sgx, red) / (float)d;
    for (int64_t j = threadIdx.x; j < d; j += kThreads) {
        const float xh = (Io<T>::ld(x, r * d + j) - mu) * rs;
        const float g = Io<T>::ld(dy, r * d + j) * Io<T>::ld(gamma, j);
        Io<T>::st(dx, r * d + j, rs * (g - sg - xh * sgx));
    }
}

// The vector kernels need 16-byte aligned rows of whole 16-byte groups.
template <typename T>
bool vec_ok(int64_t d, std::initializer_list<const void*> ptrs) {
    if (d % Pack16<T>::N != 0 || d > 2048) return false;
    for (const void* p : ptrs)
        if ((uintptr_t)p % 16 != 0) return false;
    return true;
}

// Row values per lane for the vector kernels: 4, 8, 16 or 32, at least one
// 16-byte group.
template <typename T>
int dpl_for(int64_t d) {
    const int dpl = d <= 256 ? 4 : d <= 512 ? 8 : d <= 1024 ? 16 : 32;
    return dpl < Pack16<T>::N ? Pack16<T>::N : dpl;
}

template <typename T>
int fwd(nott_ctx ctx, int64_t rows, int64_t d, const void* x, const void* gamma, const void* beta, float eps, void* y,
        float* mean, float* rstd) {
    const T* xx = static_cast<const T*>(x);
    const T* gg = static_cast<const T*>(gamma);
    const T* bb = static_cast<const T*>(beta);
    T* yy = static_cast<T*>(y);
    const bool vec = vec_ok<T>(d, {x, gamma, beta, y});
    const int64_t blocks = std::min<int64_t>(nott::ceil_div(rows, kWaves), (int64_t)ctx->num_cu * 8);
    const dim3 grid((unsigned)std::max<int64_t>(blocks, 1));
    const int dpl = vec ? dpl_for<T>(d) : 0;
    if (dpl == 4)
        hipLaunchKernelGGL((ln_fwd_kernel<T, 4>), grid, dim3(kThreads), 0, ctx->stream, xx, gg, bb, eps, yy, mean, rstd, rows, d);
    else if (dpl == 8)
        hipLaunchKernelGGL((ln_fwd_kernel<T, 8>), grid, dim3(kThreads), 0, ctx->stream, xx, gg, bb, eps, yy, mean, rstd, rows, d);
    else if (dpl == 16)
        hipLaunchKernelGGL((ln_fwd_kernel<T, 16>), grid, dim3(kThreads), 0, ctx->stream, xx, gg, bb, eps, yy, mean, rstd, rows, d);
    else if (dpl == 32)
        hipLaunchKernelGGL((ln_fwd_kernel<T, 32>), grid, dim3(kThreads), 0, ctx->stream, xx, gg, bb, eps, yy, mean, rstd, rows, d);
    else
        hipLaunchKernelGGL(ln_fwd_generic<T>, dim3((unsigned)rows), dim3(kThreads), 0, ctx->stream, xx, gg, bb, eps, yy,
                           mean, rstd, d);
    return nott::launch_status(ctx, "layernorm_fwd");
}

// Scratch for the column partials of the allocation-free entry point
// (nott_layernorm_bwd_noalloc): one copy per GPU, alive until the process
// ends.  Host code never passes `scratch` itself to a kernel; it uses the
// device address hipGetSymbolAddress returns for the current device.
constexpr size_t kScratchBytes = size_t(16) << 20;
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

// Waves per block of the vector backward kernel: 8 while the block's LDS
// column sums (waves × 2 × d floats) fit 64 KB, else 4.
inline int bwd_waves(int64_t d) { return d <= 1024 ? 8 : 4; }

// Partials need: 2 rows (dgamma, dbeta) of `pcols` columns per block.
template <typename T>
void partial_plan(nott_ctx ctx, int64_t rows, int64_t d, bool vec, int dpl, int64_t& nparts, size_t& pcols) {
    (void)dpl;
    if (vec) {
        nparts = std::min<int64_t>(nott::ceil_div(rows, bwd_waves(d)), (int64_t)ctx->num_cu);
        nparts = std::max<int64_t>(nparts, 1);
    } else {
        nparts = rows;
    }
    pcols = vec ? (size_t)nott::ceil_div(d, 16) * 16 : (size_t)d;
}

template <typename T, int DPL>
void launch_bwd_vec(nott_ctx ctx, dim3 grid, const T* x, const T* dy, const float* mean, const float* rstd,
                    const T* gamma, T* dx, float* partial, int64_t rows, int64_t d) {
    if (bwd_waves(d) == 8)
        hipLaunchKernelGGL((ln_bwd_kernel<T, DPL, 8>), grid, dim3(512), sizeof(float) * 8 * 2 * (size_t)d, ctx->stream,
                           x, dy, mean, rstd, gamma, dx, partial, rows, d);
    else
        hipLaunchKernelGGL((ln_bwd_kernel<T, DPL, 4>), grid, dim3(256), sizeof(float) * 4 * 2 * (size_t)d, ctx->stream,
                           x, dy, mean, rstd, gamma, dx, partial, rows, d);
}

// `fixed` (nullable) replaces the context workspace for the partials;
// `fixed_bytes` is its size.
template <typename T>
int bwd(nott_ctx ctx, int64_t rows, int64_t d, const void* x, const void* dy, const float* mean, const float* rstd,
        const void* gamma, void* dx, float* dgamma, float* dbeta, int accumulate, float* fixed = nullptr,
        size_t fixed_bytes = 0) {
    const T* xx = static_cast<const T*>(x);
    const T* dd = static_cast<const T*>(dy);
    const T* gg = static_cast<const T*>(gamma);
    T* out = static_cast<T*>(dx);
    const bool vec = vec_ok<T>(d, {x, dy, gamma, dx});
    const int dpl = vec ? dpl_for<T>(d) : 0;
    int64_t nparts;
    size_t pcols;
    partial_plan<T>(ctx, rows, d, vec, dpl, nparts, pcols);
    const size_t need = sizeof(float) * 2 * pcols * (size_t)nparts;
    float* partial;
    if (fixed) {
        if (need > fixed_bytes)
            return nott::fail(ctx, NOTT_ERR_UNSUPPORTED,
                              "nott_layernorm_bwd_noalloc: rows=" + std::to_string(rows) + ", d=" + std::to_string(d) +
                                  " needs " + std::to_string(need) + " bytes of scratch; the static scratch holds " +
                                  std::to_string(fixed_bytes));
        partial = fixed;
    } else {
        partial = static_cast<float*>(nott::workspace(ctx, need));
        if (!partial) return NOTT_ERR_ALLOC;
    }
    const dim3 grid((unsigned)nparts);
    if (dpl == 4)
        launch_bwd_vec<T, 4>(ctx, grid, xx, dd, mean, rstd, gg, out, partial, rows, d);
    else if (dpl == 8)
        launch_bwd_vec<T, 8>(ctx, grid, xx, dd, mean, rstd, gg, out, partial, rows, d);
    else if (dpl == 16)
        launch_bwd_vec<T, 16>(ctx, grid, xx, dd, mean, rstd, gg, out, partial, rows, d);
    else if (dpl == 32)
        launch_bwd_vec<T, 32>(ctx, grid, xx, dd, mean, rstd, gg, out, partial, rows, d);
    else
        hipLaunchKernelGGL(ln_bwd_generic<T>, grid, dim3(kThreads), 0, ctx->stream, xx, dd, mean, rstd, gg, out, partial, d);
    if ((dgamma || dbeta) && vec)
        hipLaunchKernelGGL(col_reduce_grouped_kernel, dim3((unsigned)(2 * nott::ceil_div(d, 16))), dim3(256), 0,
                           ctx->stream, partial, nparts, d, dgamma, dbeta, accumulate);
    else if (dgamma || dbeta)
        hipLaunchKernelGGL(col_reduce_kernel, dim3((unsigned)nott::ceil_div(d, 64), 2), dim3(kReduceThreads), 0, ctx->stream,
                           partial, nparts, d, dgamma, dbeta, accumulate);
    return nott::launch_status(ctx, "layernorm_bwd");
}

}  // namespace

namespace nott {

// Device address of `scratch` on each device, looked up once per device by
// nott_create (the context's device is current there).
int layernorm_scratch_setup(nott_ctx ctx) {
    static std::mutex mu;
    static void* addr[64] = {};
    std::lock_guard<std::mutex> g(mu);
    if (ctx->device < 0 || ctx->device >= 64) return fail(ctx, NOTT_ERR_INVALID_ARG, "device index out of range");
    if (!addr[ctx->device]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) return hip_fail(ctx, e, "hipGetSymbolAddress(layernorm scratch)");
        addr[ctx->device] = p;
    }
    ctx->ln_scratch = addr[ctx->device];
    return NOTT_OK;
}

}  // namespace nott

extern "C" int nott_layernorm_fwd(nott_ctx ctx, nott_dtype dtype, int64_t rows, int64_t d, const void* x,
                                  const void* gamma, const void* beta, double eps, void* y, float* mean, float* rstd) {
    NOTT_CHECK_CTX(ctx);
    NOTT_REQUIRE(ctx, nott::valid_dtype(dtype) && rows >= 0 && d > 0, "nott_layernorm_fwd: bad arguments");
    if (rows == 0) return NOTT_OK;
    NOTT_REQUIRE(ctx, x && gamma && beta && y && mean && rstd, "nott_layernorm_fwd: null buffer");
    nott::DeviceScope scope(ctx->device);
    return dtype == NOTT_F32 ? fwd<float>(ctx, rows, d, x, gamma, beta, (float)eps, y, mean, rstd)
                             : fwd<bf16_t>(ctx, rows, d, x, gamma, beta, (float)eps, y, mean, rstd);
}

extern "C" int nott_layernorm_bwd(nott_ctx ctx, nott_dtype dtype, int64_t rows, int64_t d, const void* x,
                                  const void* dy, const float* mean, const float* rstd, const void* gamma, void* dx,
                                  float* dgamma, float* dbeta, int accumulate) {
    NOTT_CHECK_CTX(ctx);
    NOTT_REQUIRE(ctx, nott::valid_dtype(dtype) && rows >= 0 && d > 0, "nott_layernorm_bwd: bad arguments");
    NOTT_REQUIRE(ctx, rows == 0 || (x && dy && mean && rstd && gamma && dx), "nott_layernorm_bwd: null buffer");
    nott::DeviceScope scope(ctx->device);
    if (rows == 0) {
        // Σ over no rows: the parameter gradients are zero (or unchanged).
        if (!accumulate) {
            if (dgamma && nott_zero(ctx, sizeof(float) * d, dgamma) != NOTT_OK) return NOTT_ERR_HIP;
            if (dbeta && nott_zero(ctx, sizeof(float) * d, dbeta) != NOTT_OK) return NOTT_ERR_HIP;
        }
        return NOTT_OK;
    }
    return dtype == NOTT_F32 ? bwd<float>(ctx, rows, d, x, dy, mean, rstd, gamma, dx, dgamma, dbeta, accumulate)
                             : bwd<bf16_t>(ctx, rows, d, x, dy, mean, rstd, gamma, dx, dgamma, dbeta, accumulate);
}

extern "C" int nott_layernorm_bwd_noalloc(nott_ctx ctx, nott_dtype dtype, int64_t rows, int64_t d, const void* x,
                                          const void* dy, const float* mean, const float* rstd, const void* gamma,
                                          void* dx, float* dgamma, float* dbeta, int accumulate) {
    NOTT_CHECK_CTX(ctx);
    NOTT_REQUIRE(ctx, nott::valid_dtype(dtype) && rows >= 0 && d > 0, "nott_layernorm_bwd_noalloc: bad arguments");
    NOTT_REQUIRE(ctx, rows == 0 || (x && dy && mean && rstd && gamma && dx), "nott_layernorm_bwd_noalloc: null buffer");
    NOTT_REQUIRE(ctx, ctx->ln_scratch != nullptr, "nott_layernorm_bwd_noalloc: scratch not set up");
    nott::DeviceScope scope(ctx->device);
    if (rows == 0) {
        if (!accumulate) {
            if (dgamma && nott_zero(ctx, sizeof(float) * d, dgamma) != NOTT_OK) return NOTT_ERR_HIP;
            if (dbeta && nott_zero(ctx, sizeof(float) * d, dbeta) != NOTT_OK) return NOTT_ERR_HIP;
        }
        return NOTT_OK;
    }
    float* sp = static_cast<float*>(ctx->ln_scratch);
    return dtype == NOTT_F32
               ? bwd<float>(ctx, rows, d, x, dy, mean, rstd, gamma, dx, dgamma, dbeta, accumulate, sp, kScratchBytes)
               : bwd<bf16_t>(ctx, rows, d, x, dy, mean, rstd, gamma, dx, dgamma, dbeta, accumulate, sp, kScratchBytes);
}
