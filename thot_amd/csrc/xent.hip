// Fused softmax cross-entropy: loss and logit gradient in one read of the
// logits.
//
// Replaces F::cross_entropy as called by Nott::Loss::Details::compute
// (reference loss/details/ce.hpp:21-37; mean reduction, ignore_index -100,
// label smoothing ε), whose backward libtorch runs as two passes
// (nll_loss_backward, then _log_softmax_backward_data).  Per valid row i:
//   lse = max + log Σ exp(z − max)
//   dz  = grad_scale · (exp(z − lse) − (1−ε)·[j == y] − ε/c) / n_valid
//   loss_i = (1−ε)·(lse − z_y) + (ε/c)·(c·lse − Σ_j z_j)
// Each row lives in registers of one workgroup: one HBM read, one write.
#include "common.hpp"

#include <algorithm>

namespace {

constexpr int64_t kIgnoreIndex = -100;

// Counts valid labels and flags out-of-range ones.  One workgroup.
__global__ __launch_bounds__(1024) void xent_count_kernel(const int64_t* __restrict__ labels, int64_t n, int64_t c,
                                                          int* __restrict__ nvalid,
                                                          unsigned long long* __restrict__ err) {
    __shared__ float red[16];
    float cnt = 0.f;
    unsigned bad = 0;
    constexpr int kBatch = 16;   // labels per thread in flight
    for (int64_t base = threadIdx.x; base < n; base += 1024 * kBatch) {
        int64_t y[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            const int64_t i = base + (int64_t)u * 1024;
            y[u] = labels[i < n ? i : n - 1];
        }
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            if (base + (int64_t)u * 1024 >= n || y[u] == kIgnoreIndex) continue;
            if (y[u] < 0 || y[u] >= c) ++bad;
            else cnt += 1.f;
        }
    }
    // counts up to 2^24 are exact in fp32; larger n is rejected on the host.
    const float total = block_sum<16>(cnt, red);
    if (bad) atomicAdd(err, (unsigned long long)bad);
    if (threadIdx.x == 0) *nvalid = (int)total;
}

template <int NWAVES>
__device__ __forceinline__ void block_sum2(float& a, float& b, float* red) {
    a = wave_sum(a);
    b = wave_sum(b);
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    if (lane == 0) {
        red[wid] = a;
        red[NWAVES + wid] = b;
    }
    __syncthreads();
    float ta = 0.f, tb = 0.f;
#pragma unroll
    for (int i = 0; i < NWAVES; ++i) {
        ta += red[i];
        tb += red[NWAVES + i];
    }
    __syncthreads();
    a = ta;
    b = tb;
}

// Row body: v holds this thread's EPT elements of row `row` (element e of
// group g is column (g·NT + tid)·G + e; −inf past the end).  Writes the
// gradient row and the row's loss.  Every thread calls it (block reductions).
// One exponential per element: p = 2^(v·log2 e − max·log2 e) = e^(v − max)
// is kept in v, and the gradient is scale·(p/Σp − ε/C − (1 − ε)·[j = y])
// (the label's term applied once, by the thread that holds it); the row sum
// of the logits is formed only when label smoothing needs it.
template <typename T, int NT, int EPT, bool VEC>
__device__ __forceinline__ void xent_row_body(float (&v)[EPT], int64_t row, int64_t y, const T* __restrict__ z,
                                              int64_t c, float smoothing, float grad_scale, int nv,
                                              T* __restrict__ dz, float* __restrict__ row_loss, float* red) {
    constexpr int NWAVES = NT / 64;
    constexpr int G = VEC ? Pack16<T>::N : 1;
    constexpr int NG = EPT / G;
    constexpr float kLog2e = 1.4426950408889634f;
    const int ci = (int)c;
    if (!(y >= 0 && y < c)) {
        // Ignored (or out-of-range) row: zero gradient, no loss.
#pragma unroll
        for (int g = 0; g < NG; ++g) {
            const int j0 = (g * NT + (int)threadIdx.x) * G;
            if (j0 >= ci) continue;
            if constexpr (VEC) {
                float t[G];
#pragma unroll
                for (int e = 0; e < G; ++e) t[e] = 0.f;
                Pack16<T>::template st<true>(dz + j0, t);
            } else {
                Io<T>::st(dz, j0, 0.f);
            }
        }
        if (threadIdx.x == 0 && row_loss) row_loss[row] = 0.f;
        return;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int e = 0; e < EPT; ++e) mx = fmaxf(mx, v[e]);
    mx = block_max<NWAVES>(mx, red);
    const float mxl = mx * kLog2e;
    float se = 0.f, sz = 0.f;
    if (smoothing != 0.f) {
#pragma unroll
        for (int e = 0; e < EPT; ++e) sz += (v[e] == -INFINITY) ? 0.f : v[e];
    }
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
        const float pe = __builtin_amdgcn_exp2f(fmaf(v[e], kLog2e, -mxl));
        se += pe;
        v[e] = pe;
    }
    block_sum2<NWAVES>(se, sz, red);
    const float lse = mx + __logf(se);
    const float scale = grad_scale / (float)nv;
    const float off = smoothing / (float)c;
    const float hit = 1.f - smoothing;
    const float ga = scale / se, gb = -scale * off;
    const int yi = (int)y;
#pragma unroll
    for (int g = 0; g < NG; ++g) {
        const int j0 = (g * NT + (int)threadIdx.x) * G;
        if (j0 >= ci) continue;
        float t[G];
#pragma unroll
        for (int e = 0; e < G; ++e) t[e] = fmaf(v[g * G + e], ga, gb);
        if ((unsigned)(yi - j0) < (unsigned)G) {
#pragma unroll
            for (int e = 0; e < G; ++e)
                if (j0 + e == yi) t[e] -= scale * hit;
        }
        if constexpr (VEC) Pack16<T>::template st<true>(dz + j0, t);
        else Io<T>::st(dz, j0, t[0]);
    }
    if (threadIdx.x == 0 && row_loss) {
        const float zy = Io<T>::ld(z, y);
        row_loss[row] = hit * (lse - zy) + off * ((float)c * lse - sz);
    }
}

// Vector path: 16-byte groups of G = 4 (fp32) or 8 (bf16) elements, strided
// by NT·G, loaded unconditionally (past-the-end groups re-read group 0 and
// count as −inf) so all of a thread's loads are in flight together.  The
// grid is persistent (rows blockIdx.x, + gridDim.x, ...) and the next row's
// loads are issued before the current row is reduced and written, so a CU's
// loads stay in flight through the block reductions and the stores.
template <typename T, int NT, int EPT>
__global__ __launch_bounds__(NT) void xent_rows_vec_kernel(const T* __restrict__ logits,
                                                           const int64_t* __restrict__ labels, int64_t n, int64_t c,
                                                           float smoothing, float grad_scale,
                                                           const int* __restrict__ nvalid, T* __restrict__ dlogits,
                                                           float* __restrict__ row_loss) {
    constexpr int G = Pack16<T>::N;
    constexpr int NG = EPT / G;
    __shared__ float red[2 * (NT / 64)];
    typename Pack16<T>::Raw raw[NG];
    int64_t ny = 0;
    auto fetch = [&](int64_t row) {
        const T* z = logits + row * c;
#pragma unroll
        for (int g = 0; g < NG; ++g) {
            const int j0 = (g * NT + (int)threadIdx.x) * G;
            raw[g] = Pack16<T>::template raw<true>(z + (j0 < (int)c ? j0 : 0));
        }
        ny = labels[row];
    };
    const int nv = *nvalid;
    if ((int64_t)blockIdx.x < n) fetch(blockIdx.x);
    for (int64_t row = blockIdx.x; row < n; row += gridDim.x) {
        float v[EPT];
#pragma unroll
        for (int g = 0; g < NG; ++g) {
            const int j0 = (g * NT + (int)threadIdx.x) * G;
            float t[G];
            Pack16<T>::unpack(raw[g], t);
#pragma unroll
            for (int e = 0; e < G; ++e) v[g * G + e] = j0 < (int)c ? t[e] : -INFINITY;
        }
        const int64_t y = ny;
        if (row + gridDim.x < n) fetch(row + gridDim.x);
        xent_row_body<T, NT, EPT, true>(v, row, y, logits + row * c, c, smoothing, grad_scale, nv,
                                        dlogits + row * c, row_loss, red);
    }
}

// Element path (unaligned rows or c not a multiple of G): one workgroup per
// row, single elements strided by NT.
template <typename T, int NT, int EPT>
__global__ __launch_bounds__(NT) void xent_row_kernel(const T* __restrict__ logits, const int64_t* __restrict__ labels,
                                                      int64_t c, float smoothing, float grad_scale,
                                                      const int* __restrict__ nvalid, T* __restrict__ dlogits,
                                                      float* __restrict__ row_loss) {
    __shared__ float red[2 * (NT / 64)];
    const int64_t row = blockIdx.x;
    const T* z = logits + row * c;
    float v[EPT];
#pragma unroll
    for (int g = 0; g < EPT; ++g) {
        const int64_t j0 = (int64_t)g * NT + threadIdx.x;
        v[g] = j0 < c ? Io<T>::ld(z, j0) : -INFINITY;
    }
    xent_row_body<T, NT, EPT, false>(v, row, labels[row], z, c, smoothing, grad_scale, *nvalid, dlogits + row * c,
                                     row_loss, red);
}

// Rows too long for registers: three passes over the row (the re-reads are
// served from L2 / MALL for rows of a few hundred KiB).
template <typename T>
__global__ __launch_bounds__(256) void xent_long_kernel(const T* __restrict__ logits, const int64_t* __restrict__ labels,
                                                        int64_t c, float smoothing, float grad_scale,
                                                        const int* __restrict__ nvalid, T* __restrict__ dlogits,
                                                        float* __restrict__ row_loss) {
    __shared__ float red[8];
    const int64_t row = blockIdx.x;
    const T* z = logits + row * c;
    T* dz = dlogits + row * c;
    const int64_t y = labels[row];
    if (!(y >= 0 && y < c)) {
        for (int64_t j = threadIdx.x; j < c; j += 256) Io<T>::st(dz, j, 0.f);
        if (threadIdx.x == 0 && row_loss) row_loss[row] = 0.f;
        return;
    }
    float mx = -INFINITY;
    for (int64_t j = threadIdx.x; j < c; j += 256) mx = fmaxf(mx, Io<T>::ld(z, j));
    mx = block_max<4>(mx, red);
    float se = 0.f, sz = 0.f;
    for (int64_t j = threadIdx.x; j < c; j += 256) {
        const float t = Io<T>::ld(z, j);
        se += __expf(t - mx);
        sz += t;
    }
    block_sum2<4>(se, sz, red);
    const float lse = mx + __logf(se);
    const float scale = grad_scale / (float)(*nvalid);
    const float off = smoothing / (float)c, hit = 1.f - smoothing;
    for (int64_t j = threadIdx.x; j < c; j += 256)
        Io<T>::st(dz, j, scale * (__expf(Io<T>::ld(z, j) - lse) - off - (j == y ? hit : 0.f)));
    if (threadIdx.x == 0 && row_loss) row_loss[row] = hit * (lse - Io<T>::ld(z, y)) + off * ((float)c * lse - sz);
}

__global__ __launch_bounds__(1024) void xent_loss_kernel(const float* __restrict__ row_loss, int64_t n,
                                                         const int* __restrict__ nvalid, float* __restrict__ loss) {
    __shared__ float red[16];
    float acc = 0.f;
    for (int64_t i = threadIdx.x; i < n; i += 1024) acc += row_loss[i];
    acc = block_sum<16>(acc, red);
    if (threadIdx.x == 0) *loss = (*nvalid > 0) ? acc / (float)(*nvalid) : __builtin_nanf("");
}

__global__ void xent_nan_kernel(float* __restrict__ loss) { *loss = __builtin_nanf(""); }

// Small problems (c <= 64 classes, n <= kSmallRows rows; a classifier head at
// a small batch): the label count, every row and the mean loss in one
// 1024-thread workgroup, where the general path takes three launches.  A wave
// owns rows wid, wid + 16, ... with lane j holding column j; the arithmetic
// and the summation orders are those of xent_count_kernel, the element path
// xent_row_kernel<T, 64, 16> and xent_loss_kernel, so where the general path
// takes the element path (c not a multiple of the 16-byte group) both give
// the same bits; its vector path sums each thread's group first.
constexpr int64_t kSmallRows = 4096;
template <typename T>
__global__ __launch_bounds__(1024) void xent_small_kernel(const T* __restrict__ logits,
                                                          const int64_t* __restrict__ labels, int64_t n, int64_t c,
                                                          float smoothing, float grad_scale, T* __restrict__ dlogits,
                                                          float* __restrict__ loss,
                                                          unsigned long long* __restrict__ err) {
    __shared__ float red[16];
    __shared__ float rl[kSmallRows];
    __shared__ int nvs;
    float cnt = 0.f;
    unsigned bad = 0;
    for (int64_t i = threadIdx.x; i < n; i += 1024) {
        const int64_t y = labels[i];
        if (y == kIgnoreIndex) continue;
        if (y < 0 || y >= c) ++bad;
        else cnt += 1.f;
    }
    const float total = block_sum<16>(cnt, red);
    if (bad) atomicAdd(err, (unsigned long long)bad);
    if (threadIdx.x == 0) nvs = (int)total;
    __syncthreads();
    const int nv = nvs;
    constexpr float kLog2e = 1.4426950408889634f;
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int ci = (int)c;
    for (int64_t row = wid; row < n; row += 16) {
        const T* z = logits + row * c;
        T* dz = dlogits + row * c;
        const int64_t y = labels[row];
        const float v = lane < ci ? Io<T>::ld(z, lane) : -INFINITY;
        if (!(y >= 0 && y < c)) {
            if (lane < ci) Io<T>::st(dz, lane, 0.f);
            if (lane == 0) rl[row] = 0.f;
            continue;
        }
        const float mx = wave_max(v);
        const float sz = smoothing != 0.f ? wave_sum(v == -INFINITY ? 0.f : v) : 0.f;
        const float pe = __builtin_amdgcn_exp2f(fmaf(v, kLog2e, -mx * kLog2e));
        const float se = wave_sum(pe);
        const float lse = mx + __logf(se);
        const float scale = grad_scale / (float)nv;
        const float off = smoothing / (float)c;
        const float hit = 1.f - smoothing;
        if (lane < ci) {
            float g = fmaf(pe, scale / se, -scale * off);
            if (lane == (int)y) g -= scale * hit;
            Io<T>::st(dz, lane, g);
        }
        if (lane == 0) rl[row] = hit * (lse - Io<T>::ld(z, y)) + off * ((float)c * lse - sz);
    }
    if (!loss) return;
    __syncthreads();
    float acc = 0.f;
    for (int64_t i = threadIdx.x; i < n; i += 1024) acc += rl[i];
    acc = block_sum<16>(acc, red);
    if (threadIdx.x == 0) *loss = nv > 0 ? acc / (float)nv : __builtin_nanf("");
}

template <typename T, int NT, int EPT, bool VEC>
void launch_rows(nott_ctx ctx, int64_t n, int64_t c, const void* logits, const int64_t* labels, float eps,
                 float scale, const int* nvalid, void* dl, float* row_loss) {
    if constexpr (VEC) {
        // Persistent grid: as many workgroups as are resident at once, at
        // most one per row.
        static int per_cu = 0;
        if (per_cu == 0 &&
            (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, xent_rows_vec_kernel<T, NT, EPT>, NT, 0) !=
                 hipSuccess ||
             per_cu < 1))
            per_cu = 1;
        const int64_t grid = std::min<int64_t>(n, (int64_t)ctx->num_cu * per_cu);
        hipLaunchKernelGGL((xent_rows_vec_kernel<T, NT, EPT>), dim3((unsigned)grid), dim3(NT), 0, ctx->stream,
                           static_cast<const T*>(logits), labels, n, c, eps, scale, nvalid, static_cast<T*>(dl),
                           row_loss);
    } else {
        hipLaunchKernelGGL((xent_row_kernel<T, NT, EPT>), dim3((unsigned)n), dim3(NT), 0, ctx->stream,
                           static_cast<const T*>(logits), labels, c, eps, scale, nvalid, static_cast<T*>(dl), row_loss);
    }
}

template <typename T>
void dispatch(nott_ctx ctx, int64_t n, int64_t c, const void* logits, const int64_t* labels, float eps, float scale,
              const int* nvalid, void* dl, float* row_loss) {
    const bool vec = (c % Pack16<T>::N == 0) && ((uintptr_t)logits % 16 == 0) && ((uintptr_t)dl % 16 == 0);
    if (vec && c <= 64 * 16)
        launch_rows<T, 64, 16, true>(ctx, n, c, logits, labels, eps, scale, nvalid, dl, row_loss);
    else if (vec && c <= 256 * 32)
        launch_rows<T, 256, 32, true>(ctx, n, c, logits, labels, eps, scale, nvalid, dl, row_loss);
    else if (vec && sizeof(T) == 2 && c <= 512 * 64)
        // bf16 rows of up to 32768: two 512-thread workgroups per CU, so that
        // two rows (plus the two prefetched ones) are in flight per CU.
        launch_rows<T, 512, 64, true>(ctx, n, c, logits, labels, eps, scale, nvalid, dl, row_loss);
    else if (vec && c <= 1024 * 32)
        launch_rows<T, 1024, 32, true>(ctx, n, c, logits, labels, eps, scale, nvalid, dl, row_loss);
    else if (c <= 64 * 16)
        launch_rows<T, 64, 16, false>(ctx, n, c, logits, labels, eps, scale, nvalid, dl, row_loss);
    else if (c <= 512 * 32)
        launch_rows<T, 512, 32, false>(ctx, n, c, logits, labels, eps, scale, nvalid, dl, row_loss);
    else
        hipLaunchKernelGGL(xent_long_kernel<T>, dim3((unsigned)n), dim3(256), 0, ctx->stream,
                           static_cast<const T*>(logits), labels, c, eps, scale, nvalid, static_cast<T*>(dl), row_loss);
}

}  // namespace

extern "C" int nott_softmax_xent_bwd(nott_ctx ctx, nott_dtype dtype, int64_t n, int64_t c, const void* logits,
                                     const int64_t* labels, double label_smoothing, double grad_scale, void* dlogits,
                                     float* loss) {
    NOTT_CHECK_CTX(ctx);
    NOTT_REQUIRE(ctx, nott::valid_dtype(dtype), "nott_softmax_xent_bwd: bad dtype");
    NOTT_REQUIRE(ctx, n >= 0 && c > 0, "nott_softmax_xent_bwd: need n >= 0 and c > 0");
    NOTT_REQUIRE(ctx, n < (int64_t(1) << 24) && n <= 0x7fffffff, "nott_softmax_xent_bwd: n too large");
    NOTT_REQUIRE(ctx, label_smoothing >= 0.0 && label_smoothing <= 1.0, "nott_softmax_xent_bwd: label_smoothing in [0,1]");
    NOTT_REQUIRE(ctx, n == 0 || (logits && labels && dlogits), "nott_softmax_xent_bwd: null buffer");
    nott::DeviceScope scope(ctx->device);
    if (n == 0) {
        if (loss) hipLaunchKernelGGL(xent_nan_kernel, dim3(1), dim3(1), 0, ctx->stream, loss);  // mean of nothing
        return nott::launch_status(ctx, "softmax_xent");
    }
    const float eps = (float)label_smoothing, scale = (float)grad_scale;
    if (c <= 64 && n <= kSmallRows) {
        if (dtype == NOTT_F32)
            hipLaunchKernelGGL(xent_small_kernel<float>, dim3(1), dim3(1024), 0, ctx->stream,
                               static_cast<const float*>(logits), labels, n, c, eps, scale,
                               static_cast<float*>(dlogits), loss, ctx->err_word);
        else
            hipLaunchKernelGGL(xent_small_kernel<bf16_t>, dim3(1), dim3(1024), 0, ctx->stream,
                               static_cast<const bf16_t*>(logits), labels, n, c, eps, scale,
                               static_cast<bf16_t*>(dlogits), loss, ctx->err_word);
        return nott::launch_status(ctx, "softmax_xent");
    }
    // workspace: [nvalid int][pad to 256 B][row_loss n floats]
    char* ws = static_cast<char*>(nott::workspace(ctx, 256 + sizeof(float) * (size_t)n));
    if (!ws) return NOTT_ERR_ALLOC;
    int* nvalid = reinterpret_cast<int*>(ws);
    float* row_loss = loss ? reinterpret_cast<float*>(ws + 256) : nullptr;
    hipLaunchKernelGGL(xent_count_kernel, dim3(1), dim3(1024), 0, ctx->stream, labels, n, c, nvalid, ctx->err_word);
    if (dtype == NOTT_F32)
        dispatch<float>(ctx, n, c, logits, labels, eps, scale, nvalid, dlogits, row_loss);
    else
        dispatch<bf16_t>(ctx, n, c, logits, labels, eps, scale, nvalid, dlogits, row_loss);
    if (loss) hipLaunchKernelGGL(xent_loss_kernel, dim3(1), dim3(1024), 0, ctx->stream, row_loss, n, nvalid, loss);
    return nott::launch_status(ctx, "softmax_xent");
}
