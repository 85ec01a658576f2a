// Linear forward and backward on the MFMA GEMM engine.
//
// Replaces torch::nn::Linear as built by build_registered_layer(Owner&, const
// FCDescriptor&, size_t) (reference layer/details/fc.hpp:32-49, module at :40)
// and the q/k/v/out projections of MultiHeadAttentionImpl
// (attention/details/head.hpp:38-41), i.e. ATen addmm / mm and their backward:
//   y  = x·wᵀ + b         (NT: both operands k-contiguous)
//   dx = dy·w             (NN: w is k-strided)
//   dw = dyᵀ·x            (TN: both k-strided; split-K over rows)
//   db = Σ_rows dy        (folded into the dw GEMM as an extra all-ones column;
//                          bf16 fast path: a two-phase column sum)
// bf16 operands whose k extent is a multiple of 64 take the direct-to-LDS
// GEMM (gemm_dma.hpp) when both output extents are at least 128, else the
// register-staged fast GEMM (gemm.hpp, namespace fast); everything else the
// generic engine, on 64×64 tiles with split-K (run_small) where its 128×128
// grid would leave CUs idle (small batches, narrow outputs).  Every product runs on the kernels in this library; no
// vendor GEMM is called.
#include "gemm_dma.hpp"

namespace {

using namespace nott::gemm;
using nott::ceil_div;
using nott::launch_status;
using nott::workspace;

template <typename T>
bool vec16(const void* p, int64_t ld) {
    return ((uintptr_t)p % 16) == 0 && ((ld * (int64_t)sizeof(T)) % 16) == 0;
}

// B operand of dw with one extra virtual row of ones: R(row=i, k=m) = x[m·kin + i]
// for i < kin and 1 for i == kin (that output column is db).
template <typename T>
struct ColKOnesLoader {
    static constexpr bool kRowFast = true;
    static constexpr int E = KTraits<T>::kElemsPerChunk;
    const T* p;
    int64_t ld, rows, K;   // rows = kin (the ones row is index `rows`)
    bool ones;
    __device__ __forceinline__ u32x4 chunk(int64_t row, int64_t k0) const {
        T v[E];
        const T one = sizeof(T) == 2 ? T(0x3f80) : T(1);
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const bool ink = k0 + e < K;
            if (row < rows) v[e] = ink ? p[(k0 + e) * ld + row] : T(0);
            else v[e] = (ones && row == rows && ink) ? one : T(0);
        }
        return Pack<T>::make(v);
    }
};

// dw[o][i] for i < kin, db[o] for i == kin.
struct DwDbStore {
    float* dw;
    float* db;
    int64_t nout, kin;
    int accumulate;
    __device__ __forceinline__ void store(int64_t o, int64_t i, float v) const {
        if (o >= nout) return;
        if (i < kin) {
            if (!dw) return;
            float* p = dw + o * kin + i;
            *p = accumulate ? *p + v : v;
        } else if (i == kin && db) {
            db[o] = accumulate ? db[o] + v : v;
        }
    }
};

// dw[o][i] for i < kin (columns past kin are tile padding), db[o] from the
// GEMM's row sums of dy.
struct DwRowsumStore {
    float* dw;
    float* db;
    int64_t nout, kin;
    int accumulate;
    __device__ __forceinline__ void store(int64_t o, int64_t i, float v) const {
        if (o >= nout || i >= kin) return;
        float* p = dw + o * kin + i;
        *p = accumulate ? *p + v : v;
    }
    __device__ __forceinline__ void rowsum(int64_t o, float v) const {
        if (o < nout) db[o] = accumulate ? db[o] + v : v;
    }
};

// db[o] (+)= Σ_r dy[r·nout + o] in two deterministic phases: kColSumSlabs
// row slabs each write a partial row (lane = column, 4 waves split the
// slab's rows), then one pass adds the partials in slab order.
constexpr int kColSumSlabs = 64;

template <typename T>
__global__ __launch_bounds__(256) void colsum_partial_kernel(const T* __restrict__ dy, int64_t rows, int64_t nout,
                                                             float* __restrict__ partial) {
    __shared__ float red[4][64];
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int64_t col = (int64_t)blockIdx.x * 64 + lane;
    const int64_t per = (rows + kColSumSlabs - 1) / kColSumSlabs;
    const int64_t r0 = (int64_t)blockIdx.y * per, r1 = r0 + per < rows ? r0 + per : rows;
    float s = 0.f;
    if (col < nout)
        for (int64_t r = r0 + wid; r < r1; r += 4) s += Io<T>::ld(dy, r * nout + col);
    red[wid][lane] = s;
    __syncthreads();
    if (wid == 0 && col < nout) partial[(int64_t)blockIdx.y * nout + col] = (red[0][lane] + red[1][lane]) + (red[2][lane] + red[3][lane]);
}

// Vector form of colsum_partial_kernel (nout a multiple of the 16-byte
// group, aligned rows): lane = one 16-byte group of columns (8 bf16 / 4
// fp32), the 4 waves split the slab's rows with kColSumUnroll loads in
// flight each, and combine in LDS in wave order.
constexpr int kColSumUnroll = 8;
template <typename T>
__global__ __launch_bounds__(256) void colsum_partial_vec_kernel(const T* __restrict__ dy, int64_t rows, int64_t nout,
                                                                 float* __restrict__ partial) {
    constexpr int G = Pack16<T>::N;
    __shared__ float red[4][64 * G];
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int64_t c0 = ((int64_t)blockIdx.x * 64 + lane) * G;
    const int64_t per = (rows + kColSumSlabs - 1) / kColSumSlabs;
    const int64_t r0 = (int64_t)blockIdx.y * per, r1 = r0 + per < rows ? r0 + per : rows;
    float s[G];
#pragma unroll
    for (int e = 0; e < G; ++e) s[e] = 0.f;
    if (c0 < nout) {
        for (int64_t rb = r0 + wid; rb < r1; rb += 4 * kColSumUnroll) {
            typename Pack16<T>::Raw raw[kColSumUnroll];
#pragma unroll
            for (int u = 0; u < kColSumUnroll; ++u) {
                const int64_t r = rb + 4 * u;
                raw[u] = Pack16<T>::template raw<true>(dy + (r < r1 ? r : r0) * nout + c0);
            }
#pragma unroll
            for (int u = 0; u < kColSumUnroll; ++u) {
                if (rb + 4 * u >= r1) break;
                float t[G];
                Pack16<T>::unpack(raw[u], t);
#pragma unroll
                for (int e = 0; e < G; ++e) s[e] += t[e];
            }
        }
    }
#pragma unroll
    for (int e = 0; e < G; ++e) red[wid][lane * G + e] = s[e];
    __syncthreads();
    for (int j = threadIdx.x; j < 64 * G; j += 256) {
        const int64_t col = (int64_t)blockIdx.x * 64 * G + j;
        if (col < nout) partial[(int64_t)blockIdx.y * nout + col] = (red[0][j] + red[1][j]) + (red[2][j] + red[3][j]);
    }
}

// db[o] (+)= Σ_z partial[z][o] in slab order.
template <typename T>
void launch_colsum(nott_ctx ctx, const T* dy, int64_t rows, int64_t nout, float* part) {
    constexpr int G = Pack16<T>::N;
    if (nout % G == 0 && ((uintptr_t)dy % 16) == 0)
        hipLaunchKernelGGL(colsum_partial_vec_kernel<T>, dim3((unsigned)ceil_div(nout, 64 * G), kColSumSlabs),
                           dim3(256), 0, ctx->stream, dy, rows, nout, part);
    else
        hipLaunchKernelGGL(colsum_partial_kernel<T>, dim3((unsigned)ceil_div(nout, 64), kColSumSlabs), dim3(256), 0,
                           ctx->stream, dy, rows, nout, part);
}

__global__ __launch_bounds__(256) void colsum_finish_kernel(const float* __restrict__ partial, int64_t nout,
                                                            float* __restrict__ db, int accumulate) {
    const int64_t col = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (col >= nout) return;
    float s = 0.f;
#pragma unroll 8
    for (int z = 0; z < kColSumSlabs; ++z) s += partial[(int64_t)z * nout + col];
    db[col] = accumulate ? db[col] + s : s;
}

// db (+)= Σ_rows dy through the two-phase column sum.
template <typename T>
int launch_db(nott_ctx ctx, const T* dy, int64_t m, int64_t nout, float* db, int accumulate) {
    float* part = static_cast<float*>(workspace(ctx, sizeof(float) * kColSumSlabs * (size_t)nout));
    if (!part) return NOTT_ERR_ALLOC;
    launch_colsum<T>(ctx, dy, m, nout, part);
    hipLaunchKernelGGL(colsum_finish_kernel, dim3((unsigned)ceil_div(nout, 256)), dim3(256), 0, ctx->stream, part,
                       nout, db, accumulate);
    return launch_status(ctx, "linear db");
}

// bf16 C = A·B on the direct-to-LDS engine, else the register-staged one;
// NOTT_ERR_UNSUPPORTED when neither takes the operands.
template <bool AT, bool BT, class EP>
int bf16_gemm(nott_ctx ctx, const bf16_t* A, int64_t lda, const bf16_t* B, int64_t ldb, const EP& ep, int64_t M,
              int64_t N, int64_t K) {
    const int st = dma::run<AT, BT>(ctx, A, lda, B, ldb, ep, M, N, K);
    if (st != NOTT_ERR_UNSUPPORTED) return st;
    return fast::run<AT, BT>(ctx, A, lda, B, ldb, ep, M, N, K);
}

template <typename T>
int fwd(nott_ctx ctx, int64_t m, int64_t kin, int64_t nout, const void* x, const void* w, const float* b, void* y,
        int relu) {
    if constexpr (sizeof(T) == 2) {
        RowMajorStore<T> ep{static_cast<T*>(y), nout, m, nout, b, 0, relu};
        const int st = bf16_gemm<false, false>(ctx, static_cast<const T*>(x), kin, static_cast<const T*>(w), kin, ep,
                                               m, nout, kin);
        if (st != NOTT_ERR_UNSUPPORTED) return st;
    }
    const T* xp = static_cast<const T*>(x);
    const T* wp = static_cast<const T*>(w);
    RowKLoader<T> la{xp, kin, m, kin, vec16<T>(x, kin)};
    RowKLoader<T> lb{wp, kin, nout, kin, vec16<T>(w, kin)};
    RowMajorStore<T> ep{static_cast<T*>(y), nout, m, nout, b, 0, relu};
    if (small_grid(ctx, m, nout)) return run_small<T>(ctx, la, lb, ep, m, nout, kin);
    return run<T>(ctx, la, lb, ep, m, nout, kin);
}

template <typename T>
int bwd(nott_ctx ctx, int64_t m, int64_t kin, int64_t nout, const void* dy, const void* x, const void* w, void* dx,
        float* dw, float* db, int accumulate, int relu_input) {
    const T* dyp = static_cast<const T*>(dy);
    // relu_input: x is a ReLU's output, whose backward dx takes (zero where x <= 0)
    const T* dx_mask = relu_input ? static_cast<const T*>(x) : nullptr;
    // A db-only request (no dw) is the column sum alone.
    if (db && !dw) {
        const int st = launch_db<T>(ctx, dyp, m, nout, db, accumulate);
        if (st != NOTT_OK) return st;
        db = nullptr;
    }
    if (!dx && !dw && !db) return NOTT_OK;
    if constexpr (sizeof(T) == 2) {
        // dx = dy·w: A = dy (k = o contiguous), B(i, o) = w[o·kin + i] (transposed)
        // dw = dyᵀ·x: A(o, r) = dy[r·nout + o], B(i, r) = x[r·kin + i] (both transposed)
        const bool fx = !dx || (nout % fast::BK == 0 && kin % 8 == 0);
        const bool fw = !dw || (m % fast::BK == 0 && nout % 8 == 0 && kin % 8 == 0);
        if (fx && fw) {
            if (dx) {
                RowMajorStore<T> ep{static_cast<T*>(dx), kin, m, kin, nullptr, 0, 0, dx_mask};
                const int st = bf16_gemm<false, true>(ctx, dyp, nout, static_cast<const T*>(w), kin, ep, m, kin, nout);
                if (st != NOTT_ERR_UNSUPPORTED) {
                    if (st != NOTT_OK) return st;
                    dx = nullptr;
                }
            }
            if (dw && db) {
                // db = Σ_rows dy summed from the dw GEMM's dy fragments.
                DwRowsumStore ep{dw, db, nout, kin, accumulate};
                const int st = dma::run<true, true, true>(ctx, dyp, nout, static_cast<const T*>(x), kin, ep, nout, kin,
                                                          m);
                if (st != NOTT_ERR_UNSUPPORTED) {
                    if (st != NOTT_OK) return st;
                    dw = nullptr;
                    db = nullptr;
                }
            }
            if (dw) {
                DwDbStore ep{dw, nullptr, nout, kin, accumulate};
                const int st = bf16_gemm<true, true>(ctx, dyp, nout, static_cast<const T*>(x), kin, ep, nout, kin, m);
                if (st != NOTT_ERR_UNSUPPORTED) {
                    if (st != NOTT_OK) return st;
                    dw = nullptr;
                    if (db) {
                        const int st2 = launch_db<T>(ctx, dyp, m, nout, db, accumulate);
                        if (st2 != NOTT_OK) return st2;
                        db = nullptr;
                    }
                }
            }
        }
    }
    if (dx) {
        RowKLoader<T> la{dyp, nout, m, nout, vec16<T>(dy, nout)};
        ColKLoader<T> lb{static_cast<const T*>(w), kin, kin, nout};
        RowMajorStore<T> ep{static_cast<T*>(dx), kin, m, kin, nullptr, 0, 0, dx_mask};
        const int st = small_grid(ctx, m, kin) ? run_small<T>(ctx, la, lb, ep, m, kin, nout)
                                               : run<T>(ctx, la, lb, ep, m, kin, nout);
        if (st != NOTT_OK) return st;
    }
    if (dw || db) {
        ColKLoader<T> la{dyp, nout, nout, m};
        ColKOnesLoader<T> lb{static_cast<const T*>(x), kin, kin, m, db != nullptr};
        DwDbStore ep{dw, db, nout, kin, accumulate};
        const int st = small_grid(ctx, nout, kin + 1) ? run_small<T>(ctx, la, lb, ep, nout, kin + 1, m)
                                                      : run<T>(ctx, la, lb, ep, nout, kin + 1, m);
        if (st != NOTT_OK) return st;
    }
    return NOTT_OK;
}

}  // namespace

extern "C" int nott_linear_fwd(nott_ctx ctx, nott_dtype dtype, int64_t m, int64_t kin, int64_t nout, const void* x,
                               const void* w, const float* b, void* y) {
    NOTT_CHECK_CTX(ctx);
    NOTT_REQUIRE(ctx, nott::valid_dtype(dtype), "nott_linear_fwd: bad dtype");
    NOTT_REQUIRE(ctx, m >= 0 && kin > 0 && nout > 0, "nott_linear_fwd: need m >= 0, kin > 0, nout > 0");
    if (m == 0) return NOTT_OK;
    NOTT_REQUIRE(ctx, x && w && y, "nott_linear_fwd: null buffer");
    nott::DeviceScope scope(ctx->device);
    return dtype == NOTT_F32 ? fwd<float>(ctx, m, kin, nout, x, w, b, y, 0) : fwd<bf16_t>(ctx, m, kin, nout, x, w, b, y, 0);
}

extern "C" int nott_linear_fwd_act(nott_ctx ctx, nott_dtype dtype, int64_t m, int64_t kin, int64_t nout,
                                   const void* x, const void* w, const float* b, int relu, void* y) {
    NOTT_CHECK_CTX(ctx);
    NOTT_REQUIRE(ctx, nott::valid_dtype(dtype), "nott_linear_fwd_act: bad dtype");
    NOTT_REQUIRE(ctx, m >= 0 && kin > 0 && nout > 0, "nott_linear_fwd_act: need m >= 0, kin > 0, nout > 0");
    if (m == 0) return NOTT_OK;
    NOTT_REQUIRE(ctx, x && w && y, "nott_linear_fwd_act: null buffer");
    nott::DeviceScope scope(ctx->device);
    const int r = relu != 0;
    return dtype == NOTT_F32 ? fwd<float>(ctx, m, kin, nout, x, w, b, y, r) : fwd<bf16_t>(ctx, m, kin, nout, x, w, b, y, r);
}

extern "C" int nott_linear_bwd_act(nott_ctx ctx, nott_dtype dtype, int64_t m, int64_t kin, int64_t nout,
                                   const void* dy, const void* x, const void* w, void* dx, float* dw, float* db,
                                   int accumulate, int relu_input) {
    NOTT_CHECK_CTX(ctx);
    NOTT_REQUIRE(ctx, nott::valid_dtype(dtype), "nott_linear_bwd: bad dtype");
    NOTT_REQUIRE(ctx, m >= 0 && kin > 0 && nout > 0, "nott_linear_bwd: need m >= 0, kin > 0, nout > 0");
    NOTT_REQUIRE(ctx, dy != nullptr || m == 0, "nott_linear_bwd: null dy");
    NOTT_REQUIRE(ctx, !dx || w, "nott_linear_bwd: dx needs w");
    NOTT_REQUIRE(ctx, !dw || x || m == 0, "nott_linear_bwd: dw needs x");
    NOTT_REQUIRE(ctx, !relu_input || !dx || x || m == 0, "nott_linear_bwd_act: relu_input needs x");
    nott::DeviceScope scope(ctx->device);
    if (m == 0) {
        // Empty batch: dx is empty; the parameter gradients sum over nothing.
        if (!accumulate) {
            if (dw && nott_zero(ctx, (int64_t)sizeof(float) * nout * kin, dw) != NOTT_OK) return NOTT_ERR_HIP;
            if (db && nott_zero(ctx, (int64_t)sizeof(float) * nout, db) != NOTT_OK) return NOTT_ERR_HIP;
        }
        return NOTT_OK;
    }
    const int r = relu_input != 0 && dx != nullptr;
    return dtype == NOTT_F32 ? bwd<float>(ctx, m, kin, nout, dy, x, w, dx, dw, db, accumulate, r)
                             : bwd<bf16_t>(ctx, m, kin, nout, dy, x, w, dx, dw, db, accumulate, r);
}

extern "C" int nott_linear_bwd(nott_ctx ctx, nott_dtype dtype, int64_t m, int64_t kin, int64_t nout, const void* dy,
                               const void* x, const void* w, void* dx, float* dw, float* db, int accumulate) {
    return nott_linear_bwd_act(ctx, dtype, m, kin, nout, dy, x, w, dx, dw, db, accumulate, 0);
}
