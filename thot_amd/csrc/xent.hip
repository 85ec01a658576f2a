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

namespace {

constexpr int64_t kIgnoreIndex = -100;

// Counts valid labels and flags out-of-range ones.  One workgroup.
__global__ __launch_bounds__(1024) void xent_count_kernel(const int64_t* __restrict__ labels, int64_t n, int64_t c,
                                                          int* __restrict__ nvalid,
                                                          unsigned long long* __restrict__ err) {
    __shared__ float red[16];
    float cnt = 0.f;
    unsigned bad = 0;
    for (int64_t i = threadIdx.x; i < n; i += 1024) {
        const int64_t y = labels[i];
        if (y == kIgnoreIndex) continue;
        if (y < 0 || y >= c) {
            ++bad;
            continue;
        }
        cnt += 1.f;
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

// One workgroup of NT threads per row; each thread holds EPT elements
// (VEC-wide groups, strided by NT·VEC) of the row in registers.
template <typename T, int NT, int EPT, int VEC>
__global__ __launch_bounds__(NT) void xent_row_kernel(const T* __restrict__ logits, const int64_t* __restrict__ labels,
                                                      int64_t c, float smoothing, float grad_scale,
                                                      const int* __restrict__ nvalid, T* __restrict__ dlogits,
                                                      float* __restrict__ row_loss) {
    constexpr int NWAVES = NT / 64;
    constexpr int NG = EPT / VEC;
    __shared__ float red[2 * NWAVES];
    const int64_t row = blockIdx.x;
    const T* z = logits + row * c;
    T* dz = dlogits + row * c;
    const int64_t y = labels[row];
    const bool valid = (y >= 0 && y < c);

    float v[EPT];
#pragma unroll
    for (int g = 0; g < NG; ++g) {
        const int64_t j0 = ((int64_t)g * NT + threadIdx.x) * VEC;
        if (VEC == 4) {
            if (j0 < c) {
                f32x4 t = Vec4<T>::ld(z + j0);
                v[g * 4 + 0] = t.x; v[g * 4 + 1] = t.y; v[g * 4 + 2] = t.z; v[g * 4 + 3] = t.w;
            } else {
                v[g * 4 + 0] = v[g * 4 + 1] = v[g * 4 + 2] = v[g * 4 + 3] = -INFINITY;
            }
        } else {
            v[g] = j0 < c ? Io<T>::ld(z, j0) : -INFINITY;
        }
    }
    if (!valid) {
        // Ignored (or out-of-range) row: zero gradient, no loss.
#pragma unroll
        for (int g = 0; g < NG; ++g) {
            const int64_t j0 = ((int64_t)g * NT + threadIdx.x) * VEC;
            if (VEC == 4) {
                if (j0 < c) Vec4<T>::st(dz + j0, f32x4{0.f, 0.f, 0.f, 0.f});
            } else if (j0 < c) {
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
    float se = 0.f, sz = 0.f;
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
        se += __expf(v[e] - mx);
        sz += (v[e] == -INFINITY) ? 0.f : v[e];
    }
    block_sum2<NWAVES>(se, sz, red);
    const float lse = mx + __logf(se);
    const float scale = grad_scale / (float)(*nvalid);
    const float off = smoothing / (float)c;
    const float hit = 1.f - smoothing;
#pragma unroll
    for (int g = 0; g < NG; ++g) {
        const int64_t j0 = ((int64_t)g * NT + threadIdx.x) * VEC;
        if (VEC == 4) {
            if (j0 < c) {
                f32x4 t;
                t.x = scale * (__expf(v[g * 4 + 0] - lse) - off - (j0 + 0 == y ? hit : 0.f));
                t.y = scale * (__expf(v[g * 4 + 1] - lse) - off - (j0 + 1 == y ? hit : 0.f));
                t.z = scale * (__expf(v[g * 4 + 2] - lse) - off - (j0 + 2 == y ? hit : 0.f));
                t.w = scale * (__expf(v[g * 4 + 3] - lse) - off - (j0 + 3 == y ? hit : 0.f));
                Vec4<T>::st(dz + j0, t);
            }
        } else if (j0 < c) {
            Io<T>::st(dz, j0, scale * (__expf(v[g] - lse) - off - (j0 == y ? hit : 0.f)));
        }
    }
    if (threadIdx.x == 0 && row_loss) {
        const float zy = Io<T>::ld(z, y);
        row_loss[row] = hit * (lse - zy) + off * ((float)c * lse - sz);
    }
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

template <typename T, int NT, int EPT, int VEC>
void launch_rows(nott_ctx ctx, int64_t n, int64_t c, const void* logits, const int64_t* labels, float eps,
                 float scale, const int* nvalid, void* dl, float* row_loss) {
    hipLaunchKernelGGL((xent_row_kernel<T, NT, EPT, VEC>), dim3((unsigned)n), dim3(NT), 0, ctx->stream,
                       static_cast<const T*>(logits), labels, c, eps, scale, nvalid, static_cast<T*>(dl), row_loss);
}

template <typename T>
void dispatch(nott_ctx ctx, int64_t n, int64_t c, const void* logits, const int64_t* labels, float eps, float scale,
              const int* nvalid, void* dl, float* row_loss) {
    const bool vec = (c % 4 == 0) && ((uintptr_t)logits % (4 * sizeof(T)) == 0) && ((uintptr_t)dl % (4 * sizeof(T)) == 0);
    if (vec && c <= 4 * 64 * 4)
        launch_rows<T, 64, 16, 4>(ctx, n, c, logits, labels, eps, scale, nvalid, dl, row_loss);
    else if (vec && c <= 4 * 256 * 8)
        launch_rows<T, 256, 32, 4>(ctx, n, c, logits, labels, eps, scale, nvalid, dl, row_loss);
    else if (vec && c <= 4 * 512 * 16)
        launch_rows<T, 512, 64, 4>(ctx, n, c, logits, labels, eps, scale, nvalid, dl, row_loss);
    else if (c <= 64 * 16)
        launch_rows<T, 64, 16, 1>(ctx, n, c, logits, labels, eps, scale, nvalid, dl, row_loss);
    else if (c <= 512 * 32)
        launch_rows<T, 512, 32, 1>(ctx, n, c, logits, labels, eps, scale, nvalid, dl, row_loss);
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
    // workspace: [nvalid int][pad to 256 B][row_loss n floats]
    char* ws = static_cast<char*>(nott::workspace(ctx, 256 + sizeof(float) * (size_t)n));
    if (!ws) return NOTT_ERR_ALLOC;
    int* nvalid = reinterpret_cast<int*>(ws);
    float* row_loss = loss ? reinterpret_cast<float*>(ws + 256) : nullptr;
    hipLaunchKernelGGL(xent_count_kernel, dim3(1), dim3(1024), 0, ctx->stream, labels, n, c, nvalid, ctx->err_word);
    const float eps = (float)label_smoothing, scale = (float)grad_scale;
    if (dtype == NOTT_F32)
        dispatch<float>(ctx, n, c, logits, labels, eps, scale, nvalid, dlogits, row_loss);
    else
        dispatch<bf16_t>(ctx, n, c, logits, labels, eps, scale, nvalid, dlogits, row_loss);
    if (loss) hipLaunchKernelGGL(xent_loss_kernel, dim3(1), dim3(1024), 0, ctx->stream, row_loss, n, nvalid, loss);
    return nott::launch_status(ctx, "softmax_xent");
}
