// Shared device and host helpers for libnott_hip (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <string>
#include <vector>

#include "nott_hip.h"

// ---------------------------------------------------------------------------
// Context
// ---------------------------------------------------------------------------
struct nott_ctx_s {
    int device = 0;
    hipStream_t stream = nullptr;
    void* ws = nullptr;            // current device workspace
    size_t ws_bytes = 0;
    std::vector<void*> retired;    // earlier, smaller workspaces: kept until nott_destroy
    size_t retired_bytes = 0;      // their total size
    void* ln_scratch = nullptr;    // this device's static LayerNorm scratch (nott_layernorm_bwd_noalloc)
    unsigned long long* err_word = nullptr;  // device counter of data errors
    int num_cu = 256;
    int conv_tap = 1;              // 0: NOTT_CONV_TAP=0 in the environment at nott_create (conv_tap.hip / conv_stem.hip kernels off)
    int conv_dma = 3;              // NOTT_CONV_DMA at nott_create: bit 0 bf16 3x3 fwd/dgrad, bit 1 bf16 3x3 wgrad on conv3x3_dma.hip
    std::string last_error;
};

namespace nott {

// Sets the calling thread's device to the context's device for the scope.
struct DeviceScope {
    int prev = -1;
    bool changed = false;
    explicit DeviceScope(int dev) {
        if (hipGetDevice(&prev) == hipSuccess && prev != dev) {
            changed = (hipSetDevice(dev) == hipSuccess);
        }
    }
    ~DeviceScope() {
        if (changed) (void)hipSetDevice(prev);
    }
};

int fail(nott_ctx ctx, int status, const std::string& msg);
int hip_fail(nott_ctx ctx, hipError_t e, const char* what);
// Returns a workspace pointer of at least `bytes`; nullptr on failure (error
// already set).  Growth allocates a new arena (at least twice the old size)
// and retires the old one without freeing it: kernels still in flight on any
// stream, and HIP graphs captured with the old pointer, keep valid memory.
// Retired arenas are freed by nott_destroy.
void* workspace(nott_ctx ctx, size_t bytes);
// Looks up this device's static LayerNorm scratch (layernorm.hip).
int layernorm_scratch_setup(nott_ctx ctx);
// Checks the last launch and records an error message.
int launch_status(nott_ctx ctx, const char* kernel);

inline size_t dtype_size(nott_dtype t) { return t == NOTT_BF16 ? 2 : 4; }
inline bool valid_dtype(int t) { return t == NOTT_F32 || t == NOTT_BF16; }

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace nott

#define NOTT_CHECK_CTX(ctx)                                          \
    do {                                                             \
        if (!(ctx)) return NOTT_ERR_INVALID_ARG;                     \
    } while (0)

#define NOTT_REQUIRE(ctx, cond, msg)                                 \
    do {                                                             \
        if (!(cond)) return nott::fail((ctx), NOTT_ERR_INVALID_ARG, (msg)); \
    } while (0)

#define NOTT_HIP(ctx, expr)                                          \
    do {                                                             \
        hipError_t _e = (expr);                                      \
        if (_e != hipSuccess) return nott::hip_fail((ctx), _e, #expr); \
    } while (0)

// ---------------------------------------------------------------------------
// Device helpers
// ---------------------------------------------------------------------------
typedef uint16_t bf16_t;   // bf16 storage

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float bf16_to_f32(bf16_t h) {
    return __builtin_bit_cast(float, (uint32_t)h << 16);
}

// Round to nearest even; NaN maps to a quiet NaN of the same sign (gfx950's
// v_cvt_pk_bf16_f32).
__device__ __forceinline__ bf16_t f32_to_bf16(float f) {
    return __builtin_bit_cast(bf16_t, (__bf16)f);
}

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
// Two floats -> packed bf16 pair (a in the low half), one instruction.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
}

template <typename T> struct Io;
template <> struct Io<float> {
    static __device__ __forceinline__ float ld(const float* p, int64_t i) { return p[i]; }
    static __device__ __forceinline__ void st(float* p, int64_t i, float v) { p[i] = v; }
};
template <> struct Io<bf16_t> {
    static __device__ __forceinline__ float ld(const bf16_t* p, int64_t i) { return bf16_to_f32(p[i]); }
    static __device__ __forceinline__ void st(bf16_t* p, int64_t i, float v) { p[i] = f32_to_bf16(v); }
};

// 4-element vector load/store in either storage type (8 or 16 bytes).
template <typename T> struct Vec4;
template <> struct Vec4<float> {
    static __device__ __forceinline__ f32x4 ld(const float* p) { return *reinterpret_cast<const f32x4*>(p); }
    static __device__ __forceinline__ void st(float* p, f32x4 v) { *reinterpret_cast<f32x4*>(p) = v; }
};
template <> struct Vec4<bf16_t> {
    static __device__ __forceinline__ f32x4 ld(const bf16_t* p) {
        u32x2 u = *reinterpret_cast<const u32x2*>(p);
        f32x4 r;
        r.x = __builtin_bit_cast(float, u.x << 16);
        r.y = __builtin_bit_cast(float, u.x & 0xffff0000u);
        r.z = __builtin_bit_cast(float, u.y << 16);
        r.w = __builtin_bit_cast(float, u.y & 0xffff0000u);
        return r;
    }
    static __device__ __forceinline__ void st(bf16_t* p, f32x4 v) {
        u32x2 u;
        u.x = (uint32_t)f32_to_bf16(v.x) | ((uint32_t)f32_to_bf16(v.y) << 16);
        u.y = (uint32_t)f32_to_bf16(v.z) | ((uint32_t)f32_to_bf16(v.w) << 16);
        *reinterpret_cast<u32x2*>(p) = u;
    }
};

// One 16-byte group (4 fp32 or 8 bf16 elements) as floats.  NT = streaming
// access (nontemporal: the line is not kept in the caches after use), for
// data that is read or written exactly once.  raw() + unpack() split a load
// so that a guarded load can be issued without converting inside the guard:
// a conversion inside the branch makes the compiler wait for each load before
// leaving it, which serialises a wave's loads.
// (The fp32 raw type is f32x4, not u32x4: bit-casting u32x4 elements to
// float makes this compiler split or drop parts of the 16-byte load.)
template <typename T> struct Pack16;
template <> struct Pack16<float> {
    static constexpr int N = 4;
    typedef f32x4 Raw;
    template <bool NT = false>
    static __device__ __forceinline__ Raw raw(const float* p) {
        const Raw* q = reinterpret_cast<const Raw*>(p);
        return NT ? __builtin_nontemporal_load(q) : *q;
    }
    static __device__ __forceinline__ void unpack(const Raw& u, float (&v)[4]) {
        v[0] = u.x; v[1] = u.y; v[2] = u.z; v[3] = u.w;
    }
    template <bool NT = false>
    static __device__ __forceinline__ void ld(const float* p, float (&v)[4]) {
        const f32x4* q = reinterpret_cast<const f32x4*>(p);
        const f32x4 t = NT ? __builtin_nontemporal_load(q) : *q;
        v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
    }
    template <bool NT = false>
    static __device__ __forceinline__ void st(float* p, const float (&v)[4]) {
        const f32x4 t = {v[0], v[1], v[2], v[3]};
        f32x4* q = reinterpret_cast<f32x4*>(p);
        if (NT) __builtin_nontemporal_store(t, q);
        else *q = t;
    }
};
template <> struct Pack16<bf16_t> {
    static constexpr int N = 8;
    typedef u32x4 Raw;
    template <bool NT = false>
    static __device__ __forceinline__ Raw raw(const bf16_t* p) {
        const Raw* q = reinterpret_cast<const Raw*>(p);
        return NT ? __builtin_nontemporal_load(q) : *q;
    }
    static __device__ __forceinline__ void unpack(const Raw& u, float (&v)[8]) {
        v[0] = __builtin_bit_cast(float, u.x << 16); v[1] = __builtin_bit_cast(float, u.x & 0xffff0000u);
        v[2] = __builtin_bit_cast(float, u.y << 16); v[3] = __builtin_bit_cast(float, u.y & 0xffff0000u);
        v[4] = __builtin_bit_cast(float, u.z << 16); v[5] = __builtin_bit_cast(float, u.z & 0xffff0000u);
        v[6] = __builtin_bit_cast(float, u.w << 16); v[7] = __builtin_bit_cast(float, u.w & 0xffff0000u);
    }
    template <bool NT = false>
    static __device__ __forceinline__ void ld(const bf16_t* p, float (&v)[8]) {
        const u32x4* q = reinterpret_cast<const u32x4*>(p);
        const u32x4 u = NT ? __builtin_nontemporal_load(q) : *q;
        v[0] = __builtin_bit_cast(float, u.x << 16); v[1] = __builtin_bit_cast(float, u.x & 0xffff0000u);
        v[2] = __builtin_bit_cast(float, u.y << 16); v[3] = __builtin_bit_cast(float, u.y & 0xffff0000u);
        v[4] = __builtin_bit_cast(float, u.z << 16); v[5] = __builtin_bit_cast(float, u.z & 0xffff0000u);
        v[6] = __builtin_bit_cast(float, u.w << 16); v[7] = __builtin_bit_cast(float, u.w & 0xffff0000u);
    }
    template <bool NT = false>
    static __device__ __forceinline__ void st(bf16_t* p, const float (&v)[8]) {
        u32x4 u;
        u.x = pack_bf16x2(v[0], v[1]);
        u.y = pack_bf16x2(v[2], v[3]);
        u.z = pack_bf16x2(v[4], v[5]);
        u.w = pack_bf16x2(v[6], v[7]);
        u32x4* q = reinterpret_cast<u32x4*>(p);
        if (NT) __builtin_nontemporal_store(u, q);
        else *q = u;
    }
};

// DPP move within a row of 16 lanes.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}

// Value of lane L (wave-uniform).
template <int L>
__device__ __forceinline__ float lane_f32(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), L));
}

// ReLU as torch::relu computes it (reference relu.hpp:13): a NaN passes.
__device__ __forceinline__ float relu_out(float x) { return (x > 0.f || x != x) ? x : 0.f; }

// Σ_{z<n} p[z·stride] (n ≥ 1) as 4 floats, added in z order, with the loads
// of 8 consecutive z in flight together (a loop over a run-time count
// otherwise waits for each load before issuing the next).  Loads past n
// re-read the last term and are not added.
__device__ __forceinline__ f32x4 ordered_sum4(const float* __restrict__ p, int64_t stride, int32_t n) {
    f32x4 s = *reinterpret_cast<const f32x4*>(p);
    for (int32_t z = 1; z < n; z += 8) {
        f32x4 t[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) t[u] = *reinterpret_cast<const f32x4*>(p + (int64_t)min(z + u, n - 1) * stride);
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (z + u < n) s += t[u];
    }
    return s;
}
__device__ __forceinline__ float ordered_sum1(const float* __restrict__ p, int64_t stride, int32_t n) {
    float s = p[0];
    for (int32_t z = 1; z < n; z += 8) {
        float t[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) t[u] = p[(int64_t)min(z + u, n - 1) * stride];
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (z + u < n) s += t[u];
    }
    return s;
}

// Full 64-lane sum; every lane receives the result.  Within a row of 16
// lanes: DPP quad_perm / half-mirror / mirror; across rows: lane reads.
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f32<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_f32<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_f32<0x141>(v);  // row_half_mirror
    v += dpp_f32<0x140>(v);  // row_mirror
    // Every lane of a 16-lane row now holds the row's sum; combine the four
    // rows through scalar registers (no LDS round trip), in the order
    // (r0 + r1) + (r2 + r3).
    return (lane_f32<0>(v) + lane_f32<16>(v)) + (lane_f32<32>(v) + lane_f32<48>(v));
}

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f32<0xB1>(v));
    v = fmaxf(v, dpp_f32<0x4E>(v));
    v = fmaxf(v, dpp_f32<0x141>(v));
    v = fmaxf(v, dpp_f32<0x140>(v));
    return fmaxf(fmaxf(lane_f32<0>(v), lane_f32<16>(v)), fmaxf(lane_f32<32>(v), lane_f32<48>(v)));
}

// Block-wide sum over NWAVES waves through LDS; all threads get the result.
// `red` must hold NWAVES floats; the call contains two barriers.
template <int NWAVES>
__device__ __forceinline__ float block_sum(float v, float* red) {
    v = wave_sum(v);
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    if (lane == 0) red[wid] = v;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < NWAVES; ++i) t += red[i];
    __syncthreads();
    return t;
}

template <int NWAVES>
__device__ __forceinline__ float block_max(float v, float* red) {
    v = wave_max(v);
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    if (lane == 0) red[wid] = v;
    __syncthreads();
    float t = -INFINITY;
#pragma unroll
    for (int i = 0; i < NWAVES; ++i) t = fmaxf(t, red[i]);
    __syncthreads();
    return t;
}

// Unsigned 32-bit division by a runtime-invariant divisor via multiply-high
// (Granlund & Montgomery 1994): q = (mulhi(n, magic) + n) >> shift, exact for
// every n < 2^32.  Used by the implicit-GEMM index decompositions.
struct FastDiv {
    uint32_t d = 1, magic = 0, shift = 0;
    FastDiv() = default;
    explicit FastDiv(uint32_t div) : d(div) {
        uint32_t l = 0;
        while (l < 32 && (uint64_t(1) << l) < div) ++l;
        shift = l;
        magic = (uint32_t)(((uint64_t(1) << 32) * ((uint64_t(1) << l) - div)) / div + 1);
    }
    __device__ __forceinline__ uint32_t div(uint32_t n) const {
        const uint64_t hi = ((uint64_t)n * magic) >> 32;
        return (uint32_t)((hi + n) >> shift);
    }
    __device__ __forceinline__ void divmod(uint32_t n, uint32_t& q, uint32_t& r) const {
        q = div(n);
        r = n - q * d;
    }
};
