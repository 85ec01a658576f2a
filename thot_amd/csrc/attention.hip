// Scaled dot-product attention forward and backward (flash-style, MFMA).
//
// Replaces ScaledDotProductKernelImpl::forward of the reference
// (attention/details/kernel.hpp:20-96) and its autograd backward:
//   s = q·kᵀ·scale (the reference divides by sqrt(dh), kernel.hpp:33),
//   causal: s[i][j] = −inf for j > i (triu(1), kernel.hpp:86-91),
//   p = softmax_j(s), o = p·v                          (kernel.hpp:93-95)
//   dv = pᵀ·do;  dp = do·vᵀ;  ds = p∘(dp − rowsum(do∘o));
//   dq = ds·k·scale;  dk = dsᵀ·q·scale
// The reference materialises s and p ([b,h,t,s]); here one workgroup keeps a
// 64-row block in registers and streams 64-row blocks of the other operand
// through LDS, recomputing p from the saved log-sum-exp (lse = m + log l).
//
// Kernels: attn_fwd (o, lse), attn_dsum (rowsum(do∘o)), attn_dkdv (one
// workgroup per key block, loops over query blocks) and attn_dq (one per
// query block, loops over key blocks).  dq has its own pass instead of
// atomics, so every result is deterministic.
//
// Register-resident probabilities: every score tile is computed in
// "transposed" MFMA form so that its accumulator layout (lane l holds
// column l%16, rows 4·(l/16)+e) is exactly the A-operand layout the next
// MFMA needs for p or ds (row l%16, k-slots 4·(l/16)+e of each 16-wide tile).
// For bf16 (k = 32 per MFMA) the two 16-wide tiles of a 32-slice are
// interleaved as k-slots {4q..4q+3, 16+4q..16+4q+3}; the B operand of that
// MFMA is stored in LDS transposed with its keys permuted the same way, so
// it is still one 16-byte read per lane.
#include "common.hpp"
#include "lds_dma.hpp"

#include <algorithm>

namespace {

using nott::ceil_div;
using nott::launch_status;
using nott::workspace;

constexpr int kThreads = 256;     // 4 waves, 16 rows each
constexpr int BR = 64;            // rows per block (queries or keys)

template <typename T> struct AT;
template <> struct AT<float> { static constexpr int E = 4, SL = 16; };    // elems per 16 B, rows per 64-byte k-slice
template <> struct AT<bf16_t> { static constexpr int E = 8, SL = 32; };

// Tile of R rows × NCH 16-byte chunks: rows grouped by 16, chunk-major inside
// a group, slot XOR-swizzled by the chunk index (conflict-free for 16 lanes
// reading 16 rows of one chunk and for 16 lanes writing 16 chunks of a row).
__device__ __forceinline__ int toff(int row, int ch, int nch) {
    return (row >> 4) * (nch << 8) + (ch << 8) + (((row ^ ch) & 15) << 4);
}

__device__ __forceinline__ uint32_t pack_bf16(float a, float b) { return pack_bf16x2(a, b); }

template <typename T>
__device__ __forceinline__ void mma(const u32x4& a, const u32x4& b, f32x4& acc) {
    if constexpr (sizeof(T) == 2) {
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), acc,
                                                      0, 0, 0);
    } else {
        const f32x4 af = __builtin_bit_cast(f32x4, a), bf = __builtin_bit_cast(f32x4, b);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(af.x, bf.x, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(af.y, bf.y, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(af.z, bf.z, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(af.w, bf.w, acc, 0, 0, 0);
    }
}

// Register tiles v[4] (4 × 16 k-slots) as MFMA A operands, packed once per
// block.  bf16: hi[s] is the 64-byte k-slice s rounded to bf16, tiles 2s and
// 2s+1 interleaved as k-slots {4q..4q+3, 16+4q..16+4q+3}; with LO, lo[s] is
// the bf16 remainder v − hi, so the two MFMAs carry ~16 mantissa bits (used
// for ds, whose entries are differences p∘(dp − rowsum) and lose the most to
// one bf16 rounding, and for p in the dk/dv pass).  fp32 passes the float
// vectors straight to the MFMA: building a u32x4 from bit-cast floats and
// casting it back makes hipcc (ROCm 7.2) feed the first component to all four
// v_mfma_f32_16x16x4_f32 issues.
template <typename T, bool LO>
struct RegA {
    u32x4 hi[2], lo[2];
    const f32x4* v;
    __device__ __forceinline__ explicit RegA(const f32x4 (&t)[4]) : v(t) {
        if constexpr (sizeof(T) == 2) {
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                const f32x4 x = t[2 * s], y = t[2 * s + 1];
                hi[s] = u32x4{pack_bf16x2(x.x, x.y), pack_bf16x2(x.z, x.w), pack_bf16x2(y.x, y.y), pack_bf16x2(y.z, y.w)};
                if constexpr (LO) {
                    auto lo_of = [](uint32_t h, float a, float b) {
                        return pack_bf16x2(a - __builtin_bit_cast(float, h << 16),
                                           b - __builtin_bit_cast(float, h & 0xffff0000u));
                    };
                    lo[s] = u32x4{lo_of(hi[s].x, x.x, x.y), lo_of(hi[s].y, x.z, x.w), lo_of(hi[s].z, y.x, y.y),
                                  lo_of(hi[s].w, y.z, y.w)};
                }
            }
        }
    }
    // acc += A(slice s) · b
    __device__ __forceinline__ void mma(int s, const u32x4& b, f32x4& acc) const {
        if constexpr (sizeof(T) == 2) {
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, hi[s]), __builtin_bit_cast(bf16x8, b),
                                                          acc, 0, 0, 0);
            if constexpr (LO)
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, lo[s]),
                                                              __builtin_bit_cast(bf16x8, b), acc, 0, 0, 0);
        } else {
            const f32x4 af = v[s];
            const f32x4 bf = __builtin_bit_cast(f32x4, b);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(af[0], bf[0], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(af[1], bf[1], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(af[2], bf[2], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(af[3], bf[3], acc, 0, 0, 0);
        }
    }
};

// Loads 16 bytes (E elements) of row `row` starting at column c0 of a
// [rows × dh] matrix, zero outside; vec = rows are 16-byte aligned.
template <typename T>
__device__ __forceinline__ u32x4 load_chunk(const T* base, int row, int nrows, int c0, int dh, int ld, bool vec) {
    constexpr int E = AT<T>::E;
    if (row >= nrows || c0 >= dh) return u32x4{0u, 0u, 0u, 0u};
    const T* p = base + (int64_t)row * ld + c0;
    if (vec && c0 + E <= dh) return *reinterpret_cast<const u32x4*>(p);
    T v[E];
#pragma unroll
    for (int e = 0; e < E; ++e) v[e] = (c0 + e < dh) ? p[e] : T(0);
    if constexpr (E == 8) {
        return u32x4{(uint32_t)v[0] | ((uint32_t)v[1] << 16), (uint32_t)v[2] | ((uint32_t)v[3] << 16),
                     (uint32_t)v[4] | ((uint32_t)v[5] << 16), (uint32_t)v[6] | ((uint32_t)v[7] << 16)};
    } else {
        return u32x4{__builtin_bit_cast(uint32_t, v[0]), __builtin_bit_cast(uint32_t, v[1]),
                     __builtin_bit_cast(uint32_t, v[2]), __builtin_bit_cast(uint32_t, v[3])};
    }
}

// Natural tile: rows r0..r0+63 of the matrix, [row][d], NCHD chunks per row.
template <typename T, int NCHD>
__device__ __forceinline__ void fill_nat(char* tile, const T* base, int r0, int nrows, int dh, int ld, bool vec) {
    constexpr int E = AT<T>::E;
    for (int t = threadIdx.x; t < BR * NCHD; t += kThreads) {
        const int ch = t % NCHD, row = t / NCHD;
        *reinterpret_cast<u32x4*>(tile + toff(row, ch, NCHD)) = load_chunk<T>(base, r0 + row, nrows, ch * E, dh, ld, vec);
    }
}

// A natural tile staged through registers, so that the next block's loads
// are in flight while the current block is computed: load() issues them,
// store() writes the tile after the barrier.  With 16-byte aligned rows and
// dh a multiple of the chunk width, every load is unconditional (rows past
// the end re-read a valid row and are zeroed at the store).
template <typename T, int NCHD>
struct TileRegs {
    static constexpr int E = AT<T>::E;
    static constexpr int N = (BR * NCHD + kThreads - 1) / kThreads;
    u32x4 r[N];
    uint32_t ok = 0;
    __device__ __forceinline__ void load(const T* base, int r0, int nrows, int dh, int ld, bool vec) {
        if (vec && dh % E == 0) {
#pragma unroll
            for (int j = 0; j < N; ++j) {
                const int t = threadIdx.x + j * kThreads;
                const int ch = t % NCHD, row = r0 + t / NCHD;
                const bool good = t < BR * NCHD && row < nrows && ch * E < dh;
                const int rr = row < nrows ? row : nrows - 1;
                r[j] = *reinterpret_cast<const u32x4*>(base + (int64_t)rr * ld + (ch * E < dh ? ch * E : 0));
                ok = good ? (ok | (1u << j)) : (ok & ~(1u << j));
            }
        } else {
#pragma unroll
            for (int j = 0; j < N; ++j) {
                const int t = threadIdx.x + j * kThreads;
                const int ch = t % NCHD, row = t / NCHD;
                r[j] = t < BR * NCHD ? load_chunk<T>(base, r0 + row, nrows, ch * E, dh, ld, vec) : u32x4{0u, 0u, 0u, 0u};
            }
            ok = ~0u;
        }
    }
    __device__ __forceinline__ void store(char* tile) const {
#pragma unroll
        for (int j = 0; j < N; ++j) {
            const int t = threadIdx.x + j * kThreads;
            if (t < BR * NCHD)
                *reinterpret_cast<u32x4*>(tile + toff(t / NCHD, t % NCHD, NCHD)) =
                    (ok >> j) & 1u ? r[j] : u32x4{0u, 0u, 0u, 0u};
        }
    }
};

// Row (within a 64-row block) stored at k-slot position `pos` of the
// transposed tile (the bf16 interleave described above; identity for fp32).
template <typename T>
__device__ __forceinline__ int perm_row(int pos) {
    if constexpr (sizeof(T) == 2) {
        const int s = pos >> 5, w = pos & 31, q = w >> 3, j = w & 7;
        return (s << 5) + (j < 4 ? 4 * q + j : 16 + 4 * q + (j - 4));
    } else {
        return pos;
    }
}

// Transposed tile: [d][row-position] for rows r0..r0+63, NCHT = 64·sizeof(T)/16
// chunks per d-row; DP rows (padded head dim).  One task moves an E×E block:
// E rows (at E consecutive positions) × E columns, transposed in registers.
template <typename T, int DP>
__device__ __forceinline__ void fill_trans(char* tile, const T* base, int r0, int nrows, int dh, int ld, bool vec) {
    constexpr int E = AT<T>::E;
    constexpr int NCHT = BR / E;
    constexpr int TASKS = NCHT * (DP / E);
    for (int t = threadIdx.x; t < TASKS; t += kThreads) {
        const int pc = t % NCHT, dc = t / NCHT;     // position chunk, d chunk
        u32x4 in[E], out[E];
#pragma unroll
        for (int i = 0; i < E; ++i) in[i] = load_chunk<T>(base, r0 + perm_row<T>(pc * E + i), nrows, dc * E, dh, ld, vec);
        if constexpr (E == 8) {
#pragma unroll
            for (int d = 0; d < 4; ++d)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint32_t a = in[2 * e][d], b = in[2 * e + 1][d];
                    out[2 * d][e] = (a & 0xffffu) | (b << 16);
                    out[2 * d + 1][e] = (a >> 16) | (b & 0xffff0000u);
                }
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) out[j] = u32x4{in[0][j], in[1][j], in[2][j], in[3][j]};
        }
#pragma unroll
        for (int i = 0; i < E; ++i) *reinterpret_cast<u32x4*>(tile + toff(dc * E + i, pc, NCHT)) = out[i];
    }
}

// Fragment of 16 rows (r0..r0+15) of a natural/transposed tile at 64-byte k-slice s.
__device__ __forceinline__ u32x4 frag(const char* tile, int r0, int s, int nch) {
    const int lane = threadIdx.x & 63;
    return *reinterpret_cast<const u32x4*>(tile + toff(r0 + (lane & 15), 4 * s + (lane >> 4), nch));
}

typedef short v4i16 __attribute__((ext_vector_type(4)));

// bf16 B fragment for columns d0..d0+15 whose 8 k-slots are rows ra+0..3 and
// rb+0..3 of a natural [row][d] tile (ra, rb per 16-lane group), read with
// two transposing LDS reads (ds_read_b64_tr_b16: within each 16-lane group,
// result lane j, element e comes from lane 4e + j/4, element j % 4; so lane
// s reads the 4 columns d0 + 4·(s%4).. of row ra + s/4).
__device__ __forceinline__ u32x4 frag_tr(const char* tile, int nch, int ra, int rb, int d0) {
    const int s = threadIdx.x & 15;
    const int d = d0 + 4 * (s & 3);
    const int ch = d >> 3, byte = (d & 7) * 2;
    const v4i16 x = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) v4i16*)(tile + toff(ra + (s >> 2), ch, nch) + byte));
    const v4i16 y = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) v4i16*)(tile + toff(rb + (s >> 2), ch, nch) + byte));
    const u32x2 xu = __builtin_bit_cast(u32x2, x), yu = __builtin_bit_cast(u32x2, y);
    return u32x4{xu.x, xu.y, yu.x, yu.y};
}

// B operand of the second-stage MFMAs (p·v, pᵀ·do, dsᵀ·q, ds·k): columns
// d0 = 16·dt, k-slice s of the register-resident tiles.  bf16 reads the
// natural tile with transposing reads, in the key interleave of RegA
// (k-slots 0..3 = rows 32s + 4·kq + e, 4..7 = rows 32s + 16 + 4·kq + e); fp32
// reads the transposed tile.
template <typename T, int NCHD, int NCHT>
__device__ __forceinline__ u32x4 frag2(const char* nat, const char* trans, int dt, int s) {
    if constexpr (sizeof(T) == 2) {
        const int kq = (threadIdx.x & 63) >> 4;
        return frag_tr(nat, NCHD, 32 * s + 4 * kq, 32 * s + 16 + 4 * kq, dt * 16);
    } else {
        return frag(trans, dt * 16, s, NCHT);
    }
}

struct AttnParams {
    int32_t t, s, dh;
    int32_t causal;
    float scale;
    int32_t nqb, nkb;     // query / key blocks
    int32_t vec;          // rows are 16-byte aligned (vector loads)
    int32_t nh;           // heads
    // Element strides: row, batch and head of q/dq (q), k/v/dk/dv (k) and
    // o/dO (o).  Head-major [b, h, rows, dh]: row dh, head rows·dh; token-major
    // [b, rows, h, ·]: row ld, head dh.
    int32_t ldq, ldk, ldo;
    int64_t sbq, shq, sbk, shk, sbo, sho;
};

// Element offset of (batch, head) pair bh in a tensor with batch / head
// strides sb / sh.
__device__ __forceinline__ int64_t bh_off(int bh, int nh, int64_t sb, int64_t sh) {
    return (int64_t)(bh / nh) * sb + (int64_t)(bh % nh) * sh;
}

// ---------------------------------------------------------------- forward
template <typename T, int NS>
__global__ __launch_bounds__(kThreads) void attn_fwd_kernel(const T* __restrict__ q, const T* __restrict__ k,
                                                           const T* __restrict__ v, T* __restrict__ o,
                                                           float* __restrict__ lse, AttnParams p) {
    constexpr int SL = AT<T>::SL;
    constexpr int DP = NS * SL;                 // padded head dim
    constexpr int NCHD = DP * (int)sizeof(T) / 16;
    constexpr int NCHT = BR * (int)sizeof(T) / 16;
    constexpr int ND = DP / 16;                 // 16-wide d tiles
    constexpr int KS = BR / SL;                 // 64-byte k-slices per 64-row block
    constexpr int X = BR * NCHD * 16;           // bytes of one 64-row tile (natural or transposed)
    extern __shared__ __attribute__((aligned(16))) char smem[];
    char* lq = smem;
    char* lk = smem + X;
    char* lvt = smem + 2 * X;

    const int bh = blockIdx.x;
    const int qb = p.nqb - 1 - (int)blockIdx.y;      // heaviest (causal) blocks dispatched first
    const int q0 = qb * BR;
    const int64_t qoff = bh_off(bh, p.nh, p.sbq, p.shq), koff = bh_off(bh, p.nh, p.sbk, p.shk);
    const int64_t ooff = bh_off(bh, p.nh, p.sbo, p.sho);
    const int wid = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r16 = lane & 15, kq = lane >> 4;
    const int my_q = q0 + wid * 16 + r16;            // this lane's query row (score layout)
    const float sl2 = p.scale * 1.4426950408889634f;  // scale·log2(e)

    fill_nat<T, NCHD>(lq, q + qoff, q0, p.t, p.dh, p.ldq, p.vec);
    float m = -INFINITY, l = 0.f;
    f32x4 acc[ND];
#pragma unroll
    for (int i = 0; i < ND; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};

    int kb_end = p.nkb;
    if (p.causal) kb_end = min(kb_end, (q0 + BR - 1) / BR + 1);
    TileRegs<T, NCHD> rk, rv;
    rk.load(k + koff, 0, p.s, p.dh, p.ldk, p.vec);
    if constexpr (sizeof(T) == 2) rv.load(v + koff, 0, p.s, p.dh, p.ldk, p.vec);
    for (int kb = 0; kb < kb_end; ++kb) {
        const int k0 = kb * BR;
        __syncthreads();
        rk.store(lk);
        if constexpr (sizeof(T) == 2) rv.store(lvt);   // natural v
        else fill_trans<T, DP>(lvt, v + koff, k0, p.s, p.dh, p.ldk, p.vec);
        __syncthreads();
        if (kb + 1 < kb_end) {
            rk.load(k + koff, k0 + BR, p.s, p.dh, p.ldk, p.vec);
            if constexpr (sizeof(T) == 2) rv.load(v + koff, k0 + BR, p.s, p.dh, p.ldk, p.vec);
        }
        // scores in transposed form: lane holds s[my_q][k0 + 16·kt + 4·kq + e]
        f32x4 sc[4];
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
            sc[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < NS; ++s) mma<T>(frag(lk, kt * 16, s, NCHD), frag(lq, wid * 16, s, NCHD), sc[kt]);
        }
        float mx = -INFINITY;
        // masking only where the block touches the diagonal or the end
        const bool full = k0 + BR <= p.s && (!p.causal || k0 + BR - 1 <= q0);
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int key = k0 + kt * 16 + kq * 4 + e;
                const bool ok = full | ((key < p.s) & !(p.causal & (key > my_q)));   // bitwise: no per-element branches
                sc[kt][e] = ok ? sc[kt][e] * sl2 : -INFINITY;   // log2 domain
                mx = fmaxf(mx, sc[kt][e]);
            }
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float m_new = fmaxf(m, mx);
        const float alpha = (m_new == -INFINITY) ? 1.f : __builtin_amdgcn_exp2f(m - m_new);
        float rs = 0.f;
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float pe = (m_new == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(sc[kt][e] - m_new);
                sc[kt][e] = pe;
                rs += pe;
            }
        rs += __shfl_xor(rs, 16, 64);
        rs += __shfl_xor(rs, 32, 64);
        l = l * alpha + rs;
        m = m_new;
        // O rows in the accumulator are 4·kq + e: fetch their alpha.
        float al[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) al[e] = __shfl(alpha, kq * 4 + e, 64);
#pragma unroll
        for (int dt = 0; dt < ND; ++dt)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[dt][e] *= al[e];
        const RegA<T, false> pa(sc);
#pragma unroll
        for (int s = 0; s < KS; ++s)
#pragma unroll
            for (int dt = 0; dt < ND; ++dt) pa.mma(s, frag2<T, NCHD, NCHT>(lvt, lvt, dt, s), acc[dt]);
    }
    // o = acc / l (rows 4·kq + e of this wave's 16), lse = m + ln l (in natural log).
    float li[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) li[e] = __shfl(l, kq * 4 + e, 64);
#pragma unroll
    for (int dt = 0; dt < ND; ++dt) {
        const int d = dt * 16 + r16;
        if (d >= p.dh) continue;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int row = q0 + wid * 16 + kq * 4 + e;
            if (row < p.t) Io<T>::st(o + ooff, (int64_t)row * p.ldo + d, acc[dt][e] / li[e]);
        }
    }
    if (kq == 0 && my_q < p.t) lse[(int64_t)bh * p.t + my_q] = (m + log2f(l)) * 0.6931471805599453f;
}

// ------------------------------------------------------- rowsum(do ∘ o)
template <typename T>
__global__ __launch_bounds__(256) void attn_dsum_kernel(const T* __restrict__ o, const T* __restrict__ dO,
                                                        float* __restrict__ dsum, int64_t rows, AttnParams p) {
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);   // (batch·head)·t + query
    const int lane = threadIdx.x & 63;
    if (r >= rows) return;
    const int bh = (int)(r / p.t), qi = (int)(r - (int64_t)bh * p.t);
    const int64_t base = bh_off(bh, p.nh, p.sbo, p.sho) + (int64_t)qi * p.ldo;
    float s = 0.f;
    for (int d = lane; d < p.dh; d += 64) s += Io<T>::ld(o, base + d) * Io<T>::ld(dO, base + d);
    s = wave_sum(s);
    if (lane == 0) dsum[r] = s;
}

// ------------------------------------------------------------ dk, dv
template <typename T, int NS>
__global__ __launch_bounds__(kThreads) void attn_dkdv_kernel(const T* __restrict__ q, const T* __restrict__ k,
                                                            const T* __restrict__ v, const T* __restrict__ dO,
                                                            const float* __restrict__ lse,
                                                            const float* __restrict__ dsum, T* __restrict__ dk,
                                                            T* __restrict__ dv, AttnParams p) {
    constexpr int SL = AT<T>::SL;
    constexpr int DP = NS * SL;
    constexpr int NCHD = DP * (int)sizeof(T) / 16;
    constexpr int NCHT = BR * (int)sizeof(T) / 16;
    constexpr int ND = DP / 16;
    constexpr int KS = BR / SL;
    constexpr int X = BR * NCHD * 16;
    extern __shared__ __attribute__((aligned(16))) char smem[];
    char* lk = smem;
    char* lv = smem + X;
    char* lq = smem + 2 * X;
    char* ldo = smem + 3 * X;
    char* lqt = smem + 4 * X;
    char* ldot = smem + 5 * X;
    float* llse = reinterpret_cast<float*>(smem + 6 * X);
    float* lds_ = llse + BR;

    const int bh = blockIdx.x;
    const int kb = blockIdx.y;       // key blocks outermost: the longest (causal) ones are dispatched first
    const int k0 = kb * BR;
    const int64_t qoff = bh_off(bh, p.nh, p.sbq, p.shq), koff = bh_off(bh, p.nh, p.sbk, p.shk);
    const int64_t ooff = bh_off(bh, p.nh, p.sbo, p.sho);
    const int wid = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r16 = lane & 15, kq = lane >> 4;
    const int my_k = k0 + wid * 16 + r16;   // this lane's key (score layout column)
    const float sl2 = p.scale * 1.4426950408889634f;

    fill_nat<T, NCHD>(lk, k + koff, k0, p.s, p.dh, p.ldk, p.vec);
    fill_nat<T, NCHD>(lv, v + koff, k0, p.s, p.dh, p.ldk, p.vec);
    f32x4 adk[ND], adv[ND];
#pragma unroll
    for (int i = 0; i < ND; ++i) adk[i] = adv[i] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int qb_begin = p.causal ? k0 / BR : 0;
    TileRegs<T, NCHD> rq, rdo;
    // lse (log2 domain) and rowsum(p∘dp) of the next query block, one per thread < BR
    float nxt_lse = 0.f, nxt_ds = 0.f;
    auto load_stats = [&](int r0) {
        const int row = r0 + (int)threadIdx.x;
        const bool in = threadIdx.x < BR && row < p.t;
        const int64_t i = (int64_t)bh * p.t + (in ? row : 0);
        nxt_lse = in ? lse[i] * 1.4426950408889634f : 0.f;
        nxt_ds = in ? dsum[i] : 0.f;
    };
    if (qb_begin < p.nqb) {
        rq.load(q + qoff, qb_begin * BR, p.t, p.dh, p.ldq, p.vec);
        rdo.load(dO + ooff, qb_begin * BR, p.t, p.dh, p.ldo, p.vec);
        load_stats(qb_begin * BR);
    }
    for (int qb = qb_begin; qb < p.nqb; ++qb) {
        const int q0 = qb * BR;
        __syncthreads();
        rq.store(lq);
        rdo.store(ldo);
        if constexpr (sizeof(T) == 4) {
            fill_trans<T, DP>(lqt, q + qoff, q0, p.t, p.dh, p.ldq, p.vec);
            fill_trans<T, DP>(ldot, dO + ooff, q0, p.t, p.dh, p.ldo, p.vec);
        }
        if (threadIdx.x < BR) {
            llse[threadIdx.x] = nxt_lse;
            lds_[threadIdx.x] = nxt_ds;
        }
        __syncthreads();
        if (qb + 1 < p.nqb) {
            rq.load(q + qoff, q0 + BR, p.t, p.dh, p.ldq, p.vec);
            rdo.load(dO + ooff, q0 + BR, p.t, p.dh, p.ldo, p.vec);
            load_stats(q0 + BR);
        }
        const bool full = q0 + BR <= p.t && k0 + BR <= p.s && (!p.causal || k0 + BR - 1 <= q0);
        // s and dp in transposed form: lane holds [q0 + 16·qt + 4·kq + e][my_k]
        f32x4 pt[4], dpt[4];
#pragma unroll
        for (int qt = 0; qt < 4; ++qt) {
            pt[qt] = dpt[qt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                mma<T>(frag(lq, qt * 16, s, NCHD), frag(lk, wid * 16, s, NCHD), pt[qt]);
                mma<T>(frag(ldo, qt * 16, s, NCHD), frag(lv, wid * 16, s, NCHD), dpt[qt]);
            }
        }
#pragma unroll
        for (int qt = 0; qt < 4; ++qt)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int ql = qt * 16 + kq * 4 + e;
                const int qrow = q0 + ql;
                const bool ok = full | ((qrow < p.t) & (my_k < p.s) & !(p.causal & (my_k > qrow)));   // bitwise: no per-element branches
                const float pe = __builtin_amdgcn_exp2f(ok ? pt[qt][e] * sl2 - llse[ql] : -INFINITY);
                pt[qt][e] = pe;
                dpt[qt][e] = pe * (dpt[qt][e] - lds_[ql]);   // ds
            }
        const RegA<T, true> pa(pt), pds(dpt);
#pragma unroll
        for (int s = 0; s < KS; ++s)
#pragma unroll
            for (int dt = 0; dt < ND; ++dt) {
                pa.mma(s, frag2<T, NCHD, NCHT>(ldo, ldot, dt, s), adv[dt]);
                pds.mma(s, frag2<T, NCHD, NCHT>(lq, lqt, dt, s), adk[dt]);
            }
    }
#pragma unroll
    for (int dt = 0; dt < ND; ++dt) {
        const int d = dt * 16 + r16;
        if (d >= p.dh) continue;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int key = k0 + wid * 16 + kq * 4 + e;
            if (key < p.s) {
                Io<T>::st(dk + koff, (int64_t)key * p.ldk + d, adk[dt][e] * p.scale);
                Io<T>::st(dv + koff, (int64_t)key * p.ldk + d, adv[dt][e]);
            }
        }
    }
}

// ------------------------------------------------------------------- dq
// EXACT_DSUM: first sweep the key blocks once to form rowsum(p∘dp) in fp32
// (= rowsum(do∘o) in exact arithmetic), write it for the dk/dv pass and use
// it here.  The bf16 path needs this: rowsum(do∘o) taken from a bf16-rounded
// o cancels badly against dp on rows with few unmasked keys.
template <typename T, int NS, bool EXACT_DSUM>
__global__ __launch_bounds__(kThreads) void attn_dq_kernel(const T* __restrict__ q, const T* __restrict__ k,
                                                          const T* __restrict__ v, const T* __restrict__ dO,
                                                          const float* __restrict__ lse,
                                                          float* __restrict__ dsum, T* __restrict__ dq,
                                                          AttnParams p) {
    constexpr int SL = AT<T>::SL;
    constexpr int DP = NS * SL;
    constexpr int NCHD = DP * (int)sizeof(T) / 16;
    constexpr int NCHT = BR * (int)sizeof(T) / 16;
    constexpr int ND = DP / 16;
    constexpr int KS = BR / SL;
    constexpr int X = BR * NCHD * 16;
    extern __shared__ __attribute__((aligned(16))) char smem[];
    char* lq = smem;
    char* ldo = smem + X;
    char* lk = smem + 2 * X;
    char* lv = smem + 3 * X;
    char* lkt = smem + 4 * X;

    const int bh = blockIdx.x;
    const int qb = p.nqb - 1 - (int)blockIdx.y;      // heaviest (causal) blocks dispatched first
    const int q0 = qb * BR;
    const int64_t qoff = bh_off(bh, p.nh, p.sbq, p.shq), koff = bh_off(bh, p.nh, p.sbk, p.shk);
    const int64_t ooff = bh_off(bh, p.nh, p.sbo, p.sho);
    const int wid = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r16 = lane & 15, kq = lane >> 4;
    const int my_q = q0 + wid * 16 + r16;
    const float sl2 = p.scale * 1.4426950408889634f;
    const float my_lse = my_q < p.t ? lse[(int64_t)bh * p.t + my_q] * 1.4426950408889634f : 0.f;

    fill_nat<T, NCHD>(lq, q + qoff, q0, p.t, p.dh, p.ldq, p.vec);
    fill_nat<T, NCHD>(ldo, dO + ooff, q0, p.t, p.dh, p.ldo, p.vec);
    f32x4 acc[ND];
#pragma unroll
    for (int i = 0; i < ND; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};

    int kb_end = p.nkb;
    if (p.causal) kb_end = min(kb_end, (q0 + BR - 1) / BR + 1);
    float my_ds;
    TileRegs<T, NCHD> rk, rv;
    if constexpr (EXACT_DSUM) {
        float part = 0.f;
        rk.load(k + koff, 0, p.s, p.dh, p.ldk, p.vec);
        rv.load(v + koff, 0, p.s, p.dh, p.ldk, p.vec);
        for (int kb = 0; kb < kb_end; ++kb) {
            const int k0 = kb * BR;
            const bool full = q0 + BR <= p.t && k0 + BR <= p.s && (!p.causal || k0 + BR - 1 <= q0);
            __syncthreads();
            rk.store(lk);
            rv.store(lv);
            __syncthreads();
            // next block (or, after the last, block 0 for the main pass)
            const int nk0 = kb + 1 < kb_end ? k0 + BR : 0;
            rk.load(k + koff, nk0, p.s, p.dh, p.ldk, p.vec);
            rv.load(v + koff, nk0, p.s, p.dh, p.ldk, p.vec);
#pragma unroll
            for (int kt = 0; kt < 4; ++kt) {
                f32x4 sc = f32x4{0.f, 0.f, 0.f, 0.f}, dp = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int s = 0; s < NS; ++s) {
                    mma<T>(frag(lk, kt * 16, s, NCHD), frag(lq, wid * 16, s, NCHD), sc);
                    mma<T>(frag(lv, kt * 16, s, NCHD), frag(ldo, wid * 16, s, NCHD), dp);
                }
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int key = k0 + kt * 16 + kq * 4 + e;
                    const bool ok = full | ((my_q < p.t) & (key < p.s) & !(p.causal & (key > my_q)));   // bitwise: no per-element branches
                    part += __builtin_amdgcn_exp2f(ok ? sc[e] * sl2 - my_lse : -INFINITY) * (ok ? dp[e] : 0.f);
                }
            }
        }
        part += __shfl_xor(part, 16, 64);
        part += __shfl_xor(part, 32, 64);
        my_ds = part;
        if (kq == 0 && my_q < p.t) dsum[(int64_t)bh * p.t + my_q] = my_ds;
    } else {
        my_ds = my_q < p.t ? dsum[(int64_t)bh * p.t + my_q] : 0.f;
        rk.load(k + koff, 0, p.s, p.dh, p.ldk, p.vec);
        rv.load(v + koff, 0, p.s, p.dh, p.ldk, p.vec);
    }
    for (int kb = 0; kb < kb_end; ++kb) {
        const int k0 = kb * BR;
        const bool full = q0 + BR <= p.t && k0 + BR <= p.s && (!p.causal || k0 + BR - 1 <= q0);
        __syncthreads();
        rk.store(lk);
        rv.store(lv);
        if constexpr (sizeof(T) == 4) fill_trans<T, DP>(lkt, k + koff, k0, p.s, p.dh, p.ldk, p.vec);
        __syncthreads();
        if (kb + 1 < kb_end) {
            rk.load(k + koff, k0 + BR, p.s, p.dh, p.ldk, p.vec);
            rv.load(v + koff, k0 + BR, p.s, p.dh, p.ldk, p.vec);
        }
        // lane holds s / dp at [my_q][k0 + 16·kt + 4·kq + e]
        f32x4 sc[4], dp[4];
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
            sc[kt] = dp[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                mma<T>(frag(lk, kt * 16, s, NCHD), frag(lq, wid * 16, s, NCHD), sc[kt]);
                mma<T>(frag(lv, kt * 16, s, NCHD), frag(ldo, wid * 16, s, NCHD), dp[kt]);
            }
        }
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int key = k0 + kt * 16 + kq * 4 + e;
                const bool ok = full | ((my_q < p.t) & (key < p.s) & !(p.causal & (key > my_q)));   // bitwise: no per-element branches
                const float pe = __builtin_amdgcn_exp2f(ok ? sc[kt][e] * sl2 - my_lse : -INFINITY);
                dp[kt][e] = pe * (dp[kt][e] - my_ds);
            }
        const RegA<T, true> pds(dp);
#pragma unroll
        for (int s = 0; s < KS; ++s)
#pragma unroll
            for (int dt = 0; dt < ND; ++dt) pds.mma(s, frag2<T, NCHD, NCHT>(lk, lkt, dt, s), acc[dt]);
    }
#pragma unroll
    for (int dt = 0; dt < ND; ++dt) {
        const int d = dt * 16 + r16;
        if (d >= p.dh) continue;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int row = q0 + wid * 16 + kq * 4 + e;
            if (row < p.t) Io<T>::st(dq + qoff, (int64_t)row * p.ldq + d, acc[dt][e] * p.scale);
        }
    }
}

// ===========================================================================
// bf16 backward for head dim 64 on 32×32×16 MFMAs.
//
// Two deterministic passes, each streaming 64-row tiles of the other side
// through an LDS ring filled by direct-to-LDS loads:
//   attn_dq64:   one workgroup per 128 query rows (4 waves × 32); forms
//                D = rowsum(dO∘O) for its rows (written for the next pass),
//                then per 64-key block: sᵀ = k·qᵀ, dpᵀ = v·dOᵀ, dsᵀ, and
//                dq += ds·k.
//   attn_dkdv64: one workgroup per 128 keys (4 waves × 32); per 64-query
//                block: s = q·kᵀ, dp = dO·vᵀ, p, ds, dv += pᵀ·dO and
//                dk += dsᵀ·q.
// Each wave keeps its own 32 rows of the fixed side (q and dO, or k and v) as
// MFMA B operands in registers for the whole pass.
//
// Precision.  p and ds enter the second-stage MFMAs as bf16.  Where a wave's
// tile holds a probability of at least kLoTau (rows with few effective keys,
// whose few large terms dominate their sums), the bf16 remainder
// (x − bf16(x), rounded again) is multiplied as well, which carries ~16
// mantissa bits; elsewhere a rounding error of 2^-9 relative on terms that
// small stays far inside the bf16 tolerance.  D must be exact: D taken from
// the bf16-rounded o is off by dO·δo, which shifts every ds of the row.  The
// dq pass therefore uses D~ = rowsum(dO∘o_bf16) during its sweep, while it
// accumulates the exact D = Σ_j p·dp and b = Σ_j p·k, and at the end sets
// dq = scale·(Σ_j p(dp − D~)k − (D − D~)·b); the exact D is what it writes
// for the dk/dv pass.  Score tiles are computed with
// the fixed side as the B operand, so a lane's accumulator column is its own
// row of the fixed side and its 16 registers are rows 8j + 4·(l/32) + e of
// the streamed side; 8 consecutive registers are then exactly a 32×16 A
// operand whose k-slots are streamed rows {4h..4h+3, 8+4h..8+4h+3} of a
// 16-row slice, and the matching B operand is read from the streamed tile
// with two transposing LDS reads (ds_read_b64_tr_b16, 4 rows each).
// Tiles are [row][64] bf16 with 128-byte rows and 16-byte chunks swizzled by
// (row>>1)&7, as in the direct-to-LDS GEMM.
namespace a64 {

using nott::lds::barrier;
using nott::lds::dma16;
using nott::lds::dma4;
using nott::lds::lds_addr;
using nott::lds::wait_vm_lgkm0;

constexpr int NW = 4;                    // waves per workgroup, 32 fixed rows each
constexpr int FIXED = 32 * NW;           // fixed rows per workgroup
constexpr int TR = 64;                   // streamed rows per stage
constexpr int TILE = TR * 128;           // one [64][64] bf16 tile
constexpr int RING = 4;                  // stages in flight + 1
constexpr float kLoTau = 1.f / 16;       // tile max of p above which the bf16 remainder is multiplied too

__device__ __forceinline__ int toff64(int r, int c) { return r * 128 + ((c ^ ((r >> 1) & 7)) << 4); }

// Fills a [64][64] tile with rows row0.. of `base` (row stride ld, rows past
// nrows clamped to the last one): 8 blocks of 1 KB, two per wave.
__device__ __forceinline__ void fill_tile(const bf16_t* base, int row0, int nrows, int ld, char NOTT_LDS* tile,
                                          int wid, int lane) {
#pragma unroll
    for (int qq = 0; qq < 8 / NW; ++qq) {
        const int q = wid + NW * qq;
        const int r = 8 * q + (lane >> 3);
        const int c = (lane & 7) ^ ((r >> 1) & 7);
        int gr = row0 + r;
        gr = gr < nrows ? gr : nrows - 1;
        dma16(base + (int64_t)gr * ld + 8 * c, lds_addr(tile) + 1024 * q);
    }
}

// 32×16 operand of tile rows r0..r0+31, d slice s: lane l gets row r0 + l%32,
// d = 16s + 8·(l/32) + 0..7.
__device__ __forceinline__ bf16x8 frag_rows(const char NOTT_LDS* tile, int r0, int s, int lane) {
    const int r = r0 + (lane & 31);
    return __builtin_bit_cast(bf16x8,
                              *reinterpret_cast<const u32x4 NOTT_LDS*>(tile + toff64(r, 2 * s + (lane >> 5))));
}

typedef short v4i16s __attribute__((ext_vector_type(4)));

// B operand over a 16-row slice starting at tile row rs: lane l gets column
// d0 + l%32 and rows rs + 4h + 0..3, rs + 8 + 4h + 0..3 (h = l/32).
__device__ __forceinline__ bf16x8 frag_cols(const char NOTT_LDS* tile, int rs, int d0, int lane) {
    const int j = lane & 15, g = lane >> 4;
    const int col = d0 + 16 * (g & 1) + 4 * (j & 3);
    const int r1 = rs + 4 * (g >> 1) + (j >> 2);
    const int byte = (col & 7) * 2;
    const v4i16s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((v4i16s NOTT_LDS*)(tile + toff64(r1, col >> 3) + byte));
    const v4i16s hi =
        __builtin_amdgcn_ds_read_tr16_b64_v4i16((v4i16s NOTT_LDS*)(tile + toff64(r1 + 8, col >> 3) + byte));
    const v4i16s w[2] = {lo, hi};
    return __builtin_bit_cast(bf16x8, w);
}

// Registers base..base+7 of an accumulator tile as a bf16 A operand.
__device__ __forceinline__ bf16x8 pack8(const f32x16& t, int base) {
    const u32x4 w = {pack_bf16x2(t[base], t[base + 1]), pack_bf16x2(t[base + 2], t[base + 3]),
                     pack_bf16x2(t[base + 4], t[base + 5]), pack_bf16x2(t[base + 6], t[base + 7])};
    return __builtin_bit_cast(bf16x8, w);
}

// The remainder x − bf16(x) of the same 8 registers, rounded to bf16.
__device__ __forceinline__ bf16x8 pack8_lo(const f32x16& t, int base, const bf16x8& hi) {
    const u32x4 h = __builtin_bit_cast(u32x4, hi);
    auto lo2 = [&](int i, uint32_t w) {
        return pack_bf16x2(t[base + i] - __builtin_bit_cast(float, w << 16),
                           t[base + i + 1] - __builtin_bit_cast(float, w & 0xffff0000u));
    };
    const u32x4 w = {lo2(0, h.x), lo2(2, h.y), lo2(4, h.z), lo2(6, h.w)};
    return __builtin_bit_cast(bf16x8, w);
}

// Wave-wide maximum (uniform result).
__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) x = fmaxf(x, __shfl_xor(x, m, 64));
    return x;
}

__device__ __forceinline__ f32x16 mfma(const bf16x8& a, const bf16x8& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// A row's 64 values as 4 B-operand slices: lane l holds d = 16s + 8·(l/32) + 0..7.
__device__ __forceinline__ void load_fixed(const bf16_t* base, int row, int nrows, int ld, int lane, u32x4 (&r)[4]) {
    const int rr = row < nrows ? row : nrows - 1;
    const bf16_t* pr = base + (int64_t)rr * ld + 8 * (lane >> 5);
#pragma unroll
    for (int s = 0; s < 4; ++s) r[s] = *reinterpret_cast<const u32x4*>(pr + 16 * s);
}

__device__ __forceinline__ float dot_bf16x8(const u32x4& a, const u32x4& b) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        s += __builtin_bit_cast(float, a[i] << 16) * __builtin_bit_cast(float, b[i] << 16);
        s += __builtin_bit_cast(float, a[i] & 0xffff0000u) * __builtin_bit_cast(float, b[i] & 0xffff0000u);
    }
    return s;
}

__global__ __launch_bounds__(64 * NW, 2) void attn_dq64_kernel(const bf16_t* __restrict__ q,
                                                                 const bf16_t* __restrict__ k,
                                                                 const bf16_t* __restrict__ v,
                                                                 const bf16_t* __restrict__ o,
                                                                 const bf16_t* __restrict__ dO,
                                                                 const float* __restrict__ lse,
                                                                 float* __restrict__ dsum, float* __restrict__ lse2,
                                                                 bf16_t* __restrict__ dq, AttnParams p) {
    constexpr int STAGE = 2 * TILE;
    extern __shared__ __attribute__((aligned(1024))) char smem_raw[];
    char NOTT_LDS* smem = (char NOTT_LDS*)smem_raw;
    const int bh = blockIdx.x;
    const int nqb = (p.t + FIXED - 1) / FIXED;
    const int q0 = (nqb - 1 - (int)blockIdx.y) * FIXED;   // heaviest (causal) blocks first
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int h = lane >> 5;
    const int qw0 = q0 + 32 * wid;
    const int my_q = qw0 + (lane & 31);
    const int64_t qoff = bh_off(bh, p.nh, p.sbq, p.shq), koff = bh_off(bh, p.nh, p.sbk, p.shk);
    const int64_t ooff = bh_off(bh, p.nh, p.sbo, p.sho);
    const float sl2 = p.scale * 1.4426950408889634f;

    u32x4 qr[4], dr[4];
    load_fixed(q + qoff, my_q, p.t, p.ldq, lane, qr);
    load_fixed(dO + ooff, my_q, p.t, p.ldo, lane, dr);
    float my_d;
    {
        u32x4 orr[4];
        load_fixed(o + ooff, my_q, p.t, p.ldo, lane, orr);
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) s += dot_bf16x8(dr[i], orr[i]);
        my_d = s + __shfl_xor(s, 32, 64);
    }
    const bool q_in = my_q < p.t;
    const float my_lse2 = lse[(int64_t)bh * p.t + (q_in ? my_q : p.t - 1)] * 1.4426950408889634f;

    int nk = p.nkb;   // 64-key blocks
    if (p.causal) nk = min(nk, (q0 + FIXED - 1) / TR + 1);
    auto issue = [&](int i, int slot) {
        char NOTT_LDS* st = smem + slot * STAGE;
        fill_tile(k + koff, i * TR, p.s, p.ldk, st, wid, lane);
        fill_tile(v + koff, i * TR, p.s, p.ldk, st + TILE, wid, lane);
    };
#pragma unroll
    for (int i = 0; i < RING - 1; ++i)
        if (i < nk) issue(i, i);

    f32x16 adq[2], abv[2];
#pragma unroll
    for (int f = 0; f < 2; ++f)
#pragma unroll
        for (int e = 0; e < 16; ++e) adq[f][e] = abv[f][e] = 0.f;
    float d_exact = 0.f;   // Σ p·dp over this lane's keys (its half of the row)
    int slot = 0, next = RING - 1;
    for (int i = 0; i < nk; ++i) {
        if (i + RING - 2 < nk) wait_vm_lgkm0<(RING - 2) * 2 * (8 / NW)>();
        else wait_vm_lgkm0<0>();
        barrier();
        if (i + RING - 1 < nk) issue(i + RING - 1, next);
        const char NOTT_LDS* tk = smem + slot * STAGE;
        const char NOTT_LDS* tv = tk + TILE;
        slot = slot + 1 == RING ? 0 : slot + 1;
        next = next + 1 == RING ? 0 : next + 1;
        const int k0 = i * TR;
        if ((p.causal && k0 > qw0 + 31) || qw0 >= p.t) continue;   // every key of the block masked for this wave
        f32x16 st[2], dpt[2];
#pragma unroll
        for (int f = 0; f < 2; ++f) {
#pragma unroll
            for (int e = 0; e < 16; ++e) st[f][e] = dpt[f][e] = 0.f;
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                st[f] = mfma(frag_rows(tk, 32 * f, s, lane), __builtin_bit_cast(bf16x8, qr[s]), st[f]);
                dpt[f] = mfma(frag_rows(tv, 32 * f, s, lane), __builtin_bit_cast(bf16x8, dr[s]), dpt[f]);
            }
        }
        // exponent arguments (log2 domain) in place
#pragma unroll
        for (int f = 0; f < 2; ++f)
#pragma unroll
            for (int r = 0; r < 16; ++r) st[f][r] = fmaf(st[f][r], sl2, -my_lse2);
        // Masking only on blocks that touch the diagonal or the end (a
        // wave-uniform test).  Element (f, r) is key k0 + 4h + c with
        // c = 32f + 8(r/4) + r%4 (0..59), kept iff c < rel: one compare against
        // a constant, no per-element branches.
        if (!(qw0 + 32 <= p.t && k0 + TR <= p.s && (!p.causal || k0 + TR - 1 <= qw0))) {
            const int rel = q_in ? min(p.s, p.causal ? my_q + 1 : p.s) - k0 - 4 * h : -1;
#pragma unroll
            for (int f = 0; f < 2; ++f)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (!(32 * f + 8 * (r >> 2) + (r & 3) < rel)) st[f][r] = -INFINITY;
        }
        float pmax = 0.f;
#pragma unroll
        for (int f = 0; f < 2; ++f)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float pe = __builtin_amdgcn_exp2f(st[f][r]);
                d_exact += pe * dpt[f][r];
                pmax = fmaxf(pmax, pe);
                st[f][r] = pe;
                dpt[f][r] = pe * (dpt[f][r] - my_d);
            }
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const bf16x8 a = pack8(dpt[s >> 1], 8 * (s & 1));
            const bf16x8 pa = pack8(st[s >> 1], 8 * (s & 1));
#pragma unroll
            for (int df = 0; df < 2; ++df) {
                const bf16x8 b = frag_cols(tk, 16 * s, 32 * df, lane);
                adq[df] = mfma(a, b, adq[df]);
                abv[df] = mfma(pa, b, abv[df]);
            }
        }
        if (wave_max(pmax) >= kLoTau) {
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const bf16x8 al = pack8_lo(dpt[s >> 1], 8 * (s & 1), pack8(dpt[s >> 1], 8 * (s & 1)));
#pragma unroll
                for (int df = 0; df < 2; ++df) adq[df] = mfma(al, frag_cols(tk, 16 * s, 32 * df, lane), adq[df]);
            }
        }
    }
    // Exact D of this lane's row (lanes l and l^32 hold the two key halves);
    // the dk/dv pass reads it.
    d_exact += __shfl_xor(d_exact, 32, 64);
    if (h == 0 && q_in) {
        dsum[(int64_t)bh * p.t + my_q] = d_exact;
        lse2[(int64_t)bh * p.t + my_q] = my_lse2;
    }
    const float corr = d_exact - my_d;
    // adq, abv: lane holds column d = 32·df + l%32, rows 8j + 4h + e of this
    // wave's 32 (row r's correction lives in lane r's column).
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int rl = 8 * (r >> 2) + 4 * h + (r & 3);
        const float c = __shfl(corr, rl, 64);
        const int row = qw0 + rl;
#pragma unroll
        for (int df = 0; df < 2; ++df)
            if (row < p.t)
                dq[qoff + (int64_t)row * p.ldq + 32 * df + (lane & 31)] =
                    f32_to_bf16((adq[df][r] - c * abv[df][r]) * p.scale);
    }
}

__global__ __launch_bounds__(64 * NW, 2) void attn_dkdv64_kernel(const bf16_t* __restrict__ q,
                                                                   const bf16_t* __restrict__ k,
                                                                   const bf16_t* __restrict__ v,
                                                                   const bf16_t* __restrict__ dO,
                                                                   const float* __restrict__ lse2,
                                                                   const float* __restrict__ dsum,
                                                                   bf16_t* __restrict__ dk, bf16_t* __restrict__ dv,
                                                                   AttnParams p) {
    constexpr int STAGE = 2 * TILE + 2 * TR * 4;   // q tile, dO tile, lse and D of its rows
    extern __shared__ __attribute__((aligned(1024))) char smem_raw[];
    char NOTT_LDS* smem = (char NOTT_LDS*)smem_raw;
    const int bh = blockIdx.x;
    const int k0 = (int)blockIdx.y * FIXED;   // causal: the longest (first) key blocks are dispatched first
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int h = lane >> 5;
    const int kw0 = k0 + 32 * wid;
    const int my_k = kw0 + (lane & 31);
    const int64_t qoff = bh_off(bh, p.nh, p.sbq, p.shq), koff = bh_off(bh, p.nh, p.sbk, p.shk);
    const int64_t ooff = bh_off(bh, p.nh, p.sbo, p.sho);
    const float sl2 = p.scale * 1.4426950408889634f;
    const float* lse_bh = lse2 + (int64_t)bh * p.t;   // lse·log2(e), written by the dq pass
    const float* d_bh = dsum + (int64_t)bh * p.t;

    u32x4 kr[4], vr[4];
    load_fixed(k + koff, my_k, p.s, p.ldk, lane, kr);
    load_fixed(v + koff, my_k, p.s, p.ldk, lane, vr);

    const int qb0 = p.causal ? k0 / TR : 0;
    const int nq = p.nqb - qb0;   // 64-query blocks
    auto issue = [&](int i, int slot) {
        char NOTT_LDS* st = smem + slot * STAGE;
        const int q0 = (qb0 + i) * TR;
        fill_tile(q + qoff, q0, p.t, p.ldq, st, wid, lane);
        fill_tile(dO + ooff, q0, p.t, p.ldo, st + TILE, wid, lane);
        if (wid < 2) {
            const int row = q0 + lane < p.t ? q0 + lane : p.t - 1;
            dma4((wid == 0 ? lse_bh : d_bh) + row, lds_addr(st + 2 * TILE) + 256 * wid);
        }
    };
#pragma unroll
    for (int i = 0; i < RING - 1; ++i)
        if (i < nq) issue(i, i);

    f32x16 adk[2], adv[2];
#pragma unroll
    for (int f = 0; f < 2; ++f)
#pragma unroll
        for (int e = 0; e < 16; ++e) adk[f][e] = adv[f][e] = 0.f;
    int slot = 0, next = RING - 1;
    for (int i = 0; i < nq; ++i) {
        // Waves 0 and 1 issue one more load per stage than 2 and 3; the count
        // of the latter is a safe bound for both.
        if (i + RING - 2 < nq) wait_vm_lgkm0<(RING - 2) * 2 * (8 / NW)>();
        else wait_vm_lgkm0<0>();
        barrier();
        if (i + RING - 1 < nq) issue(i + RING - 1, next);
        const char NOTT_LDS* tq = smem + slot * STAGE;
        const char NOTT_LDS* tdo = tq + TILE;
        const float NOTT_LDS* slse = reinterpret_cast<const float NOTT_LDS*>(tq + 2 * TILE);
        const float NOTT_LDS* sd = slse + TR;
        slot = slot + 1 == RING ? 0 : slot + 1;
        next = next + 1 == RING ? 0 : next + 1;
        const int q0 = (qb0 + i) * TR;
        if ((p.causal && kw0 > q0 + TR - 1) || kw0 >= p.s) continue;   // every query of the block masked
        f32x16 sc[2], dp[2];
#pragma unroll
        for (int f = 0; f < 2; ++f) {
#pragma unroll
            for (int e = 0; e < 16; ++e) sc[f][e] = dp[f][e] = 0.f;
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                sc[f] = mfma(frag_rows(tq, 32 * f, s, lane), __builtin_bit_cast(bf16x8, kr[s]), sc[f]);
                dp[f] = mfma(frag_rows(tdo, 32 * f, s, lane), __builtin_bit_cast(bf16x8, vr[s]), dp[f]);
            }
        }
        // exponent arguments (log2 domain; the ring holds lse·log2(e)) in place
#pragma unroll
        for (int f = 0; f < 2; ++f)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const f32x4 l4 = *reinterpret_cast<const f32x4 NOTT_LDS*>(slse + 32 * f + 8 * j + 4 * h);
#pragma unroll
                for (int e = 0; e < 4; ++e) sc[f][4 * j + e] = fmaf(sc[f][4 * j + e], sl2, -l4[e]);
            }
        // Masking only on blocks that touch the diagonal or the end (a
        // wave-uniform test).  Element (f, 4j + e) is query q0 + 4h + c with
        // c = 32f + 8j + e (0..59), kept iff lo <= c < hi.
        if (!(q0 + TR <= p.t && kw0 + 32 <= p.s && (!p.causal || kw0 + 31 <= q0))) {
            const int hi = my_k < p.s ? p.t - q0 - 4 * h : -1;
            const int lo = p.causal ? my_k - q0 - 4 * h : 0;
#pragma unroll
            for (int f = 0; f < 2; ++f)
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int c = 32 * f + 8 * j + e;
                        if (!((c >= lo) & (c < hi))) sc[f][4 * j + e] = -INFINITY;
                    }
        }
        float pmax = 0.f;
#pragma unroll
        for (int f = 0; f < 2; ++f)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const f32x4 d4 = *reinterpret_cast<const f32x4 NOTT_LDS*>(sd + 32 * f + 8 * j + 4 * h);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int r = 4 * j + e;
                    const float pe = __builtin_amdgcn_exp2f(sc[f][r]);
                    pmax = fmaxf(pmax, pe);
                    sc[f][r] = pe;
                    dp[f][r] = pe * (dp[f][r] - d4[e]);
                }
            }
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const bf16x8 pa = pack8(sc[s >> 1], 8 * (s & 1));
            const bf16x8 da = pack8(dp[s >> 1], 8 * (s & 1));
#pragma unroll
            for (int df = 0; df < 2; ++df) {
                adv[df] = mfma(pa, frag_cols(tdo, 16 * s, 32 * df, lane), adv[df]);
                adk[df] = mfma(da, frag_cols(tq, 16 * s, 32 * df, lane), adk[df]);
            }
        }
        if (wave_max(pmax) >= kLoTau) {
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const bf16x8 pl = pack8_lo(sc[s >> 1], 8 * (s & 1), pack8(sc[s >> 1], 8 * (s & 1)));
                const bf16x8 dl = pack8_lo(dp[s >> 1], 8 * (s & 1), pack8(dp[s >> 1], 8 * (s & 1)));
#pragma unroll
                for (int df = 0; df < 2; ++df) {
                    adv[df] = mfma(pl, frag_cols(tdo, 16 * s, 32 * df, lane), adv[df]);
                    adk[df] = mfma(dl, frag_cols(tq, 16 * s, 32 * df, lane), adk[df]);
                }
            }
        }
    }
#pragma unroll
    for (int df = 0; df < 2; ++df)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int key = kw0 + 8 * (r >> 2) + 4 * h + (r & 3);
            if (key < p.s) {
                const int64_t i = koff + (int64_t)key * p.ldk + 32 * df + (lane & 31);
                dk[i] = f32_to_bf16(adk[df][r] * p.scale);
                dv[i] = f32_to_bf16(adv[df][r]);
            }
        }
}

// Whether the head-dim-64 kernels take this problem: bf16, dh = 64, 16-byte
// aligned rows (the fills move 16-byte chunks).
bool applies(const nott_attn_desc* d, const AttnParams& p, int elem) { return elem == 2 && d->dh == 64 && p.vec; }

int bwd(nott_ctx ctx, const nott_attn_desc* d, const AttnParams& p, const void* q, const void* k, const void* v,
        const void* o, const void* dO, const float* lse, void* dq, void* dk, void* dv) {
    const int64_t rows = d->b * d->h * d->t;
    // dsum (the exact rowsum(P∘dP)) and lse2 (lse·log2 e), both [b, h, t],
    // handed from the dq pass to the dk/dv pass
    float* dsum = static_cast<float*>(workspace(ctx, 2 * sizeof(float) * (size_t)std::max<int64_t>(rows, 1)));
    if (!dsum) return NOTT_ERR_ALLOC;
    float* lse2 = dsum + std::max<int64_t>(rows, 1);
    const unsigned bh = (unsigned)(d->b * d->h);
    const size_t lds_q = RING * 2 * TILE, lds_kv = RING * (2 * TILE + 2 * TR * 4);
    static bool attr = false;
    if (!attr) {
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_dq64_kernel),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_q);
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_dkdv64_kernel),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_kv);
        attr = true;
    }
    const auto* qb = static_cast<const bf16_t*>(q);
    const auto* kb = static_cast<const bf16_t*>(k);
    const auto* vb = static_cast<const bf16_t*>(v);
    const auto* dob = static_cast<const bf16_t*>(dO);
    hipLaunchKernelGGL(attn_dq64_kernel, dim3(bh, (unsigned)ceil_div(d->t, FIXED)), dim3(64 * NW), lds_q, ctx->stream,
                       qb, kb, vb, static_cast<const bf16_t*>(o), dob, lse, dsum, lse2, static_cast<bf16_t*>(dq), p);
    hipLaunchKernelGGL(attn_dkdv64_kernel, dim3(bh, (unsigned)ceil_div(d->s, FIXED)), dim3(64 * NW), lds_kv,
                       ctx->stream, qb, kb, vb, dob, lse2, dsum, static_cast<bf16_t*>(dk), static_cast<bf16_t*>(dv), p);
    return launch_status(ctx, "attention_bwd");
}

}  // namespace a64

int check(nott_ctx ctx, const nott_attn_desc* d, AttnParams* p, int elem) {
    NOTT_REQUIRE(ctx, d != nullptr, "attention: null descriptor");
    NOTT_REQUIRE(ctx, d->b >= 0 && d->h >= 0 && d->t >= 0 && d->s >= 0 && d->dh > 0, "attention: bad shape");
    // LDS holds six 64-row tiles of the padded head dim in the dk/dv pass.
    NOTT_REQUIRE(ctx, d->dh <= (elem == 2 ? 128 : 64), "attention: head dim above 128 (bf16) / 64 (fp32) is not supported");
    // grid: x = (batch, head) pairs, y = 64-row blocks
    NOTT_REQUIRE(ctx, d->b * d->h <= 0x7fffffff, "attention: too many (batch, head) pairs");
    NOTT_REQUIRE(ctx, ceil_div(d->t, BR) <= 65535 && ceil_div(d->s, BR) <= 65535, "attention: sequence too long");
    NOTT_REQUIRE(ctx, d->t * d->dh < (int64_t(1) << 31) && d->s * d->dh < (int64_t(1) << 31),
                 "attention: sequence too long");
    NOTT_REQUIRE(ctx, !d->causal || d->s > 0, "attention: causal needs keys");
    NOTT_REQUIRE(ctx, d->layout == NOTT_ATTN_HEAD_MAJOR || d->layout == NOTT_ATTN_TOKEN_MAJOR, "attention: bad layout");
    p->t = (int32_t)d->t; p->s = (int32_t)d->s; p->dh = (int32_t)d->dh;
    p->causal = d->causal != 0;
    p->scale = (float)d->scale;
    p->nqb = (int32_t)ceil_div(d->t, BR);
    p->nkb = (int32_t)ceil_div(d->s, BR);
    p->nh = (int32_t)std::max<int64_t>(d->h, 1);
    if (d->layout == NOTT_ATTN_HEAD_MAJOR) {
        p->ldq = p->ldk = p->ldo = p->dh;
        p->shq = p->sho = d->t * d->dh;
        p->sbq = p->sbo = d->h * d->t * d->dh;
        p->shk = d->s * d->dh;
        p->sbk = d->h * d->s * d->dh;
    } else {
        const int64_t ldqkv = d->ld_qkv ? d->ld_qkv : d->h * d->dh, ldo = d->ld_o ? d->ld_o : d->h * d->dh;
        NOTT_REQUIRE(ctx, ldqkv >= d->h * d->dh && ldo >= d->h * d->dh, "attention: row stride below h·dh");
        NOTT_REQUIRE(ctx, std::max(d->t, d->s) * std::max(ldqkv, ldo) < (int64_t(1) << 31),
                     "attention: sequence too long");
        p->ldq = p->ldk = (int32_t)ldqkv;
        p->ldo = (int32_t)ldo;
        p->shq = p->shk = p->sho = d->dh;
        p->sbq = d->t * ldqkv;
        p->sbk = d->s * ldqkv;
        p->sbo = d->t * ldo;
    }
    p->vec = ((d->dh * elem) % 16) == 0 && ((int64_t)p->ldq * elem) % 16 == 0 && ((int64_t)p->ldo * elem) % 16 == 0;
    return NOTT_OK;
}

// Zeroes `rows` rows of `cols` elements at row stride ld (strided outputs of
// the empty cases).
__global__ __launch_bounds__(256) void zero_rows_kernel(uint16_t* __restrict__ p16, float* __restrict__ p32,
                                                        int64_t rows, int64_t cols, int64_t ld) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= rows * cols) return;
    const int64_t r = i / cols, c = i - r * cols;
    if (p16) p16[r * ld + c] = 0;
    else p32[r * ld + c] = 0.f;
}

// Zero the (b, h, rows, dh) view of a q-side (kq = 0) or k-side (kq = 1)
// tensor in the descriptor's layout.
int zero_view(nott_ctx ctx, const nott_attn_desc* d, const AttnParams& p, int elem, int64_t rows, bool kside,
              void* dst) {
    if (d->b * d->h * rows == 0) return NOTT_OK;
    NOTT_REQUIRE(ctx, dst != nullptr, "nott_attention_bwd: null buffer");
    // head-major: b·h·rows contiguous rows of dh; token-major: b·rows rows of h·dh at stride ld.
    const bool hm = d->layout == NOTT_ATTN_HEAD_MAJOR;
    const int64_t nrows = hm ? d->b * d->h * rows : d->b * rows;
    const int64_t cols = hm ? d->dh : d->h * d->dh;
    const int64_t ld = hm ? d->dh : (kside ? p.ldk : p.ldq);
    hipLaunchKernelGGL(zero_rows_kernel, dim3((unsigned)ceil_div(nrows * cols, 256)), dim3(256), 0, ctx->stream,
                       elem == 2 ? static_cast<uint16_t*>(dst) : nullptr, elem == 2 ? nullptr : static_cast<float*>(dst),
                       nrows, cols, ld);
    return launch_status(ctx, "attention zero");
}

template <typename T>
int slices_for(int dh) {
    const int sl = AT<T>::SL;
    int ns = (dh + sl - 1) / sl;
    int r = 1;
    while (r < ns) r <<= 1;
    return r;
}

template <typename T, int NS>
constexpr size_t tile_bytes() { return (size_t)BR * NS * AT<T>::SL * sizeof(T); }

template <typename T, int NS>
int fwd_ns(nott_ctx ctx, const nott_attn_desc* d, const AttnParams& p, const void* q, const void* k, const void* v,
           void* o, float* lse) {
    const size_t lds = 3 * tile_bytes<T, NS>();
    if (lds > 64 * 1024)
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_fwd_kernel<T, NS>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    hipLaunchKernelGGL((attn_fwd_kernel<T, NS>), dim3((unsigned)(d->b * d->h), (unsigned)p.nqb), dim3(kThreads), lds,
                       ctx->stream, static_cast<const T*>(q), static_cast<const T*>(k), static_cast<const T*>(v),
                       static_cast<T*>(o), lse, p);
    return launch_status(ctx, "attention_fwd");
}

template <typename T, int NS>
int bwd_ns(nott_ctx ctx, const nott_attn_desc* d, const AttnParams& p, const void* q, const void* k, const void* v,
           const void* o, const void* dO, const float* lse, void* dq, void* dk, void* dv) {
    const int64_t rows = d->b * d->h * d->t;
    float* dsum = static_cast<float*>(workspace(ctx, sizeof(float) * (size_t)std::max<int64_t>(rows, 1)));
    if (!dsum) return NOTT_ERR_ALLOC;
    constexpr bool EXACT = sizeof(T) == 2;
    const unsigned bh = (unsigned)(d->b * d->h);
    const size_t lds_kv = 6 * tile_bytes<T, NS>() + 2 * BR * sizeof(float);
    const size_t lds_q = 5 * tile_bytes<T, NS>();
    if (lds_kv > 64 * 1024)
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_dkdv_kernel<T, NS>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_kv);
    if (lds_q > 64 * 1024)
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_dq_kernel<T, NS, EXACT>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_q);
    // fp32: rowsum(do∘o) from o; bf16: the dq pass forms it exactly and runs first.
    if (!EXACT)
        hipLaunchKernelGGL(attn_dsum_kernel<T>, dim3((unsigned)ceil_div(rows, 4)), dim3(256), 0, ctx->stream,
                           static_cast<const T*>(o), static_cast<const T*>(dO), dsum, rows, p);
    hipLaunchKernelGGL((attn_dq_kernel<T, NS, EXACT>), dim3(bh, (unsigned)p.nqb), dim3(kThreads), lds_q, ctx->stream,
                       static_cast<const T*>(q), static_cast<const T*>(k), static_cast<const T*>(v),
                       static_cast<const T*>(dO), lse, dsum, static_cast<T*>(dq), p);
    hipLaunchKernelGGL((attn_dkdv_kernel<T, NS>), dim3(bh, (unsigned)p.nkb), dim3(kThreads), lds_kv, ctx->stream,
                       static_cast<const T*>(q), static_cast<const T*>(k), static_cast<const T*>(v),
                       static_cast<const T*>(dO), lse, dsum, static_cast<T*>(dk), static_cast<T*>(dv), p);
    return launch_status(ctx, "attention_bwd");
}

template <typename T>
int fwd(nott_ctx ctx, const nott_attn_desc* d, const AttnParams& p, const void* q, const void* k, const void* v,
        void* o, float* lse) {
    switch (slices_for<T>((int)d->dh)) {
        case 1: return fwd_ns<T, 1>(ctx, d, p, q, k, v, o, lse);
        case 2: return fwd_ns<T, 2>(ctx, d, p, q, k, v, o, lse);
        default: return fwd_ns<T, 4>(ctx, d, p, q, k, v, o, lse);
    }
}

template <typename T>
int bwd(nott_ctx ctx, const nott_attn_desc* d, const AttnParams& p, const void* q, const void* k, const void* v,
        const void* o, const void* dO, const float* lse, void* dq, void* dk, void* dv) {
    switch (slices_for<T>((int)d->dh)) {
        case 1: return bwd_ns<T, 1>(ctx, d, p, q, k, v, o, dO, lse, dq, dk, dv);
        case 2: return bwd_ns<T, 2>(ctx, d, p, q, k, v, o, dO, lse, dq, dk, dv);
        default: return bwd_ns<T, 4>(ctx, d, p, q, k, v, o, dO, lse, dq, dk, dv);
    }
}

bool aligned16(const void* a) { return ((uintptr_t)a % 16) == 0; }

}  // namespace

extern "C" int nott_attention_fwd(nott_ctx ctx, const nott_attn_desc* d, nott_dtype dtype, const void* q,
                                  const void* k, const void* v, void* o, float* lse) {
    NOTT_CHECK_CTX(ctx);
    NOTT_REQUIRE(ctx, nott::valid_dtype(dtype), "nott_attention_fwd: bad dtype");
    AttnParams p;
    const int st = check(ctx, d, &p, (int)nott::dtype_size(dtype));
    if (st != NOTT_OK) return st;
    if (d->b * d->h * d->t == 0) return NOTT_OK;
    NOTT_REQUIRE(ctx, q && k && v && o && lse, "nott_attention_fwd: null buffer");
    if (!(aligned16(q) && aligned16(k) && aligned16(v))) p.vec = 0;
    nott::DeviceScope scope(ctx->device);
    return dtype == NOTT_F32 ? fwd<float>(ctx, d, p, q, k, v, o, lse) : fwd<bf16_t>(ctx, d, p, q, k, v, o, lse);
}

extern "C" int nott_attention_bwd(nott_ctx ctx, const nott_attn_desc* d, nott_dtype dtype, const void* q,
                                  const void* k, const void* v, const void* o, const void* dO, const float* lse,
                                  void* dq, void* dk, void* dv) {
    NOTT_CHECK_CTX(ctx);
    NOTT_REQUIRE(ctx, nott::valid_dtype(dtype), "nott_attention_bwd: bad dtype");
    AttnParams p;
    const int st = check(ctx, d, &p, (int)nott::dtype_size(dtype));
    if (st != NOTT_OK) return st;
    if (d->b * d->h == 0) return NOTT_OK;
    if (d->t == 0 || d->s == 0) {
        // No queries: dk = dv = 0 (sums over no rows); no keys: dq = 0.
        nott::DeviceScope scope(ctx->device);
        const int elem = (int)nott::dtype_size(dtype);
        if (d->t == 0) {
            const int st1 = zero_view(ctx, d, p, elem, d->s, true, dk);
            return st1 != NOTT_OK ? st1 : zero_view(ctx, d, p, elem, d->s, true, dv);
        }
        return zero_view(ctx, d, p, elem, d->t, false, dq);
    }
    NOTT_REQUIRE(ctx, q && k && v && o && dO && lse && dq && dk && dv, "nott_attention_bwd: null buffer");
    if (!(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(dO) && aligned16(o))) p.vec = 0;
    nott::DeviceScope scope(ctx->device);
    if (a64::applies(d, p, (int)nott::dtype_size(dtype))) return a64::bwd(ctx, d, p, q, k, v, o, dO, lse, dq, dk, dv);
    return dtype == NOTT_F32 ? bwd<float>(ctx, d, p, q, k, v, o, dO, lse, dq, dk, dv)
                             : bwd<bf16_t>(ctx, d, p, q, k, v, o, dO, lse, dq, dk, dv);
}
