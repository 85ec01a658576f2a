// Building blocks shared by the LDS-staged convolution kernels (conv3x3.hip,
// conv_tap.hip): tile constants, the 16-row-grouped LDS row layout, channel
// chunks, the register transpose of the NCHW fill and the MFMA step on one
// 16-byte operand pair.
#pragma once

#include "conv_fast.hpp"

namespace nott {
namespace conv_fast {

constexpr int kThreads = 256;
constexpr int kTilePix = 256;       // pixels per workgroup (4 waves × 64)
constexpr int kTileCo = 64;         // output channels per workgroup
constexpr int kRowB = 64;           // bytes per LDS row (one channel chunk)

template <typename T> struct Chunk;
template <> struct Chunk<float> { static constexpr int CC = 16, SUB = 4; };   // channels per chunk / per 16 B
template <> struct Chunk<bf16_t> { static constexpr int CC = 32, SUB = 8; };

// LDS layout of [row][4 × 16-byte sub-chunks] tiles: rows are grouped by 16
// and stored sub-chunk-major inside a group, so the 16 lanes of a quarter-wave
// that read 16 consecutive rows at the same sub-chunk touch 16 distinct
// 16-byte slots of 256-byte blocks (4 LDS cycles per ds_read_b128, measured
// with SQ_LDS_BANK_CONFLICT = 0), whatever row the run starts at.
__device__ __forceinline__ int lds_off(int row, int sub) { return ((row >> 4) << 10) + (sub << 8) + ((row & 15) << 4); }

template <typename T>
__device__ __forceinline__ u32x4 pack_sub(const T (&v)[Chunk<T>::SUB]);
template <>
__device__ __forceinline__ u32x4 pack_sub<float>(const float (&v)[4]) {
    return u32x4{__builtin_bit_cast(uint32_t, v[0]), __builtin_bit_cast(uint32_t, v[1]),
                 __builtin_bit_cast(uint32_t, v[2]), __builtin_bit_cast(uint32_t, v[3])};
}
template <>
__device__ __forceinline__ u32x4 pack_sub<bf16_t>(const bf16_t (&v)[8]) {
    return u32x4{(uint32_t)v[0] | ((uint32_t)v[1] << 16), (uint32_t)v[2] | ((uint32_t)v[3] << 16),
                 (uint32_t)v[4] | ((uint32_t)v[5] << 16), (uint32_t)v[6] | ((uint32_t)v[7] << 16)};
}

template <typename T>
__device__ __forceinline__ void mfma_chunk(const u32x4& a, const u32x4& b, f32x4& acc) {
    if constexpr (sizeof(T) == 2) {
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                      acc, 0, 0, 0);
    } else {
        const f32x4 af = __builtin_bit_cast(f32x4, a), bf = __builtin_bit_cast(f32x4, b);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(af.x, bf.x, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(af.y, bf.y, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(af.z, bf.z, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(af.w, bf.w, acc, 0, 0, 0);
    }
}

// Channel-chunk split count for `blocks` output tiles on `slots` resident
// workgroup slots.  With S splits a workgroup runs ceil(nchunks / S) chunks
// and the grid takes ceil(S·blocks / slots) rounds, so the kernel time is
// about rounds · (chunks + per-tile overhead), plus the split reduce when
// S > 1 (both in units of one chunk's tap loop; measured: a tile's prologue
// and epilogue cost about two bf16 chunks or half an fp32 one, the reduce
// 2.5 bf16 chunks or three quarters of an fp32 one: a 49-tile fp32 forward
// of two chunks, 32 -> 64 channels at 14×14, ran 28 µs whole against 16 µs
// per single-chunk workgroup plus a 5 µs reduce).  The smallest S of least
// cost wins: a grid of a few more workgroups than slots would run a whole
// second round.
inline int32_t pick_chunk_splits(int64_t blocks, int32_t nchunks, int64_t slots, size_t elem) {
    const double overhead = elem == 2 ? 2.0 : 0.5, reduce = elem == 2 ? 2.5 : 0.75;
    double best = 0.0;
    int32_t pick = 1;
    for (int32_t s = 1; s <= std::min(nchunks, 8); ++s) {
        const int64_t per = ceil_div(nchunks, s);
        if (ceil_div(nchunks, per) != s) continue;      // same chunks per split as a smaller count
        const double t = (double)ceil_div(s * blocks, slots) * ((double)per + overhead) + (s > 1 ? reduce : 0.0);
        if (s == 1 || t < best) {
            best = t;
            pick = s;
        }
    }
    return pick;
}

// Pieces per tile for the last `blocks % slots` tiles of a grid of more than
// one round: whole, they would run a last round of their own (mostly one
// workgroup per CU, taken as 0.7 of a full round's time); split over their
// channel chunks they fill the slots that the last whole tiles free, for
// the cost of the split reduce.  1 = no tail split.
inline int32_t pick_tail_splits(int64_t blocks, int32_t nchunks, int64_t slots, size_t elem) {
    const int64_t rem = blocks % slots;
    if (blocks <= slots || rem == 0 || nchunks < 2) return 1;
    const double overhead = elem == 2 ? 2.0 : 0.5, reduce = elem == 2 ? 2.5 : 1.0;
    double best = 0.7 * ((double)nchunks + overhead);
    int32_t pick = 1;
    for (int32_t s = 2; s <= std::min(nchunks, 8); ++s) {
        const int64_t per = ceil_div(nchunks, s);
        if (ceil_div(nchunks, per) != s) continue;
        const double t = (double)ceil_div(s * rem, slots) * ((double)per + overhead) + reduce;
        if (t < best) {
            best = t;
            pick = s;
        }
    }
    return pick;
}

// Register transpose of a SUB×SUB block: in[i] holds SUB pixels of channel i,
// out[j] holds SUB channels of pixel j.
__device__ __forceinline__ void transpose_block(const u32x4 (&in)[8], u32x4 (&out)[8]) {
    // bf16: dword d of in[i] = pixels (2d, 2d+1); dword e of out[j] = channels (2e, 2e+1).
#pragma unroll
    for (int d = 0; d < 4; ++d) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t a = in[2 * e][d], b = in[2 * e + 1][d];
            out[2 * d][e] = (a & 0xffffu) | (b << 16);
            out[2 * d + 1][e] = (a >> 16) | (b & 0xffff0000u);
        }
    }
}
__device__ __forceinline__ void transpose_block(const u32x4 (&in)[4], u32x4 (&out)[4]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) out[j] = u32x4{in[0][j], in[1][j], in[2][j], in[3][j]};
}

// Fill tasks per thread whose global loads are issued one channel chunk ahead
// and held in registers across the MFMA loop; a tile with more tasks (one
// that spans more padded rows, e.g. across an image boundary) loads the rest
// when it stores them.
template <typename T> struct VecTasks;
template <> struct VecTasks<bf16_t> { static constexpr int VT = 1; };
template <> struct VecTasks<float> { static constexpr int VT = 2; };

// Chunk ch (E elements, 16 bytes) of an image row of w elements, read with
// LW-byte loads (LW = 16 when rows are whole 16-byte chunks; 8, 4 or 2 when
// w is only a multiple of 4, 2 or 1 bf16 / of 2 or 1 fp32): pieces past the
// row end read as zero.
template <typename T, int LW, bool NT = false>
__device__ __forceinline__ u32x4 load_chunk(const T* __restrict__ row, int ch, int w) {
    constexpr int E = 16 / (int)sizeof(T), PE = LW / (int)sizeof(T);   // elements per chunk / per piece
    u32x4 v = u32x4{0u, 0u, 0u, 0u};
    if constexpr (LW == 16) {
        if (ch * E < w) {
            const u32x4* q = reinterpret_cast<const u32x4*>(row + ch * E);
            v = NT ? __builtin_nontemporal_load(q) : *q;
        }
    } else if constexpr (LW == 8) {
#pragma unroll
        for (int q = 0; q < 2; ++q)
            if (ch * E + q * PE < w) {
                const uint2 t = *reinterpret_cast<const uint2*>(row + ch * E + q * PE);
                v[2 * q] = t.x;
                v[2 * q + 1] = t.y;
            }
    } else if constexpr (LW == 4) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
            if (ch * E + q * PE < w) v[q] = *reinterpret_cast<const uint32_t*>(row + ch * E + q * PE);
    } else {
        static_assert(LW == 2 && sizeof(T) == 2, "2-byte pieces are bf16 elements");
#pragma unroll
        for (int q = 0; q < 8; ++q)
            if (ch * E + q < w) v[q >> 1] |= (uint32_t)reinterpret_cast<const uint16_t*>(row)[ch * E + q] << (16 * (q & 1));
    }
    return v;
}

// bf16 chunk ch of a row whose start is only 2-byte aligned (LW = 2 above),
// in at most two loads: the 16 bytes from the dword at or below
// the chunk start (one more dword when the start is odd in elements and the
// chunk has 8 elements), realigned with funnel shifts; elements past the row
// end read as zero.  Multi-dword global loads need only dword alignment.
// The loads reach up to 7 elements past the row end (the next row or plane):
// the caller must not use it on the tensor's last row.
typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));
template <typename T>
__device__ __forceinline__ u32x4 load_chunk_narrow(const T* __restrict__ row, int ch, int w) {
    static_assert(sizeof(T) == 2, "realigning loads are for bf16 rows");
    u32x4 v = u32x4{0u, 0u, 0u, 0u};
    const int n = min(8, w - 8 * ch);        // elements of the chunk inside the row
    if (n <= 0) return v;
    const T* s = row + 8 * ch;
    const bool odd = ((uintptr_t)s & 2) != 0;
    const u32x4 d = *reinterpret_cast<const u32x4_a4*>(odd ? s - 1 : s);
    if (odd) {
        const uint32_t d4 = n == 8 ? *reinterpret_cast<const uint32_t*>(s + 7) : 0u;
        v = u32x4{__builtin_amdgcn_alignbit(d.y, d.x, 16), __builtin_amdgcn_alignbit(d.z, d.y, 16),
                  __builtin_amdgcn_alignbit(d.w, d.z, 16), __builtin_amdgcn_alignbit(d4, d.w, 16)};
    } else {
        v = d;
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        if (2 * q >= n) v[q] = 0u;
        else if (2 * q + 1 >= n) v[q] &= 0xffffu;
    }
    return v;
}

}  // namespace conv_fast
}  // namespace nott
