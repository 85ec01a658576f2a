// LDS DMA and ring-synchronisation helpers shared by the kernels that stream
// operand tiles from global memory straight into LDS (gfx950).
//
// global_load_lds_dword[x4] moves 4 or 16 bytes per lane from a per-lane
// global address to LDS byte `base + size·lane`, with the wave-uniform base in
// M0; no VGPRs hold the data.  Completion is tracked by vmcnt like any other
// vector load.  A ring of LDS stages is then ordered by two things only: this
// wave's s_waitcnt vmcnt (how many of its loads may still be outstanding)
// and an s_barrier (every wave's loads of the stage have landed, and every
// wave has finished reading the slot about to be refilled).
#pragma once

#include "common.hpp"

#define NOTT_LDS __attribute__((address_space(3)))

namespace nott {
namespace lds {

// s_waitcnt vmcnt(n) and lgkmcnt(0) (gfx9 encoding: vmcnt[3:0] and [15:14],
// expcnt[6:4], lgkmcnt[11:8]).
template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0x0 << 8));
}

// Workgroup barrier without a memory fence: the ring's ordering comes from
// the explicit waits (a workgroup fence would make the compiler wait for
// every outstanding load); the empty asm statements keep the compiler from
// moving memory accesses across the barrier.
__device__ __forceinline__ void barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

__device__ __forceinline__ uint32_t lds_addr(const char NOTT_LDS* p) { return (uint32_t)(uintptr_t)p; }

// global_load_lds_dwordx4: 16 bytes per lane from `src` to LDS byte
// lds + 16·lane (lds wave-uniform).  Issued as inline assembly so that the
// compiler does not see an LDS DMA in flight: it would otherwise make every
// later transposing LDS read wait for all outstanding loads (vmcnt(0)),
// which serialises the ring.  The ring's own waits order the DMA against the
// reads.
// M0 is listed as clobbered for the reader; the compiler reserves M0 and
// warns that it ignores the listing, which is harmless here because no
// kernel using these helpers has any other M0 reader (the generated code
// sets M0 only in these statements).  tests/test_lds_dma_m0.py compiles
// every source that includes this header to device assembly and fails if
// the compiler writes M0 itself or emits any other M0 reader.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(const void* src, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds), "v"(src) : "memory", "m0");
}

// global_load_lds_dword: 4 bytes per lane from `src` to LDS byte lds + 4·lane.
__device__ __forceinline__ void dma4(const void* src, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, off" ::"s"(lds), "v"(src) : "memory", "m0");
}
#pragma clang diagnostic pop

}  // namespace lds
}  // namespace nott
