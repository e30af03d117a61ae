// Direct-to-LDS DMA, wait and barrier plumbing shared by the history kernels and the fused
// post-attention finisher (inline asm: the compiler cannot tell ring stages apart).
#pragma once

#include "common.h"

namespace oscar {

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Direct-to-LDS loads are issued by asm so that the compiler does not serialize LDS reads
// behind outstanding DMA (it cannot tell the two ring stages apart); ordering comes from
// the explicit vmcnt waits below. M0 holds the LDS base (any dword address). Lane l writes
// LDS bytes [M0 + 16 l, +16).
// Each asm starts with 5 wait states: a vector-memory instruction that reads an SGPR (the
// saddr base, M0) must follow a VALU write of that SGPR (v_readfirstlane, which the compiler
// emits when it cannot prove the operand uniform) by 5 wait states, and the compiler's hazard
// check does not look inside asm. Without them a load can use a stale base.
// A wave-uniform pointer, kept in SGPRs for the saddr form of the DMA.
__device__ __forceinline__ const uint8_t* uniform_ptr(const uint8_t* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
  return reinterpret_cast<const uint8_t*>((static_cast<uint64_t>(hi) << 32) | lo);
}
__device__ __forceinline__ void dma_x4(const uint8_t* base, uint32_t voff, uint32_t lds) {
  base = uniform_ptr(base);
  asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %1, %2" : : "{m0}"(lds), "v"(voff), "s"(base)
               : "memory");
}
// The same with the non-temporal hint: records read once per step, which should not displace
// the step's reused data (rotations, query rows, split partials) from the caches.
__device__ __forceinline__ void dma_x4_stream(const uint8_t* base, uint32_t voff, uint32_t lds) {
  base = uniform_ptr(base);
  asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %1, %2 nt" : : "{m0}"(lds), "v"(voff), "s"(base)
               : "memory");
}
__device__ __forceinline__ void dma_dwordx4(const void* src, uint32_t lds) {
  asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %1, off" : : "{m0}"(lds), "v"(src)
               : "memory");
}
// The same with the device-coherent cache policy (sc1): rows that another workgroup of the
// launch wrote with device-coherent stores (the L2 of each XCD is not coherent with the others').
__device__ __forceinline__ void dma_dwordx4_coherent(const void* src, uint32_t lds) {
  asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %1, off sc1" : : "{m0}"(lds), "v"(src)
               : "memory");
}
#define OSCAR_WAIT_VM(n) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(n) : "memory")
// vmcnt(0) as the compiler's own wait instruction (gfx9 encoding: expcnt and lgkmcnt left
// open). The compiler's wait insertion does not see the DMAs of the inline assembly above,
// nor waits written in inline assembly: a register loaded by an ordinary load before a loop
// of DMAs gets a wait for it placed inside the loop, where at run time it also waits for
// every DMA in flight. After this wait the compiler counts such loads as landed.
#define OSCAR_WAIT_VM0_SEEN() __builtin_amdgcn_s_waitcnt(0xF70)
#define OSCAR_WAIT_LGKM() asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory")

// Workgroup barrier that waits for this wavefront's LDS traffic but not for its DMA
// (__syncthreads would also drain every outstanding load).
__device__ __forceinline__ void barrier_lds() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_ptr_t)p));
}

}  // namespace oscar
