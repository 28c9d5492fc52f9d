// Global -> LDS DMA for the MFMA kernels (gfx950).
//
// One instruction moves 16 bytes per lane: lane l writes bytes 16l..16l+15 of the 1 KB that
// starts at the (wave-uniform) LDS address in M0. The instructions are issued through inline
// assembly rather than the compiler builtins on purpose: for a builtin the compiler sees an LDS
// write it cannot tell apart from the double buffer being read, so it puts an
// `s_waitcnt vmcnt(0)` in front of the next LDS read -- which waits for the DMA of the *next*
// stage and serialises loading with computing. Hidden in assembly, the DMAs are ordered only by
// the callers' explicit waits (`s_waitcnt vmcnt`, then a barrier, before a buffer is read) and by
// the asm's memory clobber. The compiler still counts its own loads correctly: vector memory
// operations retire in issue order, so a wait for "at most N outstanding" that does not count
// these DMAs only waits longer. M0 is saved and restored around each DMA, and one wait state
// separates the M0 write from the DMA that reads it.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace ku::hipbk {

// buffer form: byte offset voff (per lane, bounds-checked against the descriptor) + soff
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff,
                                          __attribute__((address_space(3))) void* lds) {
  uint32_t m0save;
  const uint32_t la = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds);
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %2, %3, %4 offen lds\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(m0save)
      : "s"(la), "v"(voff), "s"(r), "s"(soff)
      : "memory");
}

// 64-bit address form (operands spanning 2^31 bytes or more)
__device__ __forceinline__ void lds_dma16_g(const void* g, __attribute__((address_space(3))) void* lds) {
  uint32_t m0save;
  const uint32_t la = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds);
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %2, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(m0save)
      : "s"(la), "v"(g)
      : "memory");
}

// s_waitcnt vmcnt(N) through the builtin, so the compiler's own wait bookkeeping knows its loads
// have completed too (an inline-asm wait is opaque to it, and it would wait again, later and for
// everything, before using them)
template <int N>
__device__ __forceinline__ void vm_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  // gfx9 encoding: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] << 14; others at maximum
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

}  // namespace ku::hipbk
