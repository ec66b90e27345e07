// LDS DMA helpers for gfx950 (global_load_lds_dwordx4), shared by the score /
// product kernels (syrk.hip) and the gated GEMM (model.hip).
//
// Operand streams are moved by LDS DMA issued from inline asm, so the
// compiler neither counts them in its own vmcnt waits nor orders LDS
// accesses behind them; kernels wait for them explicitly (sy_wait) and hand
// a landed stage to the other waves with a barrier.
#pragma once

#include <stdint.h>

// (the DMA asm sets m0, which clang reports as a reserved register)
#pragma clang diagnostic ignored "-Winline-asm"

#include <hip/hip_runtime.h>

namespace bdh {

typedef __attribute__((address_space(3))) uint8_t lds_u8;

// A wave-uniform pointer made explicitly scalar (the asm takes it in SGPRs).
__device__ __forceinline__ const void* sgpr_ptr(const void* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(uint32_t(v));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(uint32_t(v >> 32));
  return reinterpret_cast<const void*>((uint64_t(hi) << 32) | lo);
}

// 16 bytes per lane from gbase + voff to LDS address m0base + IMM + 16 * lane.
// m0base must be wave-uniform (an SGPR); voff is a 32-bit byte offset.  The
// immediate keeps one scalar base per stage instead of one per instruction.
template <int IMM>
__device__ __forceinline__ void dma16(uint32_t m0base, const void* gbase, uint32_t voff) {
  asm volatile("s_add_u32 m0, %0, %3\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
               :
               : "s"(m0base), "v"(voff), "s"(gbase), "i"(IMM)
               : "memory", "m0", "scc");
}

// Wait until at most N vector-memory operations of this wave are outstanding
// (they complete in issue order).
template <int N>
__device__ __forceinline__ void sy_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

}  // namespace bdh
