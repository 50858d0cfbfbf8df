// Direct global->LDS loads (gfx950 global_load_lds_dwordx4) issued from
// inline asm, and the explicit waits that go with them.
#pragma once

#include "tm_common.h"

// One wave-wide 16-byte-per-lane direct load into LDS at `lds_base` (wave
// uniform) + 16 * lane.  Issued from inline asm so the compiler's own wait
// insertion does not treat it as an LDS store (it would drain every in-flight
// stage before each LDS read); the loads are waited for explicitly.  M0 is
// saved and restored around the load.
__device__ __forceinline__ void tm_dma16(const void *gaddr, const void *lds_base) {
  const uint32_t base = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds_base);
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "global_load_lds_dwordx4 %1, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(gaddr), "s"(base)
      : "memory");
}

template <int N>
__device__ __forceinline__ void tm_wait_vm_lgkm0() {
  // s_waitcnt vmcnt(N) lgkmcnt(0), expcnt left at its maximum
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4));
}
