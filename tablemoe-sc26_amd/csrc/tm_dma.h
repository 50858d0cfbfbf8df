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

// The same direct-to-LDS load through a buffer resource (4 SGPRs: base,
// stride 0, size in bytes, raw 32-bit format): lanes whose byte offset is at
// or past the size are range-checked by the hardware and read nothing, so a
// stage that runs past the end of the table needs no clamping.
typedef uint32_t tm_rsrc_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ tm_rsrc_t tm_make_rsrc(const void *base, uint64_t bytes) {
  const uint64_t a = (uint64_t)(uintptr_t)base;
  tm_rsrc_t r;
  r.x = __builtin_amdgcn_readfirstlane((uint32_t)a);
  r.y = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32) & 0xffffu);  // stride 0
  r.z = __builtin_amdgcn_readfirstlane((uint32_t)(bytes < 0xffffffffull ? bytes : 0xffffffffull));
  r.w = 0x00020000u;  // raw buffer, 32-bit data format
  return r;
}

__device__ __forceinline__ void tm_dma16_buf(tm_rsrc_t rsrc, uint32_t voff, uint32_t lds_base) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %3\n\t"
      "buffer_load_dwordx4 %1, %2, 0 offen lds\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(voff), "s"(rsrc), "s"(lds_base)
      : "memory");
}

// tm_dma16_buf with a scalar byte offset added to every lane's (soff: one
// SGPR, so a loop can step through a matrix's K dimension without touching
// the per-lane offsets) and the LDS base already in an SGPR.
__device__ __forceinline__ void tm_dma16_buf_so(tm_rsrc_t rsrc, uint32_t voff, uint32_t soff, uint32_t lds_base) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %4\n\t"
      "buffer_load_dwordx4 %1, %2, %3 offen lds\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(voff), "s"(rsrc), "s"(soff), "s"(lds_base)
      : "memory");
}

// tm_dma16 with the LDS base already in an SGPR (no readfirstlane).
__device__ __forceinline__ void tm_dma16_s(const void *gaddr, uint32_t lds_base) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "global_load_lds_dwordx4 %1, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(gaddr), "s"(lds_base)
      : "memory");
}

template <int N>
__device__ __forceinline__ void tm_wait_vm_lgkm0() {
  // s_waitcnt vmcnt(N) lgkmcnt(0), expcnt left at its maximum
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4));
}
