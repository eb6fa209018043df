// Tile pipelines fed by direct-to-LDS loads: explicit vmcnt waits, an LDS
// barrier that leaves global loads in flight, and the 16-byte direct-to-LDS
// load (shared by the prefill attention and the QKV projection).
#pragma once

#include "gkv_device.hpp"

namespace gkv {

typedef __attribute__((address_space(3))) void *lds_ptr;

// s_waitcnt with vmcnt = N and the other counters left alone (gfx9 encoding:
// vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Workgroup barrier for LDS data: this wave's LDS writes complete
// (lgkmcnt(0)), then s_barrier. Unlike __syncthreads() it does not wait for
// the global loads in flight: a workgroup fence also waits for the tile
// pipeline's direct-to-LDS loads, which are waited for explicitly
// (wait_vmcnt). The empty asm statements keep the compiler from moving
// memory accesses across the barrier.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14)); // lgkmcnt(0) only
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// 16 bytes per lane from global memory straight into LDS: lane l's bytes land
// at l_base + 16 l (l_base wave-uniform, held in M0). Written as asm so that
// the compiler, which would count these loads as pending LDS stores and wait
// for all of them before unrelated LDS reads, leaves their waits to the
// pipeline's explicit wait_vmcnt; the compiler's own waits for its loads can
// then only be stricter than needed, never weaker.
__device__ __forceinline__ void dma16(const void *src, void *l_base) {
  const uint32_t m = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_ptr)l_base);
  uint32_t saved;
  asm volatile("s_mov_b32 %0, m0\n\t"
               "s_mov_b32 m0, %2\n\t"
               "s_nop 0\n\t" // one wait state between an SALU write of M0 and an LDS-DMA load
               "global_load_lds_dwordx4 %1, off\n\t"
               "s_mov_b32 m0, %0" // M0 as the compiler left it
               : "=&s"(saved)
               : "v"(src), "s"(m)
               : "memory");
}

// dma16 with a wave-uniform base address (held in SGPRs) and a 32-bit byte
// offset per lane: no 64-bit address per lane is formed or kept.
__device__ __forceinline__ void dma16_s(const void *base, uint32_t byte_off, void *l_base) {
  const uint32_t m = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_ptr)l_base);
  const uint64_t b = (uint64_t)(uintptr_t)base;
  // (readfirstlane returns a signed int: each half is taken as unsigned
  // before it is widened, or a low half >= 2^31 would fill the high one)
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32));
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b);
  const uint64_t sb = ((uint64_t)hi << 32) | lo;
  uint32_t saved;
  asm volatile("s_mov_b32 %0, m0\n\t"
               "s_mov_b32 m0, %3\n\t"
               "s_nop 0\n\t"
               "global_load_lds_dwordx4 %1, %2\n\t"
               "s_mov_b32 m0, %0"
               : "=&s"(saved)
               : "v"(byte_off), "s"(sb), "s"(m)
               : "memory");
}

// 4 bytes per lane straight into LDS: lane l's dword lands at l_base + 4 l.
__device__ __forceinline__ void dma4(const void *src, void *l_base) {
  const uint32_t m = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_ptr)l_base);
  uint32_t saved;
  asm volatile("s_mov_b32 %0, m0\n\t"
               "s_mov_b32 m0, %2\n\t"
               "s_nop 0\n\t"
               "global_load_lds_dword %1, off\n\t"
               "s_mov_b32 m0, %0"
               : "=&s"(saved)
               : "v"(src), "s"(m)
               : "memory");
}

} // namespace gkv
