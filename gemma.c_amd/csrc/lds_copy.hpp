// LDS copies issued from inline asm (gfx950): global_load_lds rows that the
// compiler neither orders against its own LDS reads nor waits on. The caller
// waits for them (wait_copies) before the barrier that publishes the data,
// and never reads a buffer that a copy in flight may still write.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gemma4 {

// LDS byte address of a __shared__ object (for M0).
__device__ __forceinline__ uint32_t lds_address(const void *ptr) {
  return (uint32_t)reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const char *)ptr);
}

// One 1 KiB LDS copy (global_load_lds, 16 bytes per lane): LDS bytes
// [lds_addr, +1024) from the per-lane addresses src. The copy is invisible
// to the compiler's memory counters: the caller waits for it (vmcnt) before
// the barrier that publishes the tile.
__device__ __forceinline__ void copy_row_pair(uint64_t src, uint32_t lds_addr) {
  uint32_t m0_saved;
  asm volatile(
      "s_mov_b32 %[m0s], m0\n\t"
      "s_mov_b32 m0, %[lds]\n\t"
      "s_nop 0\n\t"  // SALU write of M0 -> LDS DMA reading it: one wait state (gfx9)
      "global_load_lds_dwordx4 %[src], off\n\t"
      "s_mov_b32 m0, %[m0s]"
      : [m0s] "=&s"(m0_saved)
      : [lds] "s"(lds_addr), [src] "v"(src));
}

// One 4-byte-per-lane LDS copy: LDS bytes [lds_addr, +256) from the
// per-lane addresses src (global_load_lds_dword); waited for like
// copy_row_pair.
__device__ __forceinline__ void copy_dwords(const void *src, uint32_t lds_addr) {
  uint32_t m0_saved;
  asm volatile(
      "s_mov_b32 %[m0s], m0\n\t"
      "s_mov_b32 m0, %[lds]\n\t"
      "s_nop 0\n\t"  // SALU write of M0 -> LDS DMA reading it: one wait state (gfx9)
      "global_load_lds_dword %[src], off\n\t"
      "s_mov_b32 m0, %[m0s]"
      : [m0s] "=&s"(m0_saved)
      : [lds] "s"(lds_addr), [src] "v"(src));
}

// Waits for every vector memory operation of this wave, the copies
// included (s_waitcnt vmcnt(0); a builtin rather than inline asm so the
// compiler's own counter bookkeeping sees it as well).
__device__ __forceinline__ void wait_copies() {
  constexpr int kVmcnt0 = 0x0F70;  // gfx9 encoding: vmcnt 0, expcnt 7, lgkmcnt 15 (no wait)
  __builtin_amdgcn_s_waitcnt(kVmcnt0);
}

}  // namespace gemma4
