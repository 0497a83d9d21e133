// lds_copy.h — direct global-to-LDS copies for the matrix-core kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qmm {

// One global-to-LDS copy of 16 bytes a lane (global_load_lds_dwordx4): lane
// L's 16 bytes at base + off[L] land at LDS byte lds + 16 L (lds uniform,
// through M0, which is restored). Written as inline assembly: the compiler
// counts its own form of this load among the LDS operations, in a way it
// cannot order against them, and then waits for every LDS read with
// lgkmcnt(0) for the rest of the loop body. A kernel waits for its copies
// itself (vmcnt(0) before the barrier after which they are read) and copies
// only into buffers no wave reads until then.
__device__ __forceinline__ void dma16(const void* base, uint32_t off, uint32_t lds) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %3\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, %2\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(off), "s"(base), "s"(lds)
      : "memory");
}

// The same copy of 4 bytes a lane (global_load_lds_dword): lane L's dword at
// base + off[L] lands at LDS byte lds + 4 L.
__device__ __forceinline__ void dma4(const void* base, uint32_t off, uint32_t lds) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %3\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dword %1, %2\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(off), "s"(base), "s"(lds)
      : "memory");
}

// The LDS byte address of a __shared__ object.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

}  // namespace qmm
