// lds_copy.h — direct global-to-LDS copies for the matrix-core kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qmm {

// One global-to-LDS copy of 16 bytes a lane (global_load_lds_dwordx4): lane
// L's 16 bytes at base + off[L] land at LDS byte lds + 16 L (lds uniform,
// through M0). Written as inline assembly: the compiler counts its own form
// of this load among the LDS operations, in a way it cannot order against
// them, and then waits for every LDS read with lgkmcnt(0) for the rest of
// the loop body. M0 is declared clobbered rather than saved and restored:
// writing M0 back right after the copy holds the wave until the copy has
// read it (a copy probe on gfx950 moved 28% more bytes a cycle without the
// restore); no instruction of the kernels that copy this way reads M0
// elsewhere (their ISA shows none). The compiler warns that M0 in a clobber
// list is a reserved register and does not track it: a kernel that adds an
// instruction reading M0 (s_sendmsg, LDS-direct or indexed moves) must set
// it again after the copies. A kernel waits for its copies itself (vmcnt(0) before the barrier
// after which they are read) and copies only into buffers no wave reads
// until then.
__device__ __forceinline__ void dma16(const void* base, uint32_t off, uint32_t lds) {
  asm volatile(
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, %1"
      :
      : "v"(off), "s"(base), "s"(lds)
      : "memory", "m0");
}

// The same copy of 4 bytes a lane (global_load_lds_dword): lane L's dword at
// base + off[L] lands at LDS byte lds + 4 L.
__device__ __forceinline__ void dma4(const void* base, uint32_t off, uint32_t lds) {
  asm volatile(
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dword %0, %1"
      :
      : "v"(off), "s"(base), "s"(lds)
      : "memory", "m0");
}

// The LDS byte address of a __shared__ object.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

}  // namespace qmm
