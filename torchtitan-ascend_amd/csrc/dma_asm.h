// Inline-asm memory operations shared by the persistent LDS-DMA GEMMs
// (internal to libttamd_moe.so).
//
// The LDS DMA loads (global_load_lds_*), the stage barrier and the
// tile-table loads are inline asm: the compiler neither tracks the DMA (with
// DMA and other loads in flight it would wait for everything before each LDS
// read) nor moves memory operations across them ("memory" clobber).  A
// kernel using them counts its own vector-memory operations: those of one
// wave complete in issue order, so "at most N in flight" means "all but the
// N most recent have completed", and any later load or store only makes a
// wait stricter.
//
// GFX9-family manual wait states the compiler cannot see through inline asm:
// a VMEM/SMEM instruction reading an SGPR written by a VALU instruction
// (v_readfirstlane) needs 5, an LDS DMA reading M0 written by SALU needs 1.
// Every asm statement that reads SGPR operands starts with s_nop 4.
// Nothing here writes through the scalar cache.
#pragma once

#include "common.h"

namespace ttamd {
namespace dma {

typedef __attribute__((address_space(3))) char* lds_ptr_t;
typedef int i32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t lds_addr(const char* p) {
  return (uint32_t)(uintptr_t)(lds_ptr_t)p;
}

// Chunk permutation of 128-byte LDS rows.
__device__ __forceinline__ int cswz(int r) { return (r ^ (r >> 3)) & 7; }

__device__ __forceinline__ uint64_t uniform64(uint64_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return ((uint64_t)hi << 32) | lo;
}

// 16 bytes per lane from sbase + voff to LDS [lds + 16 * lane].
__device__ __forceinline__ void dma16(uint32_t voff, uint64_t sbase, uint32_t lds) {
  asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(uniform64(sbase)),
               "{m0}"(__builtin_amdgcn_readfirstlane(lds))
               : "memory");
}

// 4 bytes per lane from sbase + voff to LDS [lds + 4 * lane].
__device__ __forceinline__ void dma4(uint32_t voff, uint64_t sbase, uint32_t lds) {
  asm volatile("s_nop 4\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(uniform64(sbase)),
               "{m0}"(__builtin_amdgcn_readfirstlane(lds))
               : "memory");
}

// At most N vector-memory operations of this wave in flight, its LDS reads
// complete, then a workgroup barrier.
template <int N>
__device__ __forceinline__ void wait_vm_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Wave-uniform loads through the scalar cache (read only).
__device__ __forceinline__ int4 sload_int4(const int4* p) {
  i32x4_t v;
  asm volatile("s_nop 4\n\ts_load_dwordx4 %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)"
               : "=s"(v)
               : "s"(uniform64((uint64_t)p))
               : "memory");
  return make_int4(__builtin_amdgcn_readfirstlane(v[0]), __builtin_amdgcn_readfirstlane(v[1]),
                   __builtin_amdgcn_readfirstlane(v[2]), __builtin_amdgcn_readfirstlane(v[3]));
}

__device__ __forceinline__ int sload_int(const int* p) {
  int v;
  asm volatile("s_nop 4\n\ts_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)"
               : "=s"(v)
               : "s"(uniform64((uint64_t)p))
               : "memory");
  return __builtin_amdgcn_readfirstlane(v);
}

}  // namespace dma
}  // namespace ttamd
