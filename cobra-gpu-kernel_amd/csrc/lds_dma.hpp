// Global -> LDS DMA (global_load_lds_dwordx4 on gfx950) and the waits around it.
//
// One wave instruction moves 16 bytes per lane into LDS at
// (wave-uniform base) + 16 * lane: the LDS destination is fixed by the lane
// index, the global source of each lane is free.  The transfer bypasses the
// VGPRs and counts in vmcnt like any global load.
#pragma once

#include "common.hpp"

namespace cobra {

typedef __attribute__((address_space(3))) void* lds_ptr;

// 16 bytes per lane from `src` to lds_base + 16 * lane; lds_base must be wave-uniform.
__device__ __forceinline__ void dma16(const void* src, void* lds_base) {
  __builtin_amdgcn_global_load_lds(src, (lds_ptr)lds_base, 16, 0, 0);
}

// s_waitcnt vmcnt(n), leaving the other counters unconstrained (gfx9 encoding).
// The empty asm statement keeps the compiler from hoisting reads of the DMA'd
// LDS above the wait.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
  asm volatile("" ::: "memory");
}

// Workgroup barrier without the memory fence of __syncthreads(): that fence
// waits for every outstanding LDS-DMA (vmcnt(0)), including ones issued for
// later pipeline stages.  Callers wait for exactly the DMA they need with
// wait_vmcnt; the empty asm statements keep the compiler from moving memory
// accesses across.
__device__ __forceinline__ void stage_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Workgroup barrier that publishes this wave's LDS writes (lgkmcnt(0)) but,
// unlike __syncthreads(), does not wait for outstanding global loads or DMA.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt((63 & 15) | ((63 >> 4) << 14) | (7 << 4) | (0 << 8));
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

}  // namespace cobra
