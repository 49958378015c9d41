// dsv_dma.h — LDS-DMA helpers shared by the attention kernel and the fused
// lm_head on gfx950.
//
// buffer_load_dwordx4 ... offen lds moves 16 bytes per lane from global
// memory straight into LDS: lane l of the instruction lands at LDS address
// m0 + 16*l.  The source goes through a buffer resource (base, byte range):
// the hardware checks every lane's offset against the range and returns
// zeros past it.  Callers keep every destination below 64 KiB.
#pragma once

#include "dsv_internal.h"

namespace dsv {

typedef int i32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// A buffer resource (base, byte range) in SGPRs, built once and reused.
__device__ __forceinline__ i32x4 make_rsrc(const void* base, uint32_t range) {
  const uint64_t p = (uint64_t)base;
  i32x4 r;
  r[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)p);
  r[1] = __builtin_amdgcn_readfirstlane((int)(uint32_t)(p >> 32));
  r[2] = __builtin_amdgcn_readfirstlane((int)range);
  r[3] = 0x00020000;
  return r;
}

// One LDS-DMA instruction through resource r_in: this lane's 16 bytes at
// byte offset voff.  NT marks the loads non-temporal (read once).
template <bool NT = true>
__device__ __forceinline__ void dma_rs(uint32_t lds, i32x4 r_in, uint32_t voff) {
  // Uniform by construction; readfirstlane keeps the resource in SGPRs where
  // the compiler cannot prove it (free when it already is).
  i32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = __builtin_amdgcn_readfirstlane(r_in[i]);
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds);
  if constexpr (NT)
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen nt lds" ::"s"(m0), "v"(voff), "s"(r)
                 : "memory", "m0");
  else
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(m0), "v"(voff), "s"(r)
                 : "memory", "m0");
}

// Wait until at most N of this wave's vector-memory operations are pending.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Workgroup barrier that the compiler may not move LDS accesses across and
// that adds no memory-counter waits of its own (the DMA loads are waited for
// explicitly with wait_vmcnt before it).
__device__ __forceinline__ void barrier_lds() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

}  // namespace dsv
