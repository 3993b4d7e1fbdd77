// Direct global->LDS loads (global_load_lds_dword[x4]) issued from inline
// assembly.
//
// Lane i of one instruction writes the i-th slot (4 or 16 bytes) after the
// LDS base held in M0.  The compiler is not told about these loads: left to
// itself it cannot prove that later transposed LDS reads
// (ds_read_b64_tr_b16) do not alias the pending writes, and it then waits for
// every outstanding load (vmcnt(0)) before each such read, which cancels any
// prefetch.  Kernels using these helpers therefore wait for their own loads
// explicitly (s_waitcnt vmcnt(n) before the barrier that publishes a tile).
// Loads the compiler does not count only make its own vmcnt waits more
// conservative, never less.  M0 is saved and restored around each load.
#pragma once

#include <stdint.h>

#define ALODLM_LDS_AS __attribute__((address_space(3)))

// LDS byte address of a pointer into a __shared__ array, made wave-uniform.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(ALODLM_LDS_AS const void*)p);
}

// 16 bytes per lane from the per-lane address g.
__device__ __forceinline__ void dma16_v(const void* g, uint32_t lds) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "global_load_lds_dwordx4 %1, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(g), "s"(lds)
      : "memory");
}

// 16 bytes per lane from the wave-uniform base plus the lane's 32-bit offset.
__device__ __forceinline__ void dma16_s(const void* base, uint32_t off, uint32_t lds) {
  uint32_t saved;
  const uint64_t b = (uint64_t)(uintptr_t)base;
  // readfirstlane returns int: go through uint32_t so the low word is
  // zero-extended, never sign-extended into the high word
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32));
  const uint64_t ub = ((uint64_t)hi << 32) | (uint64_t)lo;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %3\n\t"
      "global_load_lds_dwordx4 %1, %2\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(off), "s"(ub), "s"(lds)
      : "memory");
}

// dma16_s for data read once: non-temporal (streamed past the caches' normal
// retention), so it does not evict operands that other workgroups re-read.
__device__ __forceinline__ void dma16_s_nt(const void* base, uint32_t off, uint32_t lds) {
  uint32_t saved;
  const uint64_t b = (uint64_t)(uintptr_t)base;
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32));
  const uint64_t ub = ((uint64_t)hi << 32) | (uint64_t)lo;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %3\n\t"
      "global_load_lds_dwordx4 %1, %2 nt\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(off), "s"(ub), "s"(lds)
      : "memory");
}

// 4 bytes per lane from the per-lane address g.
__device__ __forceinline__ void dma4_v(const void* g, uint32_t lds) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "global_load_lds_dword %1, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(g), "s"(lds)
      : "memory");
}
