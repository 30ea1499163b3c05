// lds_dma.h — gfx950 LDS-DMA helpers shared by the SpMM and SDDMM kernels:
// buffer loads that write straight into LDS (buffer_load ... lds), their
// SGPR buffer descriptors, and explicit vmcnt waits for rings of stages.
//
// The loads are inline asm, invisible to the compiler's wait insertion: given
// the builtin, it cannot tell a ring's slots apart and waits for every
// outstanding LDS load (vmcnt(0)) before each LDS read, which drains the
// ring.  Invisible loads only ever make the compiler's own vmcnt waits
// stricter (they return in order), so its waits stay correct; a ring's waits
// are explicit.

#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

// Raw buffers (stride 0) span 2^31 - 1 bytes; callers check that every
// operand's offsets fit in 31 bits.  A per-lane offset of kOutOfRange makes
// a load return zeros without a memory request, so that the number of issued
// loads (and so every vmcnt wait) can stay fixed.
constexpr int kOutOfRange = (int)0x80000000u;

// A raw buffer descriptor (stride 0, 2^31 - 1 bytes) held in SGPRs.
typedef int v4s __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v4s sgpr_rsrc(const void* p) {
  const uint64_t a = (uint64_t)(uintptr_t)p;
  return v4s{__builtin_amdgcn_readfirstlane((int)(uint32_t)a), __builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32)),
             0x7fffffff, 0x00020000};
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
}

// 16 bytes per lane: lane l writes LDS bytes lds + 16 l .. + 15.  soff must be
// wave-uniform (it is made an SGPR here).
__device__ __forceinline__ void dma_b128(v4s r, const void* lds, int voff, int soff) {
  asm volatile("buffer_load_dwordx4 %0, %1, %2 offen lds"
               :: "v"(voff), "s"(r), "s"(__builtin_amdgcn_readfirstlane(soff)), "{m0}"(lds_addr(lds)) : "memory");
}

// 4 bytes per lane: lane l writes LDS bytes lds + 4 l .. + 3.
__device__ __forceinline__ void dma_b32(v4s r, const void* lds, int voff, int soff) {
  asm volatile("buffer_load_dword %0, %1, %2 offen lds"
               :: "v"(voff), "s"(r), "s"(__builtin_amdgcn_readfirstlane(soff)), "{m0}"(lds_addr(lds)) : "memory");
}

// s_waitcnt vmcnt(n), also a compiler barrier for memory accesses (the
// builtin is not one: LDS reads could move above it).
template <int N>
__device__ __forceinline__ void wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" :: "n"(N) : "memory");
}

// Wait until at most `ahead` stages of C loads each are outstanding.
template <int C>
__device__ __forceinline__ void wait_stages(int ahead) {
  if (ahead >= 2) wait_vm<2 * C>();
  else if (ahead == 1) wait_vm<C>();
  else wait_vm<0>();
}

}  // namespace
