// lds_ring.h -- global -> LDS transfer rings: the transfers, exact vmcnt waits and the
// inline-asm LDS reads of ring slots (shared by the LDS-ring MFMA kernels).
#pragma once

#include "common.h"

namespace nve {

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt immediate");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

typedef __attribute__((address_space(3))) void lds_void_t;
__device__ __forceinline__ void lds_dma16(const void* g, char* l) {
  __builtin_amdgcn_global_load_lds(g, (lds_void_t*)l, 16, 0, 0);
}
__device__ __forceinline__ void lds_dma4(const void* g, char* l) {
  __builtin_amdgcn_global_load_lds(g, (lds_void_t*)l, 4, 0, 0);
}

// Ring reads are inline asm: the compiler's wait insertion cannot tell the ring slots
// apart and would drain every transfer in flight (vmcnt(0)) before each LDS read of a
// slot that a transfer has targeted.  The slot's own transfers are waited for with the
// exact vmcnt above; the reads' results are waited for with lgkm_wait() and passed
// through tie() so no use is scheduled above that wait.
typedef __attribute__((address_space(3))) const char lds_cchar_t;
__device__ __forceinline__ uint32_t lds_addr(const char* p) { return (uint32_t)(uintptr_t)(lds_cchar_t*)p; }
__device__ __forceinline__ u32x4_t ds_read128(uint32_t a) {
  u32x4_t v;
  asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(a));
  return v;
}
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
template <int O0, int O1>
__device__ __forceinline__ u32x2_t ds_read2(uint32_t a) {
  u32x2_t v;
  asm volatile("ds_read2_b32 %0, %1 offset0:%2 offset1:%3" : "=v"(v) : "v"(a), "i"(O0), "i"(O1));
  return v;
}
__device__ __forceinline__ void lgkm_wait() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
template <class V>
__device__ __forceinline__ void tie(V& v) {
  asm volatile("" : "+v"(v));
}
__device__ __forceinline__ u32x2_t ds_read64(uint32_t a) {
  u32x2_t v;
  asm volatile("ds_read_b64 %0, %1" : "=v"(v) : "v"(a));
  return v;
}

}  // namespace nve
