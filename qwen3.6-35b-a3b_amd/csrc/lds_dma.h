// Helpers of the persistent MFMA kernels (gfx950): direct global->LDS loads with explicit vmcnt
// waits, LDS addresses and values kept opaque to the compiler.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace moe {
namespace dma {

// 32-bit LDS byte address of a __shared__ object (wave-uniform)
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p);
}

// 16 bytes per lane from base + off to LDS bytes [lds + 16 lane, +16). Issued as inline asm so
// that the compiler does not wait for it before unrelated LDS reads (it would, for every LDS read
// while any such load is in flight); the caller waits with explicit vmcnt counts (vector memory
// operations complete in issue order). base and lds must be wave-uniform.
__device__ __forceinline__ void load16(uint32_t off, const void* base, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(lds)
               : "memory");
}

// s_waitcnt vmcnt(n), other counters untouched (gfx9 encoding: vmcnt bits 3:0 and 15:14)
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}

// a value the compiler cannot see through: what derives from it is not hoisted out of the loop
// that produces it
__device__ __forceinline__ int opaque(int v) {
  asm volatile("" : "+s"(v));
  return v;
}

// the thread index through an empty asm: derived lane constants are recomputed where they are
// used instead of being kept (or spilled) across a long loop
__device__ __forceinline__ int tid_fresh() {
  int t = (int)threadIdx.x;
  asm volatile("" : "+v"(t));
  return t;
}

// raw buffer descriptor over [p, p + bytes): stores past the end are dropped by the hardware (the
// range check covers the VGPR offset, not the SGPR one)
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, bytes, 0x00020000);
}

}  // namespace dma
}  // namespace moe
