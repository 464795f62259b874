// Q4_K operand helpers of the f16 MFMA grouped GEMMs (gemm4.hip, gemm6.hip): LDS swizzles, the
// 32x32x16 f16 MFMA, and the in-register decode of Q4_K nibbles into B fragments.
#pragma once
#include "common.h"

namespace moe {

typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

namespace q4m {

// activation rows: 16-byte chunk c of row m at chunk c ^ a_swz(m); nibble rows: half h of row n
// at half h ^ q_swz(n)
__device__ __forceinline__ int a_swz(int m) { return (m ^ (m >> 1)) & 7; }
__device__ __forceinline__ int q_swz(int n) { return ((n >> 2) ^ (n >> 3)) & 1; }

__device__ __forceinline__ f32x16_t mfma(uint4 a, uint4 b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                               __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

__device__ __forceinline__ uint32_t and_or_s(uint32_t p, uint32_t mask, uint32_t magic) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(p), "s"(mask), "v"(magic));
  return r;
}

// 2 nibbles (bytes of w at positions sel) -> f16x2, scale applied: a low nibble under the f16
// 0x6400 (1024) gives 1024 + q, a high nibble left at bits 4-7 under 0x5400 (64, ulp 1/16) gives
// 64 + q; one packed subtract leaves q exactly and one packed FMA gives q * ds + ndm.
template <bool HIGH>
__device__ __forceinline__ uint32_t q4_pair(uint32_t w, uint32_t sel, f16x2_t ds, f16x2_t ndm) {
  const uint32_t p = __builtin_amdgcn_perm(0u, w, sel);
  const uint32_t magic = HIGH ? and_or_s(p, 0x00F000F0u, 0x54005400u)
                              : and_or_s(p, 0x000F000Fu, 0x64006400u);
  const _Float16 off = HIGH ? (_Float16)64.0f : (_Float16)1024.0f;
  const f16x2_t q = __builtin_bit_cast(f16x2_t, magic) - (f16x2_t){off, off};
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(q, ds, ndm));
}

// 8 bytes of nibbles (w0, w1) -> the 8 f16 of one B fragment (low or high nibbles, byte order)
template <bool HIGH>
__device__ __forceinline__ uint4 q4_frag(uint32_t w0, uint32_t w1, f16x2_t ds, f16x2_t ndm) {
  return make_uint4(q4_pair<HIGH>(w0, 0x0C010C00u, ds, ndm), q4_pair<HIGH>(w0, 0x0C030C02u, ds, ndm),
                    q4_pair<HIGH>(w1, 0x0C010C00u, ds, ndm), q4_pair<HIGH>(w1, 0x0C030C02u, ds, ndm));
}

// scale and negated min of sub-block j of a super-block header as f16 pairs (get_scale_min_k4,
// tools/gguf_reader.py:165-175; d * sc and dmin * m rounded to f16 once)
__device__ __forceinline__ void q4_scales(uint4 hdr, int j, f16x2_t& ds, f16x2_t& ndm) {
  uint32_t sc, m;
  q4k_scale_min(hdr.y, hdr.z, hdr.w, j, sc, m);
  const _Float16 d = (_Float16)(f16_to_f32(hdr.x & 0xFFFFu) * (float)sc);
  const _Float16 n = (_Float16)(-(f16_to_f32(hdr.x >> 16) * (float)m));
  ds = (f16x2_t){d, d};
  ndm = (f16x2_t){n, n};
}

}  // namespace q4m
}  // namespace moe
