// Device helpers of the fused-decode GEMV kernels (shared by gemv.hip, shared.hip, decode.hip).
#pragma once
#include "common.h"

namespace moe {

// 32 activations for (row-block blk, chunk c): cols 256*blk + 64g + l0 + i and +32
template <int XDT>
__device__ __forceinline__ void load_x32(const void* x, size_t off, float* xl, float* xh) {
  if (XDT == MOE_DT_F32) {
    const float* p = reinterpret_cast<const float*>(x) + off;
#pragma unroll
    for (int i = 0; i < 16; i += 4) {
      float4 a = *reinterpret_cast<const float4*>(p + i);
      float4 b = *reinterpret_cast<const float4*>(p + 32 + i);
      xl[i] = a.x; xl[i + 1] = a.y; xl[i + 2] = a.z; xl[i + 3] = a.w;
      xh[i] = b.x; xh[i + 1] = b.y; xh[i + 2] = b.z; xh[i + 3] = b.w;
    }
  } else {
    const uint16_t* p = reinterpret_cast<const uint16_t*>(x) + off;
#pragma unroll
    for (int i = 0; i < 16; i += 8) {
      uint4 a = *reinterpret_cast<const uint4*>(p + i);
      uint4 b = *reinterpret_cast<const uint4*>(p + 32 + i);
      const uint32_t aa[4] = {a.x, a.y, a.z, a.w}, bb[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        xl[i + 2 * j] = bf16_to_f32(aa[j] & 0xFFFFu);
        xl[i + 2 * j + 1] = bf16_to_f32(aa[j] >> 16);
        xh[i + 2 * j] = bf16_to_f32(bb[j] & 0xFFFFu);
        xh[i + 2 * j + 1] = bf16_to_f32(bb[j] >> 16);
      }
    }
  }
}

// partial dot of one lane's 16-byte Q4_K chunk with its 32 activations
__device__ __forceinline__ float q4k_chunk_dot(uint4 hdr, uint4 qs, int g, const float* xl,
                                               const float* xh, float sxl, float sxh) {
  const float d = f16_to_f32(hdr.x & 0xFFFFu), dmin = f16_to_f32(hdr.x >> 16);
  uint32_t sc0, m0, sc1, m1;
  q4k_scale_min(hdr.y, hdr.z, hdr.w, 2 * g, sc0, m0);
  q4k_scale_min(hdr.y, hdr.z, hdr.w, 2 * g + 1, sc1, m1);
  const uint32_t w[4] = {qs.x, qs.y, qs.z, qs.w};
  float dl = 0.0f, dh = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const uint32_t byte = (w[i >> 2] >> (8 * (i & 3))) & 0xFFu;
    dl = fmaf(xl[i], (float)(byte & 15u), dl);
    dh = fmaf(xh[i], (float)(byte >> 4), dh);
  }
  return d * ((float)sc0 * dl + (float)sc1 * dh) - dmin * ((float)m0 * sxl + (float)m1 * sxh);
}

template <int XDT>
__device__ __forceinline__ void load_x8(const void* x, size_t off, float* v) {
  if (XDT == MOE_DT_F32) {
    const float* p = reinterpret_cast<const float*>(x) + off;
    float4 a = *reinterpret_cast<const float4*>(p);
    float4 b = *reinterpret_cast<const float4*>(p + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
    uint4 a = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(x) + off);
    const uint32_t aa[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[2 * j] = bf16_to_f32(aa[j] & 0xFFFFu);
      v[2 * j + 1] = bf16_to_f32(aa[j] >> 16);
    }
  }
}

__device__ __forceinline__ float dot8_bf16(uint4 w, const float* x) {
  const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
  float a = 0.0f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    a = fmaf(bf16_to_f32(ww[j] & 0xFFFFu), x[2 * j], a);
    a = fmaf(bf16_to_f32(ww[j] >> 16), x[2 * j + 1], a);
  }
  return a;
}

}  // namespace moe
