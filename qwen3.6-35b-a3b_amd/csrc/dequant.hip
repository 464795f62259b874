// Bit-exact standalone super-block decode (test entry point; the hot kernels decode in registers).
// Q4_K: v = fma(d*sc, q, -(dmin*m)) — both products are exact in f32, so this is the one rounding
// the f64 route (tools/gguf_reader.py:248-268) also makes (prototype/q4k_dequant/
// q4k_dequant_kernels.h:43-59). Q6_K: v = (d*sc)*(q-32) is exact in f32 (<= 23 significant bits).
#include "common.h"
#include "moe_internal.h"

namespace moe {

// one thread per 16-byte quarter of a Q4_K block's nibble array: 32 elements
template <int OUT>
__global__ __launch_bounds__(256) void k_dequant_q4k(const uint8_t* __restrict__ blk, int64_t nb,
                                                      void* __restrict__ out) {
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t b = gid >> 3;
  const int c = gid & 7;
  if (b >= nb) return;
  const uint8_t* p = blk + b * 144;
  const uint4 hdr = *reinterpret_cast<const uint4*>(p);      // blocks are 16-byte aligned
  const uint4 qs = *reinterpret_cast<const uint4*>(p + 16 + 16 * c);
  const float d = f16_to_f32(hdr.x & 0xFFFFu), dmin = f16_to_f32(hdr.x >> 16);
  const int g = c >> 1, l0 = 16 * (c & 1);
  uint32_t sc0, m0, sc1, m1;
  q4k_scale_min(hdr.y, hdr.z, hdr.w, 2 * g, sc0, m0);
  q4k_scale_min(hdr.y, hdr.z, hdr.w, 2 * g + 1, sc1, m1);
  const float ds0 = d * (float)sc0, dm0 = dmin * (float)m0;
  const float ds1 = d * (float)sc1, dm1 = dmin * (float)m1;
  const uint32_t w[4] = {qs.x, qs.y, qs.z, qs.w};
  const int64_t e0 = b * 256 + 64 * g + l0;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const uint32_t byte = (w[i >> 2] >> (8 * (i & 3))) & 0xFFu;
    const float v0 = fmaf(ds0, (float)(byte & 15u), -dm0);
    const float v1 = fmaf(ds1, (float)(byte >> 4), -dm1);
    if (OUT == MOE_DT_F32) {
      reinterpret_cast<float*>(out)[e0 + i] = v0;
      reinterpret_cast<float*>(out)[e0 + 32 + i] = v1;
    } else {
      reinterpret_cast<uint16_t*>(out)[e0 + i] = (uint16_t)f32_to_bf16(v0);
      reinterpret_cast<uint16_t*>(out)[e0 + 32 + i] = (uint16_t)f32_to_bf16(v1);
    }
  }
}

// Q5_K: one thread per 16-byte quarter of the nibble array as in Q4_K, plus the 16 qh bytes of its
// element positions (176-byte blocks are 16-byte aligned); q = nibble | 5th bit << 4 <= 31, so
// (d*sc)*q is exact in f32 (<= 22 bits) and fma(d*sc, q, -(dmin*m)) again rounds once.
template <int OUT>
__global__ __launch_bounds__(256) void k_dequant_q5k(const uint8_t* __restrict__ blk, int64_t nb,
                                                      void* __restrict__ out) {
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t b = gid >> 3;
  const int c = gid & 7;
  if (b >= nb) return;
  const uint8_t* p = blk + b * 176;
  const uint4 hdr = *reinterpret_cast<const uint4*>(p);
  const int g = c >> 1, l0 = 16 * (c & 1);
  const uint4 qh = *reinterpret_cast<const uint4*>(p + 16 + l0);
  const uint4 qs = *reinterpret_cast<const uint4*>(p + 48 + 16 * c);
  const float d = f16_to_f32(hdr.x & 0xFFFFu), dmin = f16_to_f32(hdr.x >> 16);
  uint32_t sc0, m0, sc1, m1;
  q4k_scale_min(hdr.y, hdr.z, hdr.w, 2 * g, sc0, m0);
  q4k_scale_min(hdr.y, hdr.z, hdr.w, 2 * g + 1, sc1, m1);
  const float ds0 = d * (float)sc0, dm0 = dmin * (float)m0;
  const float ds1 = d * (float)sc1, dm1 = dmin * (float)m1;
  const uint32_t w[4] = {qs.x, qs.y, qs.z, qs.w};
  const uint32_t h[4] = {qh.x, qh.y, qh.z, qh.w};
  const int64_t e0 = b * 256 + 64 * g + l0;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const uint32_t byte = (w[i >> 2] >> (8 * (i & 3))) & 0xFFu;
    const uint32_t hb = (h[i >> 2] >> (8 * (i & 3))) & 0xFFu;
    const uint32_t q0 = (byte & 15u) | (((hb >> (2 * g)) & 1u) << 4);
    const uint32_t q1 = (byte >> 4) | (((hb >> (2 * g + 1)) & 1u) << 4);
    const float v0 = fmaf(ds0, (float)q0, -dm0);
    const float v1 = fmaf(ds1, (float)q1, -dm1);
    if (OUT == MOE_DT_F32) {
      reinterpret_cast<float*>(out)[e0 + i] = v0;
      reinterpret_cast<float*>(out)[e0 + 32 + i] = v1;
    } else {
      reinterpret_cast<uint16_t*>(out)[e0 + i] = (uint16_t)f32_to_bf16(v0);
      reinterpret_cast<uint16_t*>(out)[e0 + 32 + i] = (uint16_t)f32_to_bf16(v1);
    }
  }
}

// one thread per 32-element chunk (g, k) of a Q6_K block; bytes read one at a time because the
// 210-byte blocks are only 2-byte aligned.
template <int OUT>
__global__ __launch_bounds__(256) void k_dequant_q6k(const uint8_t* __restrict__ blk, int64_t nb,
                                                      void* __restrict__ out) {
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t b = gid >> 3;
  const int c = gid & 7;
  if (b >= nb) return;
  const uint8_t* p = blk + b * 210;
  const int g = c >> 2, k = c & 3;
  const uint32_t dbits = (uint32_t)p[208] | ((uint32_t)p[209] << 8);
  const float d = f16_to_f32(dbits);
  const float s0 = d * (float)(int8_t)p[192 + 8 * g + 2 * k];
  const float s1 = d * (float)(int8_t)p[192 + 8 * g + 2 * k + 1];
  const uint8_t* ql = p + 64 * g + 32 * (k & 1);
  const uint8_t* qh = p + 128 + 32 * g;
  const int64_t e0 = b * 256 + 128 * g + 32 * k;
  for (int l = 0; l < 32; ++l) {
    const int q = ((ql[l] >> (4 * (k >> 1))) & 15) | (((qh[l] >> (2 * k)) & 3) << 4);
    const float v = (l < 16 ? s0 : s1) * (float)(q - 32);
    if (OUT == MOE_DT_F32) reinterpret_cast<float*>(out)[e0 + l] = v;
    else reinterpret_cast<uint16_t*>(out)[e0 + l] = (uint16_t)f32_to_bf16(v);
  }
}

}  // namespace moe

using namespace moe;

int moe_launch_dequant(const void* blocks, int fmt, int64_t n_elts, void* out, int out_dtype,
                       hipStream_t st) {
  const int64_t nb = n_elts / 256;
  const int64_t threads = nb * 8;
  const dim3 grid((unsigned)((threads + 255) / 256));
  const uint8_t* b = reinterpret_cast<const uint8_t*>(blocks);
  if (fmt == MOE_FMT_Q4_K) {
    if (out_dtype == MOE_DT_F32) hipLaunchKernelGGL(k_dequant_q4k<MOE_DT_F32>, grid, dim3(256), 0, st, b, nb, out);
    else hipLaunchKernelGGL(k_dequant_q4k<MOE_DT_BF16>, grid, dim3(256), 0, st, b, nb, out);
  } else if (fmt == MOE_FMT_Q5_K) {
    if (out_dtype == MOE_DT_F32) hipLaunchKernelGGL(k_dequant_q5k<MOE_DT_F32>, grid, dim3(256), 0, st, b, nb, out);
    else hipLaunchKernelGGL(k_dequant_q5k<MOE_DT_BF16>, grid, dim3(256), 0, st, b, nb, out);
  } else if (fmt == MOE_FMT_Q6_K) {
    if (out_dtype == MOE_DT_F32) hipLaunchKernelGGL(k_dequant_q6k<MOE_DT_F32>, grid, dim3(256), 0, st, b, nb, out);
    else hipLaunchKernelGGL(k_dequant_q6k<MOE_DT_BF16>, grid, dim3(256), 0, st, b, nb, out);
  } else {
    return moe_set_error(MOE_E_FORMAT, "moe_dequant: unsupported format %d", fmt);
  }
  return moe_check_launch("dequant");
}
