// Device helpers of the fused-decode GEMV kernels (shared by gemv.hip, shared.hip, decode.hip,
// decode_layer.hip).
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

// v & mask, opaque to the optimizer: it would otherwise fold the mask into each later byte
// extraction (v_bfe_u32 + v_cvt_f32_ubyte0 per value instead of one v_cvt_f32_ubyteN)
__device__ __forceinline__ uint32_t and_opaque(uint32_t v, uint32_t mask) {
  uint32_t r;
  asm("v_and_b32 %0, %1, %2" : "=v"(r) : "v"(v), "s"(mask));
  return r;
}

// partial dot of one lane's 16-byte Q4_K chunk with its 32 activations: chunk g (0..3) of a
// super-block holds sub-blocks 2g (low nibbles) and 2g+1 (high nibbles). The nibbles are masked
// four at a time and converted by byte (v_cvt_f32_ubyte0..3: one instruction per value); the
// 6-bit scales of get_scale_min_k4 (tools/gguf_reader.py:165-175) are extracted without branches.
__device__ __forceinline__ float q4k_chunk_dot(uint4 hdr, uint4 qs, int g, const float* xl,
                                               const float* xh, float sxl, float sxh) {
  const float d = f16_to_f32(hdr.x & 0xFFFFu), dmin = f16_to_f32(hdr.x >> 16);
  // sub-blocks j = 2g + h, byte b = j & 3 of the 12 scale bytes s0 = hdr.y, s1 = hdr.z, s2 = hdr.w
  const uint32_t sh0 = 16u * (uint32_t)(g & 1), sh1 = sh0 + 8u;
  // sub-blocks 0..3 take plain 6-bit fields, 4..7 the split ones; both forms are computed and one
  // is picked by a lane mask (a select the compiler keeps as bit operations, not as two
  // exec-masked paths)
  const uint32_t low = 0u - (uint32_t)(g < 2);
  const uint32_t y0 = hdr.y >> sh0, z0 = hdr.z >> sh0, w0 = hdr.w >> sh0;
  const uint32_t y1 = hdr.y >> sh1, z1 = hdr.z >> sh1, w1 = hdr.w >> sh1;
  const uint32_t sc0 = ((y0 & 63u) & low) | (((w0 & 15u) | ((y0 >> 2) & 48u)) & ~low);
  const uint32_t m0 = ((z0 & 63u) & low) | ((((w0 >> 4) & 15u) | ((z0 >> 2) & 48u)) & ~low);
  const uint32_t sc1 = ((y1 & 63u) & low) | (((w1 & 15u) | ((y1 >> 2) & 48u)) & ~low);
  const uint32_t m1 = ((z1 & 63u) & low) | ((((w1 >> 4) & 15u) | ((z1 >> 2) & 48u)) & ~low);
  const uint32_t w[4] = {qs.x, qs.y, qs.z, qs.w};
  float dl = 0.0f, dh = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t lo = and_opaque(w[i], 0x0F0F0F0Fu), hi = and_opaque(w[i] >> 4, 0x0F0F0F0Fu);
    dl = fmaf(xl[4 * i], (float)(lo & 0xFFu), dl);
    dh = fmaf(xh[4 * i], (float)(hi & 0xFFu), dh);
    dl = fmaf(xl[4 * i + 1], (float)((lo >> 8) & 0xFFu), dl);
    dh = fmaf(xh[4 * i + 1], (float)((hi >> 8) & 0xFFu), dh);
    dl = fmaf(xl[4 * i + 2], (float)((lo >> 16) & 0xFFu), dl);
    dh = fmaf(xh[4 * i + 2], (float)((hi >> 16) & 0xFFu), dh);
    dl = fmaf(xl[4 * i + 3], (float)(lo >> 24), dl);
    dh = fmaf(xh[4 * i + 3], (float)(hi >> 24), dh);
  }
  return d * ((float)sc0 * dl + (float)sc1 * dh) - dmin * ((float)m0 * sxl + (float)m1 * sxh);
}

// The same for a Q5_K chunk: qs holds the low 4 bits as in Q4_K and qh the 16 bytes qh[l0..l0+15]
// of its element positions; the 5th bit of element 64g + l is bit 2g of qh[l], that of element
// 64g + 32 + l bit 2g + 1 (tools/gguf_reader.py:271-296). Shifting a qh word right by 2g puts
// each byte's bit 2g at that byte's bit 0 (bits leaving the next byte land at bit 2 or above), so
// one shift and one mask per word place the 5th bits at bit 4 of each byte, next to the nibble.
__device__ __forceinline__ float q5k_chunk_dot(uint4 hdr, uint4 qs, uint4 qh, int g, const float* xl,
                                               const float* xh, float sxl, float sxh) {
  const float d = f16_to_f32(hdr.x & 0xFFFFu), dmin = f16_to_f32(hdr.x >> 16);
  const uint32_t sh0 = 16u * (uint32_t)(g & 1), sh1 = sh0 + 8u;
  const uint32_t low = 0u - (uint32_t)(g < 2);
  const uint32_t y0 = hdr.y >> sh0, z0 = hdr.z >> sh0, w0 = hdr.w >> sh0;
  const uint32_t y1 = hdr.y >> sh1, z1 = hdr.z >> sh1, w1 = hdr.w >> sh1;
  const uint32_t sc0 = ((y0 & 63u) & low) | (((w0 & 15u) | ((y0 >> 2) & 48u)) & ~low);
  const uint32_t m0 = ((z0 & 63u) & low) | ((((w0 >> 4) & 15u) | ((z0 >> 2) & 48u)) & ~low);
  const uint32_t sc1 = ((y1 & 63u) & low) | (((w1 & 15u) | ((y1 >> 2) & 48u)) & ~low);
  const uint32_t m1 = ((z1 & 63u) & low) | ((((w1 >> 4) & 15u) | ((z1 >> 2) & 48u)) & ~low);
  const uint32_t w[4] = {qs.x, qs.y, qs.z, qs.w};
  const uint32_t h[4] = {qh.x, qh.y, qh.z, qh.w};
  const uint32_t hs = 2u * (uint32_t)g;
  float dl = 0.0f, dh = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t hb = h[i] >> hs;
    const uint32_t lo = and_opaque(w[i], 0x0F0F0F0Fu) | ((hb << 4) & 0x10101010u);
    const uint32_t hi = and_opaque(w[i] >> 4, 0x0F0F0F0Fu) | ((hb << 3) & 0x10101010u);
    dl = fmaf(xl[4 * i], (float)(lo & 0xFFu), dl);
    dh = fmaf(xh[4 * i], (float)(hi & 0xFFu), dh);
    dl = fmaf(xl[4 * i + 1], (float)((lo >> 8) & 0xFFu), dl);
    dh = fmaf(xh[4 * i + 1], (float)((hi >> 8) & 0xFFu), dh);
    dl = fmaf(xl[4 * i + 2], (float)((lo >> 16) & 0xFFu), dl);
    dh = fmaf(xh[4 * i + 2], (float)((hi >> 16) & 0xFFu), dh);
    dl = fmaf(xl[4 * i + 3], (float)(lo >> 24), dl);
    dh = fmaf(xh[4 * i + 3], (float)(hi >> 24), dh);
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

// 8 weights from element i of a bf16 or f32 vector (dt = MOE_DT_BF16 / MOE_DT_F32, uniform across
// the wave) dotted with 8 activations: the scalar shared gate is bf16 in the synthetic configs and
// f32 in the shipped artifact (ffn_gate_inp_shexp, engine/block_forward.py:221-231).
__device__ __forceinline__ float dot8_w(const void* w, size_t i, int dt, const float* x) {
  if (dt == MOE_DT_F32) {
    const float4 a = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(w) + i);
    const float4 b = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(w) + i + 4);
    float s = fmaf(a.x, x[0], 0.0f);
    s = fmaf(a.y, x[1], s); s = fmaf(a.z, x[2], s); s = fmaf(a.w, x[3], s);
    s = fmaf(b.x, x[4], s); s = fmaf(b.y, x[5], s); s = fmaf(b.z, x[6], s); s = fmaf(b.w, x[7], s);
    return s;
  }
  return dot8_bf16(*reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(w) + i), x);
}

// 8 consecutive weights of a Q8_0 row (blocks of f16 d + 32 x int8, 34 B, value d * q:
// tools/gguf_reader.py:238-245) from element e0 (e0 % 8 == 0), as the block's d and two words of
// quants. Blocks are 2-byte aligned; a pair of blocks (68 B) is 4-byte aligned when the row is and
// has an even block count, so the reads are aligned dwords of the pair, realigned with
// v_alignbyte, and never leave it.
__device__ __forceinline__ void q8_0_load8(const uint8_t* row, int e0, float& d, uint32_t& qlo,
                                           uint32_t& qhi) {
  const int b = e0 >> 5, qq = (e0 >> 3) & 3;
  const uint32_t* pair = reinterpret_cast<const uint32_t*>(row + 68 * (b >> 1));
  const int s = (b & 1) * 34;                                  // the block's byte in the pair
  d = f16_to_f32((pair[s >> 2] >> ((s & 3) * 8)) & 0xFFFFu);
  const int o = s + 2 + 8 * qq, i0 = o >> 2, sh = o & 3;      // sh: 2 (even block) or 0 (odd)
  const uint32_t w0 = pair[i0], w1 = pair[i0 + 1];
  const uint32_t w2 = sh ? pair[i0 + 2] : 0u;
  qlo = __builtin_amdgcn_alignbyte(w1, w0, sh);
  qhi = __builtin_amdgcn_alignbyte(w2, w1, sh);
}
__device__ __forceinline__ float q8_0_dot8(float d, uint32_t qlo, uint32_t qhi, const float* x) {
  float a = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) a = fmaf(x[i], (float)(int8_t)(qlo >> (8 * i)), a);
#pragma unroll
  for (int i = 0; i < 4; ++i) a = fmaf(x[4 + i], (float)(int8_t)(qhi >> (8 * i)), a);
  return d * a;
}
// One Q8_0 block held as the 9 aligned dwords of its half of a 4-byte-aligned block pair (odd =
// the pair's second block: dwords 8..16 of the pair) dotted with its 32 activations x:
// d * sum_i x_i q_i, the quants as exact floats.
__device__ __forceinline__ float q8_0_block_dot(const uint32_t* w, int odd, const float* x) {
  const float d = f16_to_f32(odd ? (w[0] >> 16) : (w[0] & 0xFFFFu));
  float a = 0.0f;
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    // quants start at byte 2 of the window (even block) or byte 4 (odd block)
    const uint32_t q = odd ? w[m + 1] : __builtin_amdgcn_alignbyte(w[m + 1], w[m], 2);
#pragma unroll
    for (int b = 0; b < 4; ++b) a = fmaf(x[4 * m + b], (float)(int8_t)(q >> (8 * b)), a);
  }
  return d * a;
}

// the shared expert's weight rows: bf16 (SFMT = MOE_FMT_BF16) or Q8_0 (the shipped artifact's
// ffn_*_shexp); element e0 of row `row` (cols elements), 8 weights dotted with x
template <int SFMT>
__device__ __forceinline__ float dot8_shared(const void* w, size_t row, int cols, int e0, const float* x) {
  if (SFMT == MOE_FMT_Q8_0) {
    float d;
    uint32_t lo, hi;
    q8_0_load8(reinterpret_cast<const uint8_t*>(w) + row * (size_t)(cols / 32 * 34), e0, d, lo, hi);
    return q8_0_dot8(d, lo, hi, x);
  }
  return dot8_bf16(*reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(w) + row * cols + e0), x);
}

}  // namespace moe
