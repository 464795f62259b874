// Shared device helpers for the gfx950 MoE library: bf16/f16 bit handling, wave64 reductions,
// and the GGUF Q4_K / Q6_K element decode (GGUF layout as read by tools/gguf_reader.py:17-51).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define MOE_WAVE 64

// ------------------------------------------------------------------------------ bit handling --
__device__ __forceinline__ float bf16_to_f32(uint32_t u16) { return __uint_as_float(u16 << 16); }

// f32 -> bf16 round-to-nearest-even; NaN quieted to 0x7FC0 (prototype/moe_router/
// moe_router_kernels.h:196-205 states the same RNE rule).
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
  uint32_t b = __float_as_uint(f);
  if ((b & 0x7F800000u) == 0x7F800000u && (b & 0x007FFFFFu)) return 0x7FC0u;
  return (b + 0x7FFFu + ((b >> 16) & 1u)) >> 16;
}

__device__ __forceinline__ float f16_to_f32(uint32_t u16) {
  _Float16 h;
  uint16_t v = (uint16_t)u16;
  __builtin_memcpy(&h, &v, 2);
  return (float)h;                      // exact for every finite f16 pattern
}

// ------------------------------------------------------------------------- wave64 reductions --
// DPP data movement (gfx9 encodings): quad_perm xor1 = 0xB1, xor2 = 0x4E, row_half_mirror 0x141,
// row_mirror 0x140 (inside a 16-lane row), row_bcast15 0x142 / row_bcast31 0x143 (across rows).
// A butterfly over them costs a few cycles per step, where a __shfl_xor goes through the LDS
// crossbar (ds_bpermute) at LDS latency.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROW_MASK, 0xF, true);
}
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_f32(float v) {
  return __uint_as_float(dpp_u32<CTRL, ROW_MASK>(__float_as_uint(v)));
}
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ double dpp_f64(double v) {
  const uint64_t b = __double_as_longlong(v);
  const uint64_t lo = dpp_u32<CTRL, ROW_MASK>((uint32_t)b);
  const uint64_t hi = dpp_u32<CTRL, ROW_MASK>((uint32_t)(b >> 32));
  return __longlong_as_double((long long)(lo | (hi << 32)));
}
__device__ __forceinline__ float readlane_f32(float v, int l) {
  return __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(v), l));
}

// sum over each 16-lane row, result in every lane of the row
__device__ __forceinline__ float row16_sum_f32(float v) {
  v += dpp_f32<0xB1>(v);
  v += dpp_f32<0x4E>(v);
  v += dpp_f32<0x141>(v);
  v += dpp_f32<0x140>(v);
  return v;
}
// sum over the wave, result in every lane
__device__ __forceinline__ float wave_sum_f32(float v) {
  v = row16_sum_f32(v);
  v += dpp_f32<0x142, 0xA>(v);     // rows 1, 3 += last lane of rows 0, 2
  v += dpp_f32<0x143, 0xC>(v);     // rows 2, 3 += lane 31
  return readlane_f32(v, 63);
}
__device__ __forceinline__ float wave_max_f32(float v) {
  v = fmaxf(v, dpp_f32<0xB1>(v));
  v = fmaxf(v, dpp_f32<0x4E>(v));
  v = fmaxf(v, dpp_f32<0x141>(v));
  v = fmaxf(v, dpp_f32<0x140>(v));
  // rows 0/2 keep their own value where the broadcast is masked off (the row_mask keeps `old`
  // = 0 there, and fmaxf with a row's own max leaves it unchanged only for non-negative rows),
  // so combine rows through readlane instead
  const float r0 = readlane_f32(v, 15), r1 = readlane_f32(v, 31);
  const float r2 = readlane_f32(v, 47), r3 = readlane_f32(v, 63);
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}
__device__ __forceinline__ double wave_sum_f64(double v) {
  v += dpp_f64<0xB1>(v);
  v += dpp_f64<0x4E>(v);
  v += dpp_f64<0x141>(v);
  v += dpp_f64<0x140>(v);
  v += dpp_f64<0x142, 0xA>(v);
  v += dpp_f64<0x143, 0xC>(v);
  const uint64_t b = __double_as_longlong(v);
  const uint64_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, 63);
  const uint64_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), 63);
  return __longlong_as_double((long long)(lo | (hi << 32)));
}

// The same sums without the scalar hop (a readlane and its SALU consumers cost ~60 cycles): after
// the row sums, gfx950's lane swaps add rows i ^ 16, then halves i ^ 32. Every lane ends with
// (r0 + r1) + (r2 + r3) up to the order of the operands of each addition, the value wave_sum_*
// reads from lane 63 ((r3 + r2) + (r1 + r0)): the same bits.
__device__ __forceinline__ float wave_sum_f32_v(float v) {
  v = row16_sum_f32(v);
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}
__device__ __forceinline__ double swap_add_f64_16(double v) {
  const uint64_t u = __double_as_longlong(v);
  const auto lo = __builtin_amdgcn_permlane16_swap((uint32_t)u, (uint32_t)u, false, false);
  const auto hi = __builtin_amdgcn_permlane16_swap((uint32_t)(u >> 32), (uint32_t)(u >> 32), false, false);
  return __longlong_as_double((long long)((uint64_t)lo[0] | ((uint64_t)hi[0] << 32))) +
         __longlong_as_double((long long)((uint64_t)lo[1] | ((uint64_t)hi[1] << 32)));
}
__device__ __forceinline__ double swap_add_f64_32(double v) {
  const uint64_t u = __double_as_longlong(v);
  const auto lo = __builtin_amdgcn_permlane32_swap((uint32_t)u, (uint32_t)u, false, false);
  const auto hi = __builtin_amdgcn_permlane32_swap((uint32_t)(u >> 32), (uint32_t)(u >> 32), false, false);
  return __longlong_as_double((long long)((uint64_t)lo[0] | ((uint64_t)hi[0] << 32))) +
         __longlong_as_double((long long)((uint64_t)lo[1] | ((uint64_t)hi[1] << 32)));
}
__device__ __forceinline__ double wave_sum_f64_v(double v) {
  v += dpp_f64<0xB1>(v);
  v += dpp_f64<0x4E>(v);
  v += dpp_f64<0x141>(v);
  v += dpp_f64<0x140>(v);
  return swap_add_f64_32(swap_add_f64_16(v));
}

// Maximum over the wave, in every lane, without a scalar round trip (a VALU -> SGPR -> SALU hop
// costs ~60 cycles): DPP maxima inside each 16-lane row, then gfx950's lane swaps, whose two
// results hold lanes i and i ^ 16 (i ^ 32) of the value in either order.
__device__ __forceinline__ uint32_t wave_max_u32_v(uint32_t v) {
  v = max(v, dpp_u32<0xB1>(v));
  v = max(v, dpp_u32<0x4E>(v));
  v = max(v, dpp_u32<0x141>(v));
  v = max(v, dpp_u32<0x140>(v));
  const auto a = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  v = max(a[0], a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return max(b[0], b[1]);
}

__device__ __forceinline__ float silu_f32(float z) { return z / (1.0f + __expf(-z)); }

// ------------------------------------------------------------------- the combine's roundings --
// The block's final sums round every product and every sum to f32 on its own, as the reference's
// torch ops do (speccheck/moe_ref.py:466-474: prod = raw * w, then acc += prod;
// engine/m3_forward.py:464, 475, 737): out = x1 + (routed + gate * shared_raw). The contraction
// pragma keeps the compiler from fusing a product into the following add (an FMA rounds once).
// acc + w * v with the product rounded first
__device__ __forceinline__ float comb_madd(float acc, float w, float v) {
#pragma clang fp contract(off)
  const float p = w * v;
  return acc + p;
}
// residual + (routed + gate * shared_raw), the residual NaN-free zero when absent
__device__ __forceinline__ float comb_out(float resid, float routed, float gate, float sraw) {
#pragma clang fp contract(off)
  const float sh = gate * sraw;
  return resid + (routed + sh);
}

// ----------------------------------------------------------------------------- Q4_K element --
// 144-byte super-block: f16 d | f16 dmin | 12 B packed 6-bit (sc, m) x 8 | 128 B nibbles.
// get_scale_min_k4 (tools/gguf_reader.py:165-175), with the 12 scale bytes held as 3 dwords
// s0 = bytes 0..3, s1 = 4..7, s2 = 8..11:
//   j < 4 : sc = byte(s0, j) & 63,                          m = byte(s1, j) & 63
//   j >= 4: sc = (byte(s2, j-4) & 15) | ((byte(s0, j-4) >> 6) << 4)
//           m  = (byte(s2, j-4) >> 4) | ((byte(s1, j-4) >> 6) << 4)
__device__ __forceinline__ void q4k_scale_min(uint32_t s0, uint32_t s1, uint32_t s2, int j,
                                              uint32_t& sc, uint32_t& m) {
  if (j < 4) {
    sc = (s0 >> (8 * j)) & 63u;
    m = (s1 >> (8 * j)) & 63u;
  } else {
    const int b = 8 * (j - 4);
    const uint32_t hi = (s2 >> b) & 0xFFu;
    sc = (hi & 15u) | (((s0 >> b) >> 6 & 3u) << 4);
    m = (hi >> 4) | (((s1 >> b) >> 6 & 3u) << 4);
  }
}

// Q6_K (210-byte super-block): ql[128] | qh[64] | int8 sc[16] | f16 d at byte 208.
// Element e = 128g + 32k + l: q = ((ql[64g+32(k&1)+l] >> 4(k>>1)) & 15) | (((qh[32g+l] >> 2k) & 3)
// << 4), value = d * sc[8g + 2k + (l>>4)] * (q - 32)   (tools/gguf_reader.py:299-322).
