// The small-T shared expert's dense GEMM pieces (gemm5.hip's own launches, and the blocks the
// routed small-T launches run for it, gemm6.hip): one block per (64-row token tile, narrow weight
// slab), the block's NW waves splitting K into contiguous ranges, each wave holding the tile's two
// 32-row groups for its range in registers (no LDS staging: every operand is used once per block);
// the NW f32 partial tiles meet in LDS and are added in wave order before the epilogue (gate/up:
// SiLU(gate) * up to f16, a slab = 16 gate + the matching 16 up rows in one 32-column MFMA group;
// down: f32 rows, a slab = 32 rows of w_down).
#pragma once
#include "common.h"
#include "gemv_dev.h"

namespace moe {

typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

namespace shs {

constexpr int kBM = 64;                 // token rows per tile
constexpr int kCK = 64;                 // K per register chunk (4 MFMA substeps)
constexpr int kF16 = 2;                 // activation type of f16 rows (beside MOE_DT_F32 / _BF16)

template <bool BF>
__device__ __forceinline__ f32x16_t mfma(uint4 a, uint4 b, f32x16_t c) {
  if constexpr (BF)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                  __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                 __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

// 8 bf16 (16 bytes, element order kept) -> 8 f16, round to nearest even
__device__ __forceinline__ uint32_t bf16x2_to_f16x2(uint32_t d) {
  const _Float16 lo = (_Float16)__uint_as_float(d << 16);
  const _Float16 hi = (_Float16)__uint_as_float(d & 0xFFFF0000u);
  return (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
}
__device__ __forceinline__ uint4 bf16x8_to_f16(uint4 w) {
  return make_uint4(bf16x2_to_f16x2(w.x), bf16x2_to_f16x2(w.y), bf16x2_to_f16x2(w.z),
                    bf16x2_to_f16x2(w.w));
}

// f32 pair -> f16 pair, saturated to +-65504, round to nearest even (k_to_f16's conversion)
__device__ __forceinline__ uint32_t f16x2_sat(float u, float v) {
  u = fminf(fmaxf(u, -65504.0f), 65504.0f);
  v = fminf(fmaxf(v, -65504.0f), 65504.0f);
  return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)u) |
         ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v) << 16);
}

// 8 activations of one row: f32 (32 bytes, converted to f16 at use), bf16 or f16 (16 bytes)
template <int AT>
struct ARaw {
  uint4 v[AT == MOE_DT_F32 ? 2 : 1];
};
template <int AT>
__device__ __forceinline__ void ld_a(ARaw<AT>& r, const uint8_t* p) {
  r.v[0] = *reinterpret_cast<const uint4*>(p);
  if constexpr (AT == MOE_DT_F32) r.v[1] = *reinterpret_cast<const uint4*>(p + 16);
}
template <int AT>
__device__ __forceinline__ uint4 a_frag(const ARaw<AT>& r) {
  if constexpr (AT == MOE_DT_F32)
    return make_uint4(f16x2_sat(__uint_as_float(r.v[0].x), __uint_as_float(r.v[0].y)),
                      f16x2_sat(__uint_as_float(r.v[0].z), __uint_as_float(r.v[0].w)),
                      f16x2_sat(__uint_as_float(r.v[1].x), __uint_as_float(r.v[1].y)),
                      f16x2_sat(__uint_as_float(r.v[1].z), __uint_as_float(r.v[1].w)));
  else
    return r.v[0];
}

// This wave's K range of the tile: rows ar0 (group 0) and ar1 (group 1, TWO) and weight row br at
// the lane's first element; AT's element size es. The K order is permuted inside each 64-wide
// chunk, the same way for both operands: lane half h takes the chunk's elements [32 h, 32 h + 32),
// substep ss the 8 at 32 h + 8 ss. A lane's four substep slices are then one contiguous run, so a
// cache line is consumed by consecutive loads of one wave (in MFMA order, lanes 0-31 and 32-63 of
// a substep taking elements 8 apart, each line was revisited by four loads issued far apart, and
// eight waves' working sets overflowed L1). BF16 activations run
// the bf16 MFMA on the weights as they are, the others the f16 MFMA on converted weights.
template <int AT, bool TWO>
__device__ __forceinline__ void wave_k(const uint8_t* ar0, const uint8_t* ar1, const uint8_t* br,
                                       int nch, f32x16_t& acc0, f32x16_t& acc1) {
  constexpr int es = AT == MOE_DT_F32 ? 4 : 2;
  constexpr bool BF = AT == MOE_DT_BF16;
  ARaw<AT> a0[4], a1[4];
  uint4 b[4];
  auto load = [&](int c, ARaw<AT>(&x0)[4], ARaw<AT>(&x1)[4], uint4(&y)[4]) {
#pragma unroll
    for (int ss = 0; ss < 4; ++ss) {
      const size_t k = (size_t)(c * kCK + 8 * ss);
      y[ss] = *reinterpret_cast<const uint4*>(br + k * 2);
      ld_a<AT>(x0[ss], ar0 + k * es);
      if constexpr (TWO) ld_a<AT>(x1[ss], ar1 + k * es);
    }
  };
  load(0, a0, a1, b);
  for (int c = 0; c < nch; ++c) {
    ARaw<AT> n0[4], n1[4];
    uint4 nb[4];
    if (c + 1 < nch) load(c + 1, n0, n1, nb);
#pragma unroll
    for (int ss = 0; ss < 4; ++ss) {
      const uint4 w = BF ? b[ss] : bf16x8_to_f16(b[ss]);
      acc0 = mfma<BF>(a_frag<AT>(a0[ss]), w, acc0);
      if constexpr (TWO) acc1 = mfma<BF>(a_frag<AT>(a1[ss]), w, acc1);
    }
    if (c + 1 < nch) {
#pragma unroll
      for (int ss = 0; ss < 4; ++ss) {
        a0[ss] = n0[ss];
        if constexpr (TWO) a1[ss] = n1[ss];
        b[ss] = nb[ss];
      }
    }
  }
}

// The block's partial tiles: wave w's element i of group mg at red[((2 w + mg) 16 + i) 64 + lane]
// (element i of lane l: row 8 (i / 4) + 4 (l / 32) + i % 4 of the group, column l % 32).
template <int AT, int NW, int TM = kBM>
__device__ __forceinline__ void tile_k(const void* a, int T, int K, int m0, const uint16_t* brow,
                                       float* red) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int h = lane >> 5, r = lane & 31;
  constexpr int es = AT == MOE_DT_F32 ? 4 : 2;
  const int kw = K / NW, k0 = wave * kw + 32 * h;
  const uint8_t* ab = reinterpret_cast<const uint8_t*>(a);
  const uint8_t* ar0 = ab + ((size_t)min(m0 + r, T - 1) * K + k0) * es;
  const uint8_t* ar1 = ab + ((size_t)min(m0 + 32 + r, T - 1) * K + k0) * es;
  const uint8_t* br = reinterpret_cast<const uint8_t*>(brow + k0);
  f32x16_t acc0 = {}, acc1 = {};
  if (TM > 32 && T - m0 > 32) wave_k<AT, true>(ar0, ar1, br, kw / kCK, acc0, acc1);
  else wave_k<AT, false>(ar0, ar1, br, kw / kCK, acc0, acc1);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    red[((2 * wave) * 16 + i) * 64 + lane] = acc0[i];
    red[((2 * wave + 1) * 16 + i) * 64 + lane] = acc1[i];
  }
  __syncthreads();
}
// sum over the NW waves (in wave order) of tile element (row rr, column c)
template <int NW>
__device__ __forceinline__ float red_sum(const float* red, int rr, int c) {
  const int mg = rr >> 5, q = rr & 31;
  const int idx = (mg * 16 + 4 * (q >> 3) + (q & 3)) * 64 + 32 * ((q >> 2) & 1) + c;
  float s = red[idx];
#pragma unroll
  for (int w = 1; w < NW; ++w) s += red[idx + w * 2 * 16 * 64];
  return s;
}


// LDS floats of one block's partial tiles
template <int NW>
constexpr int red_floats() { return NW * 2 * 16 * 64; }

// Gate/up block: S rows m0 .. m0 + TM - 1 (< T; TM = 64 or 32), columns 16 slab .. 16 slab + 15
// (f16) = SiLU(a wg^T) * (a wu^T) from the activation rows a (type AT) of length H.
template <int AT, int NW, int TM = kBM>
__device__ __forceinline__ void gateup_tile(const void* a, const uint16_t* wg, const uint16_t* wu,
                                            int T, int H, int Is, int slab, int m0,
                                            uint16_t* __restrict__ S, float* red) {
  const int r = threadIdx.x & 31;
  const uint16_t* brow = (r < 16 ? wg : wu) + (size_t)(16 * slab + (r & 15)) * H;
  tile_k<AT, NW, TM>(a, T, H, m0, brow, red);
  // item o: tile row o / 8, S columns 16 slab + 2 (o % 8) + 0..1 (gate at tile column c, up at
  // c + 16)
  for (int o = threadIdx.x; o < TM * 8; o += NW * 64) {
    const int rr = o >> 3, c = 2 * (o & 7);
    if (m0 + rr < T) {
      float v[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const float gv = red_sum<NW>(red, rr, c + j), uv = red_sum<NW>(red, rr, c + j + 16);
        v[j] = gv * __builtin_amdgcn_rcpf(1.0f + __expf(-gv)) * uv;
      }
      *reinterpret_cast<uint32_t*>(S + (size_t)(m0 + rr) * Is + 16 * slab + c) = f16x2_sat(v[0], v[1]);
    }
  }
}

// Down block: y rows m0 .. m0 + TM - 1 (< T), columns 32 slab .. 32 slab + 31 (f32) = S wd^T.
template <int NW, int TM = kBM>
__device__ __forceinline__ void down_tile(const uint16_t* S, const uint16_t* wd, int T, int H, int Is,
                                          int slab, int m0, float* __restrict__ y, float* red) {
  tile_k<kF16, NW, TM>(S, T, Is, m0, wd + (size_t)(32 * slab + (threadIdx.x & 31)) * Is, red);
  // item o: tile row o / 8, columns 32 slab + 4 (o % 8) + 0..3
  for (int o = threadIdx.x; o < TM * 8; o += NW * 64) {
    const int rr = o >> 3, c = 4 * (o & 7);
    if (m0 + rr < T) {
      float4 v;
      v.x = red_sum<NW>(red, rr, c);
      v.y = red_sum<NW>(red, rr, c + 1);
      v.z = red_sum<NW>(red, rr, c + 2);
      v.w = red_sum<NW>(red, rr, c + 3);
      *reinterpret_cast<float4*>(y + (size_t)(m0 + rr) * H + 32 * slab + c) = v;
    }
  }
}

// The scalar gate of tokens gw, gw + nw, ... (< T), one wave each: gate_prob[t] = sigmoid(x . wsg)
// with k_shared_gate's arithmetic (lane partials over the 8-element chunks at 512 c + 8 lane in
// chunk order, one wave sum)
template <int XDT>
__device__ __forceinline__ void gate_rows(const void* x, const void* wsg, int gdt, int T, int H,
                                          float* __restrict__ gate_prob, int gw, int nw) {
  const int lane = threadIdx.x & 63;
  for (int t = gw; t < T; t += nw) {
    float a = 0.0f;
    for (int c = 0; c < H / 512; ++c) {
      float xv[8];
      load_x8<XDT>(x, (size_t)t * H + 512 * c + 8 * lane, xv);
      a += dot8_w(wsg, (size_t)512 * c + 8 * lane, gdt, xv);
    }
    a = wave_sum_f32(a);
    if (lane == 0) gate_prob[t] = 1.0f / (1.0f + expf(-a));
  }
}

}  // namespace shs
}  // namespace moe
