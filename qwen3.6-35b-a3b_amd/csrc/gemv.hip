// Decode-path expert contraction: fused Q4_K / Q5_K / Q6_K super-block decode + f32 GEMV, one pass over
// each hit expert's bytes (engine/m3_forward.py:452-463; speccheck/moe_ref.py:367-392).
//
// Q4_K gate_up (rows of H = 8 blocks x 144 B): a wave covers one full 2048-wide row per step,
// lane = 8*block + chunk, so each lane keeps the same 32 activations in registers for every row:
// chunk c of a block is qs bytes [16c, 16c+16), i.e. elements 64(c>>1) + 16(c&1) + i (low
// nibbles, sub-block 2(c>>1)) and the same +32 (high nibbles, sub-block 2(c>>1)+1). The row dot is
//   sum_sub d*sc_j * sum(q x) - dmin*m_j * sum(x)
// so the min term costs one multiply per 16 elements. gate row i and up row i (gate first,
// spec §11.4: rows i and I + i of a fused record, or row i of the separate gate and up tensors)
// are contracted together and s = silu(gate)*up is written in f32.
//
// down (rows of I = 512 = 2 blocks): 16 lanes per row, 4 rows per wave step.
#include "common.h"
#include "moe_internal.h"
#include "gemv_dev.h"

namespace moe {

// grid (I/16, max_hits), block 256; wave w handles intermediate rows i0 = 16*bx + 4w .. +4
template <int XDT>
__global__ __launch_bounds__(256) void k_gemv_gateup_q4k(
    const void* __restrict__ x, const uint8_t* __restrict__ gate, const uint8_t* __restrict__ up,
    size_t estride, const int32_t* __restrict__ offsets, const int32_t* __restrict__ sorted_pairs,
    const int32_t* __restrict__ hit_list, int H, int I, int K, float* __restrict__ S) {
  const int hidx = blockIdx.y;
  if (hidx >= hit_list[0]) return;
  const int e = hit_list[1 + hidx];
  const int p0 = offsets[e], p1 = offsets[e + 1];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int b = lane >> 3, c = lane & 7, g = c >> 1, l0 = 16 * (c & 1);
  const size_t rowb = (size_t)(H / 256) * 144;
  const uint8_t* gbase = gate + (size_t)e * estride;
  const uint8_t* ubase = up + (size_t)e * estride;
  const int i0 = blockIdx.x * 16 + wave * 4;
  const int nbg = H / 2048;
  for (int q = p0; q < p1; ++q) {
    const int t = sorted_pairs[q] / K;
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int bg = 0; bg < nbg; ++bg) {
      const int blk = bg * 8 + b;
      float xl[16], xh[16];
      load_x32<XDT>(x, (size_t)t * H + 256 * blk + 64 * g + l0, xl, xh);
      float sxl = 0.0f, sxh = 0.0f;
#pragma unroll
      for (int i = 0; i < 16; ++i) { sxl += xl[i]; sxh += xh[i]; }
      uint4 hdr[8], qs[8];
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const uint8_t* p = ((r & 1) ? ubase : gbase) + (size_t)(i0 + (r >> 1)) * rowb + (size_t)blk * 144;
        hdr[r] = *reinterpret_cast<const uint4*>(p);
        qs[r] = *reinterpret_cast<const uint4*>(p + 16 + 16 * c);
      }
#pragma unroll
      for (int r = 0; r < 8; ++r) acc[r] += q4k_chunk_dot(hdr[r], qs[r], g, xl, xh, sxl, sxh);
    }
#pragma unroll
    for (int r = 0; r < 8; ++r) acc[r] = wave_sum_f32(acc[r]);
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (lane == r) S[(size_t)q * I + i0 + r] = silu_f32(acc[2 * r]) * acc[2 * r + 1];
  }
}

// ----------------------------------------------------------------------- down, Q4_K / Q5_K --
// grid (H/64, max_hits); wave w: rows 64*bx + 16w + 4*step + (lane>>4), step 0..3. Q5_K rows
// (176-byte blocks) add the lane's 16 qh bytes to the Q4_K chunk.
template <int FMT>
__global__ __launch_bounds__(256) void k_gemv_down_k(const float* __restrict__ S,
                                                        const uint8_t* __restrict__ dn,
                                                        const int32_t* __restrict__ offsets,
                                                        const int32_t* __restrict__ hit_list,
                                                        int H, int I, float* __restrict__ y) {
  const int hidx = blockIdx.y;
  if (hidx >= hit_list[0]) return;
  const int e = hit_list[1 + hidx];
  const int p0 = offsets[e], p1 = offsets[e + 1];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15, rsub = lane >> 4;
  const int b = l16 >> 3, c = l16 & 7, g = c >> 1, l0 = 16 * (c & 1);
  constexpr int kBB = FMT == MOE_FMT_Q5_K ? 176 : 144;     // block bytes
  constexpr int kQs = FMT == MOE_FMT_Q5_K ? 48 : 16;       // nibble array offset
  const size_t rowb = (size_t)(I / 256) * kBB;
  const uint8_t* ebase = dn + (size_t)e * H * rowb;
  const int rbase = blockIdx.x * 64 + wave * 16;
  const int nbg = I / 512;
  for (int q = p0; q < p1; ++q) {
    float acc[4] = {0, 0, 0, 0};
    for (int bg = 0; bg < nbg; ++bg) {
      const int blk = bg * 2 + b;
      float xl[16], xh[16];
      load_x32<MOE_DT_F32>(S, (size_t)q * I + 256 * blk + 64 * g + l0, xl, xh);
      float sxl = 0.0f, sxh = 0.0f;
#pragma unroll
      for (int i = 0; i < 16; ++i) { sxl += xl[i]; sxh += xh[i]; }
      uint4 hdr[4], qs[4], qh[4];
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const int row = rbase + 4 * st + rsub;
        const uint8_t* p = ebase + (size_t)row * rowb + (size_t)blk * kBB;
        hdr[st] = *reinterpret_cast<const uint4*>(p);
        qs[st] = *reinterpret_cast<const uint4*>(p + kQs + 16 * c);
        if (FMT == MOE_FMT_Q5_K) qh[st] = *reinterpret_cast<const uint4*>(p + 16 + l0);
      }
#pragma unroll
      for (int st = 0; st < 4; ++st)
        acc[st] += FMT == MOE_FMT_Q5_K ? q5k_chunk_dot(hdr[st], qs[st], qh[st], g, xl, xh, sxl, sxh)
                                       : q4k_chunk_dot(hdr[st], qs[st], g, xl, xh, sxl, sxh);
    }
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      float v = acc[st];
      v = row16_sum_f32(v);
      if (l16 == 0) y[(size_t)q * H + rbase + 4 * st + rsub] = v;
    }
  }
}

// ------------------------------------------------------------------------------ down, Q6_K --
// 210-byte blocks are only 2-byte aligned: read them as 16-bit words.
// Lane (b, c = 4g + k) covers elements 128g + 32k + l, l = 0..31 of block b.
__global__ __launch_bounds__(256) void k_gemv_down_q6k(const float* __restrict__ S,
                                                        const uint8_t* __restrict__ dn,
                                                        const int32_t* __restrict__ offsets,
                                                        const int32_t* __restrict__ hit_list,
                                                        int H, int I, float* __restrict__ y) {
  const int hidx = blockIdx.y;
  if (hidx >= hit_list[0]) return;
  const int e = hit_list[1 + hidx];
  const int p0 = offsets[e], p1 = offsets[e + 1];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15, rsub = lane >> 4;
  const int b = l16 >> 3, c = l16 & 7, g = c >> 2, k = c & 3;
  const size_t rowb = (size_t)(I / 256) * 210;
  const uint8_t* ebase = dn + (size_t)e * H * rowb;
  const int rbase = blockIdx.x * 64 + wave * 16;
  const int nbg = I / 512;
  for (int q = p0; q < p1; ++q) {
    float acc[4] = {0, 0, 0, 0};
    for (int bg = 0; bg < nbg; ++bg) {
      const int blk = bg * 2 + b;
      const float* sp = S + (size_t)q * I + 256 * blk + 128 * g + 32 * k;
      float sv[32];
#pragma unroll
      for (int i = 0; i < 32; i += 4) {
        float4 a = *reinterpret_cast<const float4*>(sp + i);
        sv[i] = a.x; sv[i + 1] = a.y; sv[i + 2] = a.z; sv[i + 3] = a.w;
      }
      float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
      for (int i = 0; i < 16; ++i) { s0 += sv[i]; s1 += sv[16 + i]; }
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const int row = rbase + 4 * st + rsub;
        const uint16_t* p = reinterpret_cast<const uint16_t*>(ebase + (size_t)row * rowb + (size_t)blk * 210);
        const uint16_t* ql = p + (64 * g + 32 * (k & 1)) / 2;
        const uint16_t* qh = p + (128 + 32 * g) / 2;
        const uint32_t scw = p[(192 + 8 * g + 2 * k) / 2];
        const float d = f16_to_f32(p[104]);
        const float ds0 = d * (float)(int8_t)(scw & 0xFFu);
        const float ds1 = d * (float)(int8_t)(scw >> 8);
        const int sh_l = 4 * (k >> 1), sh_h = 2 * k;
        float d0 = 0.0f, d1 = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const uint32_t lw = ql[i], hw = qh[i];
          const uint32_t qa = ((lw >> sh_l) & 15u) | (((hw >> sh_h) & 3u) << 4);
          const uint32_t qb = (((lw >> 8) >> sh_l) & 15u) | ((((hw >> 8) >> sh_h) & 3u) << 4);
          if (i < 8) {
            d0 = fmaf(sv[2 * i], (float)qa, d0);
            d0 = fmaf(sv[2 * i + 1], (float)qb, d0);
          } else {
            d1 = fmaf(sv[2 * i], (float)qa, d1);
            d1 = fmaf(sv[2 * i + 1], (float)qb, d1);
          }
        }
        acc[st] += ds0 * (d0 - 32.0f * s0) + ds1 * (d1 - 32.0f * s1);
      }
    }
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      float v = acc[st];
      v = row16_sum_f32(v);
      if (l16 == 0) y[(size_t)q * H + rbase + 4 * st + rsub] = v;
    }
  }
}

}  // namespace moe

using namespace moe;

int moe_launch_gemv_gateup(const void* x, int x_dtype, const void* gate, const void* up, size_t estride,
                           int fmt, const int32_t* offsets, const int32_t* sorted_pairs,
                           const int32_t* hit_list, int max_hits, int H, int I, int K, float* S,
                           hipStream_t st) {
  if (fmt != MOE_FMT_Q4_K)
    return moe_set_error(MOE_E_FORMAT, "GEMV gate_up supports Q4_K only (got %d)", fmt);
  if (H % 2048 || I % 16)
    return moe_set_error(MOE_E_UNSUPPORTED, "GEMV gate_up needs H %% 2048 == 0, I %% 16 == 0");
  dim3 grid(I / 16, max_hits);
  const uint8_t* g = reinterpret_cast<const uint8_t*>(gate);
  const uint8_t* u = reinterpret_cast<const uint8_t*>(up);
  if (x_dtype == MOE_DT_F32)
    hipLaunchKernelGGL(k_gemv_gateup_q4k<MOE_DT_F32>, grid, dim3(256), 0, st, x, g, u, estride, offsets, sorted_pairs, hit_list, H, I, K, S);
  else
    hipLaunchKernelGGL(k_gemv_gateup_q4k<MOE_DT_BF16>, grid, dim3(256), 0, st, x, g, u, estride, offsets, sorted_pairs, hit_list, H, I, K, S);
  return moe_check_launch("gemv_gateup");
}

int moe_launch_gemv_down(const float* S, const void* dn, int fmt, const int32_t* offsets,
                         const int32_t* hit_list, int max_hits, int H, int I, float* y,
                         hipStream_t st) {
  if (H % 64 || I % 512)
    return moe_set_error(MOE_E_UNSUPPORTED, "GEMV down needs H %% 64 == 0, I %% 512 == 0");
  dim3 grid(H / 64, max_hits);
  const uint8_t* w = reinterpret_cast<const uint8_t*>(dn);
  if (fmt == MOE_FMT_Q4_K)
    hipLaunchKernelGGL(k_gemv_down_k<MOE_FMT_Q4_K>, grid, dim3(256), 0, st, S, w, offsets, hit_list, H, I, y);
  else if (fmt == MOE_FMT_Q5_K)
    hipLaunchKernelGGL(k_gemv_down_k<MOE_FMT_Q5_K>, grid, dim3(256), 0, st, S, w, offsets, hit_list, H, I, y);
  else if (fmt == MOE_FMT_Q6_K)
    hipLaunchKernelGGL(k_gemv_down_q6k, grid, dim3(256), 0, st, S, w, offsets, hit_list, H, I, y);
  else
    return moe_set_error(MOE_E_FORMAT, "GEMV down supports Q4_K / Q5_K / Q6_K (got %d)", fmt);
  return moe_check_launch("gemv_down");
}
