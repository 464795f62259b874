// Shared expert (bf16 or Q8_0 weights) and its scalar sigmoid gate (bf16 or f32 weights), decode path
// (specification/11-moe-block.md §11.6; speccheck/moe_ref.py:480-495; engine/m3_forward.py:436-442).
//   s[t,i] = silu(gate_i . x_t) * (up_i . x_t)        (f32)
//   shared_raw[t,h] = down_h . s[t]                   (f32)
//   gate_prob[t] = sigmoid(wsg . x_t)                 one scalar per token
#include "common.h"
#include "moe_internal.h"
#include "gemv_dev.h"

namespace moe {

// grid (Is/4 + 1); wave w of block bx < Is/4 owns intermediate row i = 4*bx + w; the last block's
// wave 0 computes the scalar gate. Rows are H bf16; lane covers cols 512*c + 8*lane + 0..7.
template <int XDT, int SFMT>
__global__ __launch_bounds__(256) void k_shared_gateup(const void* __restrict__ x,
                                                        const void* __restrict__ wg,
                                                        const void* __restrict__ wu,
                                                        const void* __restrict__ wsg, int gdt, int T,
                                                        int H, int Is, float* __restrict__ s,
                                                        float* __restrict__ gate_prob) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nc = H / 512;
  if (blockIdx.x == Is / 4) {
    if (wave != 0 || gate_prob == nullptr) return;
    for (int t = 0; t < T; ++t) {
      float a = 0.0f;
      for (int c = 0; c < nc; ++c) {
        float xv[8];
        load_x8<XDT>(x, (size_t)t * H + 512 * c + 8 * lane, xv);
        a += dot8_w(wsg, (size_t)512 * c + 8 * lane, gdt, xv);
      }
      a = wave_sum_f32(a);
      if (lane == 0) gate_prob[t] = 1.0f / (1.0f + expf(-a));
    }
    return;
  }
  const int i = blockIdx.x * 4 + wave;
  for (int t = 0; t < T; ++t) {
    float ag = 0.0f, au = 0.0f;
    for (int c = 0; c < nc; ++c) {
      float xv[8];
      load_x8<XDT>(x, (size_t)t * H + 512 * c + 8 * lane, xv);
      ag += dot8_shared<SFMT>(wg, i, H, 512 * c + 8 * lane, xv);
      au += dot8_shared<SFMT>(wu, i, H, 512 * c + 8 * lane, xv);
    }
    ag = wave_sum_f32(ag);
    au = wave_sum_f32(au);
    if (lane == 0) s[(size_t)t * Is + i] = silu_f32(ag) * au;
  }
}

// grid (H/16); wave w owns rows 16*bx + 4w + (lane>>4); 16 lanes per row of Is weights
template <int SFMT>
__global__ __launch_bounds__(256) void k_shared_down(const float* __restrict__ s,
                                                      const void* __restrict__ wd, int T,
                                                      int H, int Is,
                                                      float* __restrict__ shared_raw) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15;
  const int row = blockIdx.x * 16 + wave * 4 + (lane >> 4);
  const int nc = Is / 128;
  for (int t = 0; t < T; ++t) {
    float a = 0.0f;
    for (int c = 0; c < nc; ++c) {
      float sv[8];
      load_x8<MOE_DT_F32>(s, (size_t)t * Is + 128 * c + 8 * l16, sv);
      a += dot8_shared<SFMT>(wd, row, Is, 128 * c + 8 * l16, sv);
    }
    a = row16_sum_f32(a);
    if (l16 == 0) shared_raw[(size_t)t * H + row] = a;
  }
}

// f16 RNE of two values saturated to +-65504, packed (k_to_f16's conversion)
__device__ __forceinline__ uint32_t f16x2_sat_pk(float u, float v) {
  u = fminf(fmaxf(u, -65504.0f), 65504.0f);
  v = fminf(fmaxf(v, -65504.0f), 65504.0f);
  return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)u) |
         ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v) << 16);
}

// scalar gate only (used beside the MFMA path): one wave per token. With x16 given, the wave also
// writes its token's f16 row (same bits as k_to_f16), since it reads the whole row anyway.
template <int XDT>
__global__ __launch_bounds__(64) void k_shared_gate(const void* __restrict__ x,
                                                     const void* __restrict__ wsg, int gdt, int T,
                                                     int H, float* __restrict__ gate_prob,
                                                     uint16_t* __restrict__ x16) {
  const int t = blockIdx.x, lane = threadIdx.x;
  float a = 0.0f;
  for (int c = 0; c < H / 512; ++c) {
    float xv[8];
    const size_t o = (size_t)t * H + 512 * c + 8 * lane;
    load_x8<XDT>(x, o, xv);
    if (x16)
      *reinterpret_cast<uint4*>(x16 + o) = make_uint4(f16x2_sat_pk(xv[0], xv[1]), f16x2_sat_pk(xv[2], xv[3]),
                                                      f16x2_sat_pk(xv[4], xv[5]), f16x2_sat_pk(xv[6], xv[7]));
    a += dot8_w(wsg, (size_t)512 * c + 8 * lane, gdt, xv);
  }
  a = wave_sum_f32(a);
  if (lane == 0) gate_prob[t] = 1.0f / (1.0f + expf(-a));
}

}  // namespace moe

using namespace moe;

template <int SFMT>
static void launch_shared_gemv(const void* x, int x_dtype, const void* g, const void* u, const void* d,
                               const void* wsg, int gate_dtype, int T, int H, int Is, float* s_tmp,
                               float* shared_raw, float* gate_prob, hipStream_t st) {
  if (x_dtype == MOE_DT_F32)
    hipLaunchKernelGGL((k_shared_gateup<MOE_DT_F32, SFMT>), dim3(Is / 4 + 1), dim3(256), 0, st, x, g, u, wsg, gate_dtype, T, H, Is, s_tmp, gate_prob);
  else
    hipLaunchKernelGGL((k_shared_gateup<MOE_DT_BF16, SFMT>), dim3(Is / 4 + 1), dim3(256), 0, st, x, g, u, wsg, gate_dtype, T, H, Is, s_tmp, gate_prob);
  hipLaunchKernelGGL(k_shared_down<SFMT>, dim3(H / 16), dim3(256), 0, st, s_tmp, d, T, H, Is, shared_raw);
}

int moe_launch_shared_gemv(const void* x, int x_dtype, const void* wg, const void* wu,
                           const void* wd, int shared_fmt, const void* wsg, int gate_dtype, int T,
                           int H, int Is, float* s_tmp, float* shared_raw, float* gate_prob,
                           hipStream_t st) {
  if (H % 512 || Is % 128 || H % 16 || Is % 4)
    return moe_set_error(MOE_E_UNSUPPORTED, "shared GEMV needs H %% 512 == 0, Is %% 128 == 0");
  if (shared_fmt == MOE_FMT_Q8_0)
    launch_shared_gemv<MOE_FMT_Q8_0>(x, x_dtype, wg, wu, wd, wsg, gate_dtype, T, H, Is, s_tmp, shared_raw, gate_prob, st);
  else
    launch_shared_gemv<MOE_FMT_BF16>(x, x_dtype, wg, wu, wd, wsg, gate_dtype, T, H, Is, s_tmp, shared_raw, gate_prob, st);
  return moe_check_launch("shared_gemv");
}

int moe_launch_shared_gate(const void* x, int x_dtype, const void* wsg, int gate_dtype, int T, int H,
                           float* gate_prob, hipStream_t st, uint16_t* x16) {
  if (x_dtype == MOE_DT_F32)
    hipLaunchKernelGGL(k_shared_gate<MOE_DT_F32>, dim3(T), dim3(64), 0, st, x, wsg, gate_dtype, T, H, gate_prob, x16);
  else
    hipLaunchKernelGGL(k_shared_gate<MOE_DT_BF16>, dim3(T), dim3(64), 0, st, x, wsg, gate_dtype, T, H, gate_prob, x16);
  return moe_check_launch("shared_gate");
}
