// Post-attention RMSNorm in front of the block (Form A, engine/m3_forward.py:303-307, :732-733):
// xn = (x * r) * w with r = f32(1 / sqrt(mean(x^2) + eps)), the mean and the reciprocal square
// root evaluated in f64 (every square is exact in f64) and rounded once to f32. The artifact's
// (1 + w) is already in w. One 256-thread block per token row, f32 output.
#include "common.h"
#include "moe_internal.h"

namespace moe {

template <int XDT>
__global__ __launch_bounds__(256) void k_rmsnorm(const void* x, int H, const float* w, float eps,
                                                  float* out) {
  __shared__ double s_red[4];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const size_t row = (size_t)blockIdx.x * H;
  double ss = 0.0;
  for (int j = t; j < H; j += 256) {
    const double v = XDT == MOE_DT_F32 ? (double)reinterpret_cast<const float*>(x)[row + j]
                                       : (double)bf16_to_f32(reinterpret_cast<const uint16_t*>(x)[row + j]);
    ss += v * v;
  }
  ss = wave_sum_f64(ss);
  if (lane == 0) s_red[wave] = ss;
  __syncthreads();
  const double tot = ((s_red[0] + s_red[1]) + s_red[2]) + s_red[3];
  const float r = (float)(1.0 / sqrt(tot / (double)H + (double)eps));
  for (int j = t; j < H; j += 256) {
    const float v = XDT == MOE_DT_F32 ? reinterpret_cast<const float*>(x)[row + j]
                                      : bf16_to_f32(reinterpret_cast<const uint16_t*>(x)[row + j]);
    out[row + j] = (v * r) * w[j];
  }
}

}  // namespace moe

using namespace moe;

int moe_launch_rmsnorm(const void* x, int x_dtype, int T, int H, const float* w, float eps,
                       float* out, hipStream_t st) {
  if (x_dtype == MOE_DT_F32)
    hipLaunchKernelGGL(k_rmsnorm<MOE_DT_F32>, dim3(T), dim3(256), 0, st, x, H, w, eps, out);
  else
    hipLaunchKernelGGL(k_rmsnorm<MOE_DT_BF16>, dim3(T), dim3(256), 0, st, x, H, w, eps, out);
  return moe_check_launch("rmsnorm");
}
