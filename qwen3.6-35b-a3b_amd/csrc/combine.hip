// Top-K weighted combine + gated shared expert (specification/11-moe-block.md §11.5-§11.6;
// speccheck/moe_ref.py:452-476, 516-518; engine/block_forward.py:664-667, 680):
//   routed[t,h] = sum over the token's K experts in ascending expert id of
//                 f32(w_bf16[t, rank]) * y[pair_pos[t*K + rank], h]       (f32, fixed order)
//   out[t,h]    = routed[t,h] + gate_prob[t] * shared_raw[t,h]
// The weight is reached through the rank (slot) the expert holds, never through its id.
#include "common.h"
#include "moe_internal.h"

namespace moe {

__global__ __launch_bounds__(256) void k_combine(const float* __restrict__ y,
                                                 const int32_t* __restrict__ pair_pos,
                                                 const int32_t* __restrict__ ids,
                                                 const uint16_t* __restrict__ w_bf16,
                                                 const float* __restrict__ shared_raw,
                                                 const float* __restrict__ gate_prob,
                                                 const float* __restrict__ residual, int T,
                                                 int K, int H, float* __restrict__ out,
                                                 float* __restrict__ routed_sum,
                                                 float* __restrict__ shared_out,
                                                 float* __restrict__ expert_raw) {
  __shared__ int s_id[16], s_pos[16], s_order[16];
  __shared__ float s_w[16];
  const int t = blockIdx.x;
  const int h = blockIdx.y * 256 + threadIdx.x;
  if (threadIdx.x < K) {
    const int k = threadIdx.x;
    s_id[k] = ids[(size_t)t * K + k];
    s_pos[k] = pair_pos[(size_t)t * K + k];
    s_w[k] = bf16_to_f32(w_bf16[(size_t)t * K + k]);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    // slots in ascending expert id (ids within a token are distinct)
    for (int k = 0; k < K; ++k) s_order[k] = k;
    for (int i = 1; i < K; ++i) {
      const int v = s_order[i];
      int j = i;
      while (j > 0 && s_id[s_order[j - 1]] > s_id[v]) {
        s_order[j] = s_order[j - 1];
        --j;
      }
      s_order[j] = v;
    }
  }
  __syncthreads();
  if (h >= H) return;
  float acc = 0.0f;
  for (int j = 0; j < K; ++j) {
    const int k = s_order[j];
    const int pos = s_pos[k];
    const float v = pos >= 0 ? y[(size_t)pos * H + h] : 0.0f;   // dropped (out-of-range) id
    acc += s_w[k] * v;
    if (expert_raw) expert_raw[((size_t)t * K + k) * H + h] = v;
  }
  const float sh = gate_prob[t] * shared_raw[(size_t)t * H + h];
  if (routed_sum) routed_sum[(size_t)t * H + h] = acc;
  if (shared_out) shared_out[(size_t)t * H + h] = sh;
  out[(size_t)t * H + h] = (residual ? residual[(size_t)t * H + h] : 0.0f) + acc + sh;
}

}  // namespace moe

using namespace moe;

int moe_launch_combine(const float* y, const int32_t* pair_pos, const int32_t* ids,
                       const uint16_t* w_bf16, const float* shared_raw, const float* gate_prob,
                       const float* residual, int T, int K, int H, float* out, float* routed_sum,
                       float* shared_out, float* expert_raw, hipStream_t st) {
  dim3 grid(T, (H + 255) / 256);
  hipLaunchKernelGGL(k_combine, grid, dim3(256), 0, st, y, pair_pos, ids, w_bf16, shared_raw,
                     gate_prob, residual, T, K, H, out, routed_sum, shared_out, expert_raw);
  return moe_check_launch("combine");
}
