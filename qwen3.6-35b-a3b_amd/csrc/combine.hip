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
                                                 const float* __restrict__ gate_prob, int T,
                                                 int K, int H, float* __restrict__ out,
                                                 float* __restrict__ routed_sum,
                                                 float* __restrict__ shared_out,
                                                 float* __restrict__ expert_raw) {
  const int t = blockIdx.x;
  const int h = blockIdx.y * 256 + threadIdx.x;
  if (h >= H) return;
  int order[16];
  int kid[16];
  for (int k = 0; k < K; ++k) {
    kid[k] = ids[(size_t)t * K + k];
    order[k] = k;
  }
  // insertion sort of slots by expert id (ids within a token are distinct)
  for (int a = 1; a < K; ++a) {
    const int v = order[a];
    int j = a;
    while (j > 0 && kid[order[j - 1]] > kid[v]) {
      order[j] = order[j - 1];
      --j;
    }
    order[j] = v;
  }
  float acc = 0.0f;
  for (int j = 0; j < K; ++j) {
    const int k = order[j];
    const int pos = pair_pos[(size_t)t * K + k];
    const float v = pos >= 0 ? y[(size_t)pos * H + h] : 0.0f;   // dropped (out-of-range) id
    acc += bf16_to_f32(w_bf16[(size_t)t * K + k]) * v;
    if (expert_raw) expert_raw[((size_t)t * K + k) * H + h] = v;
  }
  const float sh = gate_prob[t] * shared_raw[(size_t)t * H + h];
  if (routed_sum) routed_sum[(size_t)t * H + h] = acc;
  if (shared_out) shared_out[(size_t)t * H + h] = sh;
  out[(size_t)t * H + h] = acc + sh;
}

}  // namespace moe

using namespace moe;

int moe_launch_combine(const float* y, const int32_t* pair_pos, const int32_t* ids,
                       const uint16_t* w_bf16, const float* shared_raw, const float* gate_prob,
                       int T, int K, int H, float* out, float* routed_sum, float* shared_out,
                       float* expert_raw, hipStream_t st) {
  dim3 grid(T, (H + 255) / 256);
  hipLaunchKernelGGL(k_combine, grid, dim3(256), 0, st, y, pair_pos, ids, w_bf16, shared_raw,
                     gate_prob, T, K, H, out, routed_sum, shared_out, expert_raw);
  return moe_check_launch("combine");
}
