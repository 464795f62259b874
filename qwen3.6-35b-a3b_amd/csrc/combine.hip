// Top-K weighted combine + gated shared expert (specification/11-moe-block.md §11.5-§11.6;
// speccheck/moe_ref.py:452-476, 516-518; engine/block_forward.py:664-667, 680):
//   routed[t,h] = sum over the token's K experts in ascending expert id of
//                 f32(w_bf16[t, rank]) * y[pair_pos[t*K + rank], h]       (f32, fixed order)
//   out[t,h]    = residual[t,h] + (routed[t,h] + gate_prob[t] * shared_raw[t,h])
// every product and sum rounded to f32 on its own (comb_madd / comb_out, common.h)
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
    acc = comb_madd(acc, s_w[k], v);
    if (expert_raw) expert_raw[((size_t)t * K + k) * H + h] = v;
  }
  const float gp = gate_prob[t], sr = shared_raw[(size_t)t * H + h];
  if (routed_sum) routed_sum[(size_t)t * H + h] = acc;
  if (shared_out) shared_out[(size_t)t * H + h] = gp * sr;
  out[(size_t)t * H + h] = comb_out(residual ? residual[(size_t)t * H + h] : 0.0f, acc, gp, sr);
}

// Same sums, four columns per thread (H % 4 == 0) and a compile-time K: the K expert rows are
// all in flight before the first add, and the ascending-id order comes from per-slot ranks
// (ids within a token are distinct; equal ids would keep slot order) instead of a serial sort.
// grid = (T, ceil(H / 1024)), block = 256.
template <int KK, bool Y16>
__global__ __launch_bounds__(256) void k_combine4(const void* __restrict__ y,
                                                  const int32_t* __restrict__ pair_pos,
                                                  const int32_t* __restrict__ ids,
                                                  const uint16_t* __restrict__ w_bf16,
                                                  const float* __restrict__ shared_raw,
                                                  const float* __restrict__ gate_prob,
                                                  const float* __restrict__ residual, int T,
                                                  int H, float* __restrict__ out,
                                                  float* __restrict__ routed_sum,
                                                  float* __restrict__ shared_out,
                                                  float* __restrict__ expert_raw) {
  __shared__ int s_pos[KK], s_slot[KK];
  __shared__ float s_w[KK];
  const int t = blockIdx.x;
  if (threadIdx.x < KK) {
    const int k = threadIdx.x;
    const int32_t* tid = ids + (size_t)t * KK;
    const int id = tid[k];
    int rank = 0;
#pragma unroll
    for (int j = 0; j < KK; ++j) {
      const int o = tid[j];
      rank += (o < id) || (o == id && j < k);
    }
    s_pos[rank] = pair_pos[(size_t)t * KK + k];
    s_slot[rank] = k;
    s_w[rank] = bf16_to_f32(w_bf16[(size_t)t * KK + k]);
  }
  __syncthreads();
  const int h = (blockIdx.y * 256 + threadIdx.x) * 4;
  if (h >= H) return;
  float4 v[KK];
#pragma unroll
  for (int j = 0; j < KK; ++j) {
    const int pos = s_pos[j];
    if (pos < 0) {
      v[j] = make_float4(0.f, 0.f, 0.f, 0.f);                // dropped (out-of-range) id
    } else if constexpr (Y16) {
      const uint2 q = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(y) + (size_t)pos * H + h);
      v[j] = make_float4(f16_to_f32(q.x & 0xFFFFu), f16_to_f32(q.x >> 16), f16_to_f32(q.y & 0xFFFFu),
                         f16_to_f32(q.y >> 16));
    } else {
      v[j] = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(y) + (size_t)pos * H + h);
    }
  }
  const size_t o = (size_t)t * H + h;
  const float4 sr = *reinterpret_cast<const float4*>(shared_raw + o);
  const float4 rs = residual ? *reinterpret_cast<const float4*>(residual + o) : make_float4(0.f, 0.f, 0.f, 0.f);
  const float gp = gate_prob[t];
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int j = 0; j < KK; ++j) {
    const float w = s_w[j];
    acc.x = comb_madd(acc.x, w, v[j].x);
    acc.y = comb_madd(acc.y, w, v[j].y);
    acc.z = comb_madd(acc.z, w, v[j].z);
    acc.w = comb_madd(acc.w, w, v[j].w);
    if (expert_raw)
      *reinterpret_cast<float4*>(expert_raw + ((size_t)t * KK + s_slot[j]) * H + h) = v[j];
  }
  const float4 sh = make_float4(gp * sr.x, gp * sr.y, gp * sr.z, gp * sr.w);
  if (routed_sum) *reinterpret_cast<float4*>(routed_sum + o) = acc;
  if (shared_out) *reinterpret_cast<float4*>(shared_out + o) = sh;
  *reinterpret_cast<float4*>(out + o) =
      make_float4(comb_out(rs.x, acc.x, gp, sr.x), comb_out(rs.y, acc.y, gp, sr.y),
                  comb_out(rs.z, acc.z, gp, sr.z), comb_out(rs.w, acc.w, gp, sr.w));
}


// The block forward's f16 rows, eight columns per thread (H % 8 == 0): one 16-byte non-temporal
// load per expert row (each row is read once), the same sums in the same order as k_combine4.
// grid = (T, ceil(H / 2048)), block = 256.
template <int KK>
__global__ __launch_bounds__(256) void k_combine8(const void* __restrict__ y,
                                                  const int32_t* __restrict__ pair_pos,
                                                  const int32_t* __restrict__ ids,
                                                  const uint16_t* __restrict__ w_bf16,
                                                  const float* __restrict__ shared_raw,
                                                  const float* __restrict__ gate_prob,
                                                  const float* __restrict__ residual, int T,
                                                  int H, float* __restrict__ out,
                                                  float* __restrict__ routed_sum,
                                                  float* __restrict__ shared_out,
                                                  float* __restrict__ expert_raw) {
  __shared__ int s_pos[KK], s_slot[KK];
  __shared__ float s_w[KK];
  const int t = blockIdx.x;
  if (threadIdx.x < KK) {
    const int k = threadIdx.x;
    const int32_t* tid = ids + (size_t)t * KK;
    const int id = tid[k];
    int rank = 0;
#pragma unroll
    for (int j = 0; j < KK; ++j) {
      const int o = tid[j];
      rank += (o < id) || (o == id && j < k);
    }
    s_pos[rank] = pair_pos[(size_t)t * KK + k];
    s_slot[rank] = k;
    s_w[rank] = bf16_to_f32(w_bf16[(size_t)t * KK + k]);
  }
  __syncthreads();
  const int h = (blockIdx.y * 256 + threadIdx.x) * 8;
  if (h >= H) return;
  typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
  u32x4v q[KK];
#pragma unroll
  for (int j = 0; j < KK; ++j) {
    const int pos = s_pos[j];
    q[j] = pos < 0 ? (u32x4v){0u, 0u, 0u, 0u}
                   : __builtin_nontemporal_load(reinterpret_cast<const u32x4v*>(reinterpret_cast<const uint16_t*>(y) + (size_t)pos * H + h));
  }
  const size_t o = (size_t)t * H + h;
  const float4 sr0 = *reinterpret_cast<const float4*>(shared_raw + o);
  const float4 sr1 = *reinterpret_cast<const float4*>(shared_raw + o + 4);
  const float4 rs0 = residual ? *reinterpret_cast<const float4*>(residual + o) : make_float4(0.f, 0.f, 0.f, 0.f);
  const float4 rs1 = residual ? *reinterpret_cast<const float4*>(residual + o + 4) : make_float4(0.f, 0.f, 0.f, 0.f);
  const float gp = gate_prob[t];
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < KK; ++j) {
    const float w = s_w[j];
    const uint32_t u[4] = {q[j].x, q[j].y, q[j].z, q[j].w};
    float v[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) { v[2 * i] = f16_to_f32(u[i] & 0xFFFFu); v[2 * i + 1] = f16_to_f32(u[i] >> 16); }
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = comb_madd(acc[i], w, v[i]);
    if (expert_raw) {
      float* er = expert_raw + ((size_t)t * KK + s_slot[j]) * H + h;
      *reinterpret_cast<float4*>(er) = make_float4(v[0], v[1], v[2], v[3]);
      *reinterpret_cast<float4*>(er + 4) = make_float4(v[4], v[5], v[6], v[7]);
    }
  }
  const float sr[8] = {sr0.x, sr0.y, sr0.z, sr0.w, sr1.x, sr1.y, sr1.z, sr1.w};
  const float rs[8] = {rs0.x, rs0.y, rs0.z, rs0.w, rs1.x, rs1.y, rs1.z, rs1.w};
  if (routed_sum) {
    *reinterpret_cast<float4*>(routed_sum + o) = make_float4(acc[0], acc[1], acc[2], acc[3]);
    *reinterpret_cast<float4*>(routed_sum + o + 4) = make_float4(acc[4], acc[5], acc[6], acc[7]);
  }
  if (shared_out) {
    *reinterpret_cast<float4*>(shared_out + o) = make_float4(gp * sr[0], gp * sr[1], gp * sr[2], gp * sr[3]);
    *reinterpret_cast<float4*>(shared_out + o + 4) = make_float4(gp * sr[4], gp * sr[5], gp * sr[6], gp * sr[7]);
  }
  float r[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = comb_out(rs[i], acc[i], gp, sr[i]);
  *reinterpret_cast<float4*>(out + o) = make_float4(r[0], r[1], r[2], r[3]);
  *reinterpret_cast<float4*>(out + o + 4) = make_float4(r[4], r[5], r[6], r[7]);
}

}  // namespace moe

using namespace moe;

int moe_launch_combine(const void* y, int y16, const int32_t* pair_pos, const int32_t* ids,
                       const uint16_t* w_bf16, const float* shared_raw, const float* gate_prob,
                       const float* residual, int T, int K, int H, float* out, float* routed_sum,
                       float* shared_out, float* expert_raw, hipStream_t st) {
  auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  if (y16) {
    // the block forward's f16 rows (its MFMA down GEMMs), always with K == 8 and H % 4 == 0
    if (K != 8 || H % 4 || !a16(y) || !a16(shared_raw) || !a16(residual) || !a16(out) ||
        !a16(routed_sum) || !a16(shared_out) || !a16(expert_raw))
      return moe_set_error(MOE_E_UNSUPPORTED, "combine: f16 expert rows need K == 8, H %% 4 == 0 and 16-byte aligned rows");
    if (H % 8 == 0) {
      dim3 grid(T, (H + 2047) / 2048);
      hipLaunchKernelGGL((k_combine8<8>), grid, dim3(256), 0, st, y, pair_pos, ids, w_bf16,
                         shared_raw, gate_prob, residual, T, H, out, routed_sum, shared_out, expert_raw);
      return moe_check_launch("combine");
    }
    dim3 grid(T, (H + 1023) / 1024);
    hipLaunchKernelGGL((k_combine4<8, true>), grid, dim3(256), 0, st, y, pair_pos, ids, w_bf16,
                       shared_raw, gate_prob, residual, T, H, out, routed_sum, shared_out, expert_raw);
    return moe_check_launch("combine");
  }
  if (K == 8 && H % 4 == 0 && a16(y) && a16(shared_raw) && a16(residual) && a16(out) &&
      a16(routed_sum) && a16(shared_out) && a16(expert_raw)) {
    dim3 grid(T, (H + 1023) / 1024);
    hipLaunchKernelGGL((k_combine4<8, false>), grid, dim3(256), 0, st, y, pair_pos, ids, w_bf16,
                       shared_raw, gate_prob, residual, T, H, out, routed_sum, shared_out, expert_raw);
    return moe_check_launch("combine");
  }
  dim3 grid(T, (H + 255) / 256);
  hipLaunchKernelGGL(k_combine, grid, dim3(256), 0, st, reinterpret_cast<const float*>(y), pair_pos, ids, w_bf16, shared_raw,
                     gate_prob, residual, T, K, H, out, routed_sum, shared_out, expert_raw);
  return moe_check_launch("combine");
}
