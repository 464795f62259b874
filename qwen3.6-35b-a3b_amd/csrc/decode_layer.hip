// Single-token decode of one MoE block in ONE launch: a persistent grid of 256 workgroups of 8
// waves (one per CU on MI355X, all co-resident) runs the block's three dependent phases and hands data between
// them through epoch-tagged 64-bit words instead of kernel boundaries or device-wide fences.
//
//   phase 1  wg g: router logit e = g (f64, certified bf16) | shared gate/up rows i = 2g, 2g+1 |
//            (wg 0) the scalar shared gate                 -> tagged logits[E], s_shared[I_s], gate
//   phase 2  every wg waits for the 256 logits and runs R2-R5 itself (same answer everywhere; the
//            fast top-k's slot order stands in for torch's when ties sit inside the top 8 and no
//            stage output is asked for: same experts, same weights);
//            wg g: routed gate/up rows of slot k = g/32, i in [16(g%32), +16) -> tagged s_routed;
//            shared down rows 8g..8g+7 (waits for s_shared)
//   phase 3  wg g: down rows 8g..8g+7 of all 8 routed experts (waits for s_routed, read once into
//            LDS), ascending-expert-id combine, gated shared expert, residual -> out[8g..8g+7]
//
// A tagged word is (epoch << 32 | value bits) written by one 64-bit store that bypasses the
// non-coherent L2 (agent-scope relaxed atomic store) and read the same way; a reader spins until
// the tag equals this launch's epoch, so each word validates itself and no store->flag ordering or
// L2 write-back is needed. The epoch lives in the workspace's sync words: every workgroup reads it
// at the start, the last workgroup to finish (arrival counter) advances it, so graph replays work.
// Weights that do not depend on the phase's input are loaded before the wait. Every spin is
// bounded: on a timeout the workgroup records an error bit and carries on (no hang).
#include "common.h"
#include "moe_internal.h"
#include "router_dev.h"
#include "gemv_dev.h"

namespace moe {

constexpr int kG = 256;                 // workgroups (one per CU)
constexpr int kThreads = 512;           // 8 waves
constexpr int kSpinLimit = 1 << 20;     // ~0.1-1 s of polling before giving up

struct LayerArgs {
  const void* x;
  const float* residual;
  const uint16_t* w_router;
  const float* bias;
  const uint8_t* gu;
  const uint8_t* dn;
  const uint16_t* sg;
  const uint16_t* su;
  const uint16_t* sd;
  const uint16_t* ssg;
  int* sync;                            // [0] ticket, [1] epoch, [2] arrivals, [3] error bits
  uint64_t* xch;                        // tagged exchange words
  uint16_t* logits_out;
  int32_t* ids_out;
  float* w_f32_out;
  uint16_t* w_bf16_out;
  float* gate_prob_out;
  float* out;
  float* routed_sum;
  float* shared_out;
  float* expert_raw;
  int exact_order;                      // stage outputs requested: keep torch's slot order
};

// exchange layout (uint64 words)
constexpr int XO_LOGITS = 0;            // 256
constexpr int XO_GATE = 256;            // 1 (+7 pad)
constexpr int XO_SSH = 264;             // 512
constexpr int XO_SR = 776;              // 8 x 512
constexpr int XO_END = 776 + 4096;

__device__ __forceinline__ void tag_store(uint64_t* p, uint32_t epoch, uint32_t bits) {
  __hip_atomic_store(p, ((uint64_t)epoch << 32) | bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t tag_load(uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// value bits of a tagged word once its tag is `epoch` (bounded spin)
__device__ __forceinline__ uint32_t wait_tag(uint64_t* p, uint32_t epoch, int* err) {
  uint64_t v = tag_load(p);
  int spins = 0;
  while ((uint32_t)(v >> 32) != epoch) {
    if (++spins > kSpinLimit) {
      atomicOr(err, 1);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
    v = tag_load(p);
  }
  return (uint32_t)v;
}

// N tagged words p[0], p[stride], ...: all loads issued back to back, then only the words whose
// tag is not yet `epoch` are polled again (bounded). Returns the value bits.
template <int N>
__device__ __forceinline__ void wait_tags(uint64_t* p, int stride, uint32_t epoch, int* err,
                                          uint32_t* out) {
  uint64_t v[N];
#pragma unroll
  for (int j = 0; j < N; ++j) v[j] = tag_load(p + j * stride);
#pragma unroll
  for (int j = 0; j < N; ++j) {
    out[j] = ((uint32_t)(v[j] >> 32) == epoch) ? (uint32_t)v[j] : wait_tag(p + j * stride, epoch, err);
  }
}

template <int XDT>
__global__ __launch_bounds__(kThreads) void k_dec_layer(LayerArgs a) {
  constexpr int H = 2048, I = 512, E = 256, K = 8, IS = 512;
  __shared__ TopkLds tk;
  __shared__ float s_all[K][I];          // routed s vectors, read once per workgroup
  __shared__ int s_ids[K];
  __shared__ float s_w[K];
  __shared__ float s_wf[K];
  __shared__ uint16_t s_wb[K];
  __shared__ int s_order[K];
  __shared__ float sh_raw[8];
  __shared__ float ys[8][K];
  __shared__ float s_gate;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15, g4 = lane >> 4;
  const int g = blockIdx.x;
  int* err = a.sync + 3;
  const uint32_t epoch =
      (uint32_t)__hip_atomic_load(a.sync + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;

  // ------------------------------------------------------------------------------ phase 1 --
  // waves 4, 5: shared-down weights of rows 8g + 4(w-4) + (lane >> 4), used in phase 2
  uint4 sdw[4];
  if (wave == 4 || wave == 5) {
    const uint16_t* dr = a.sd + (size_t)(8 * g + 4 * (wave - 4) + g4) * IS;
#pragma unroll
    for (int c = 0; c < 4; ++c) sdw[c] = *reinterpret_cast<const uint4*>(dr + 128 * c + 8 * l16);
  }
  if (wave < 4) {
    // x at cols 512c + 8 lane (c = 0..3)
    float xv[4][8];
#pragma unroll
    for (int c = 0; c < 4; ++c) load_x8<XDT>(a.x, (size_t)512 * c + 8 * lane, xv[c]);
    if (wave == 0) {
      const uint16_t* wr = a.w_router + (size_t)g * H;
      uint4 wv4[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) wv4[c] = *reinterpret_cast<const uint4*>(wr + 512 * c + 8 * lane);
      double acc = 0.0, xsq = 0.0, wsq = 0.0;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint32_t ww[4] = {wv4[c].x, wv4[c].y, wv4[c].z, wv4[c].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const double w0 = bf16_to_f32(ww[i] & 0xFFFFu), w1 = bf16_to_f32(ww[i] >> 16);
          const double x0 = xv[c][2 * i], x1 = xv[c][2 * i + 1];
          acc = fma(x0, w0, acc);
          acc = fma(x1, w1, acc);
          xsq = fma(x0, x0, xsq);
          xsq = fma(x1, x1, xsq);
          wsq = fma(w0, w0, wsq);
          wsq = fma(w1, w1, wsq);
        }
      }
      acc = wave_sum_f64(acc);
      xsq = wave_sum_f64(xsq);
      wsq = wave_sum_f64(wsq);
      const double bval = a.bias ? (double)a.bias[g] : 0.0;
      const double nrm = sqrt(xsq) * sqrt(wsq) + fabs(bval);
      uint32_t bits;
      if (!round_bf16_certified(acc + bval, 4.0 * (double)(H + 3) * 0x1p-53 * nrm, &bits)) {
        DD d = {0.0, 0.0};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const uint32_t ww[4] = {wv4[c].x, wv4[c].y, wv4[c].z, wv4[c].w};
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const double w_ = bf16_to_f32((i & 1) ? (ww[i >> 1] >> 16) : (ww[i >> 1] & 0xFFFFu));
            d = dd_add(d, DD{(double)xv[c][i] * w_, 0.0});
          }
        }
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) {
          DD other = {__shfl_xor(d.hi, o, 64), __shfl_xor(d.lo, o, 64)};
          d = dd_add(d, other);
        }
        d = dd_add(d, DD{bval, 0.0});
        bits = round_bf16_dd(d, (double)(H + 64) * 0x1p-104 * 16.0 * nrm);
      }
      if (lane == 0) tag_store(a.xch + XO_LOGITS + g, epoch, bits);
    } else if (wave <= 2) {
      const int i = 2 * g + (wave - 1);
      const uint16_t* gr = a.sg + (size_t)i * H;
      const uint16_t* ur = a.su + (size_t)i * H;
      uint4 gw[4], uw[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        gw[c] = *reinterpret_cast<const uint4*>(gr + 512 * c + 8 * lane);
        uw[c] = *reinterpret_cast<const uint4*>(ur + 512 * c + 8 * lane);
      }
      float ag = 0.0f, au = 0.0f;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        ag += dot8_bf16(gw[c], xv[c]);
        au += dot8_bf16(uw[c], xv[c]);
      }
      ag = wave_sum_f32(ag);
      au = wave_sum_f32(au);
      if (lane == 0) tag_store(a.xch + XO_SSH + i, epoch, __float_as_uint(silu_f32(ag) * au));
    } else if (g == 0) {
      float gs = 0.0f;
#pragma unroll
      for (int c = 0; c < 4; ++c)
        gs += dot8_bf16(*reinterpret_cast<const uint4*>(a.ssg + 512 * c + 8 * lane), xv[c]);
      gs = wave_sum_f32(gs);
      if (lane == 0) {
        const float p = 1.0f / (1.0f + expf(-gs));
        tag_store(a.xch + XO_GATE, epoch, __float_as_uint(p));
        if (a.gate_prob_out) a.gate_prob_out[0] = p;
      }
    }
  }

  // ------------------------------------------------------------------------------ phase 2 --
  if (wave == 0) {
    uint32_t lb[4];
    wait_tags<4>(a.xch + XO_LOGITS + lane, 64, epoch, err, lb);
    float lg[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) lg[j] = bf16_to_f32(lb[j] & 0xFFFFu);
    // R2, the same arithmetic as route_softmax, from registers
    float m = fmaxf(fmaxf(lg[0], lg[1]), fmaxf(lg[2], lg[3]));
    m = wave_max_f32(m);
    float p[4], sum = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) { p[j] = expf(lg[j] - m); sum += p[j]; }
    sum = wave_sum_f32(sum);
    const float rs = 1.0f / sum;
#pragma unroll
    for (int j = 0; j < 4; ++j) p[j] *= rs;
    if (g == 0 && a.logits_out) {
#pragma unroll
      for (int j = 0; j < 4; ++j) a.logits_out[64 * j + lane] = (uint16_t)(lb[j] & 0xFFFFu);
    }
    route_select_and_write(tk, p, E, K, lane, s_ids, s_wf, s_wb, nullptr, a.exact_order != 0);
    wave_sync();
    if (lane < K) {
      s_w[lane] = bf16_to_f32(s_wb[lane]);
      if (g == 0) {
        if (a.ids_out) a.ids_out[lane] = s_ids[lane];
        if (a.w_f32_out) a.w_f32_out[lane] = s_wf[lane];
        if (a.w_bf16_out) a.w_bf16_out[lane] = s_wb[lane];
      }
    }
  }
  __syncthreads();
  {
    // routed gate/up: slot k = g / 32, intermediate rows i0, i0+1 (gate and up) per wave
    const int k = g >> 5;
    const int i0 = 16 * (g & 31) + 2 * wave;
    const int e = s_ids[k];
    const int b = lane >> 3, c = lane & 7, gq = c >> 1, l0 = 16 * (c & 1);
    constexpr size_t rowb = (H / 256) * 144;
    const uint8_t* ebase = a.gu + (size_t)e * 2 * I * rowb;
    uint4 hdr[4], qs[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = (r & 1) ? (I + i0 + (r >> 1)) : (i0 + (r >> 1));
      const uint8_t* p = ebase + (size_t)row * rowb + (size_t)b * 144;
      hdr[r] = *reinterpret_cast<const uint4*>(p);
      qs[r] = *reinterpret_cast<const uint4*>(p + 16 + 16 * c);
    }
    float xl[16], xh[16];
    load_x32<XDT>(a.x, (size_t)256 * b + 64 * gq + l0, xl, xh);
    float sxl = 0.0f, sxh = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) { sxl += xl[i]; sxh += xh[i]; }
    float acc[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[r] = wave_sum_f32(q4k_chunk_dot(hdr[r], qs[r], gq, xl, xh, sxl, sxh));
#pragma unroll
    for (int r = 0; r < 2; ++r)
      if (lane == r)
        tag_store(a.xch + XO_SR + k * I + i0 + r, epoch,
                  __float_as_uint(silu_f32(acc[2 * r]) * acc[2 * r + 1]));
  }
  if (wave == 4 || wave == 5) {
    float acc = 0.0f;
    uint32_t sb[4][8];
#pragma unroll
    for (int c = 0; c < 4; ++c) wait_tags<8>(a.xch + XO_SSH + 128 * c + 8 * l16, 1, epoch, err, sb[c]);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float sv[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) sv[j] = __uint_as_float(sb[c][j]);
      acc += dot8_bf16(sdw[c], sv);
    }
    acc = row16_sum_f32(acc);
    if (l16 == 0) sh_raw[4 * (wave - 4) + g4] = acc;
  }

  // ------------------------------------------------------------------------------ phase 3 --
  // wave w: output row h0 + w for slots k = 4 pass + (lane >> 4)
  const int h0 = 8 * g;
  constexpr size_t drowb = (I / 256) * 144;
  uint4 dh[2], dq[2];
  {
    const int b = l16 >> 3, c = l16 & 7;
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {
      const int k = 4 * pass + g4;
      const uint8_t* p = a.dn + ((size_t)s_ids[k] * H + h0 + wave) * drowb + (size_t)b * 144;
      dh[pass] = *reinterpret_cast<const uint4*>(p);
      dq[pass] = *reinterpret_cast<const uint4*>(p + 16 + 16 * c);
    }
  }
  {
    constexpr int PER = (K * I) / kThreads;
    uint32_t sv[PER];
    wait_tags<PER>(a.xch + XO_SR + threadIdx.x, kThreads, epoch, err, sv);
#pragma unroll
    for (int j = 0; j < PER; ++j) (&s_all[0][0])[kThreads * j + threadIdx.x] = __uint_as_float(sv[j]);
  }
  if (threadIdx.x == 0) {
    s_gate = __uint_as_float(wait_tag(a.xch + XO_GATE, epoch, err));
    int id[K], sl[K];
#pragma unroll
    for (int k = 0; k < K; ++k) { id[k] = s_ids[k]; sl[k] = k; }
#pragma unroll
    for (int pass = 0; pass < K - 1; ++pass)
#pragma unroll
      for (int j = 0; j < K - 1; ++j)
        if (id[j] > id[j + 1]) {
          const int ti = id[j]; id[j] = id[j + 1]; id[j + 1] = ti;
          const int ts = sl[j]; sl[j] = sl[j + 1]; sl[j + 1] = ts;
        }
#pragma unroll
    for (int k = 0; k < K; ++k) s_order[k] = sl[k];
  }
  __syncthreads();
  {
    const int b = l16 >> 3, c = l16 & 7, gq = c >> 1, l0 = 16 * (c & 1);
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {
      const int k = 4 * pass + g4;
      const float* sp = &s_all[k][256 * b + 64 * gq + l0];
      float xl[16], xh[16], sxl = 0.0f, sxh = 0.0f;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        xl[i] = sp[i];
        xh[i] = sp[32 + i];
        sxl += xl[i];
        sxh += xh[i];
      }
      const float v = row16_sum_f32(q4k_chunk_dot(dh[pass], dq[pass], gq, xl, xh, sxl, sxh));
      if (l16 == 0) ys[wave][k] = v;
    }
  }
  __syncthreads();
  if (threadIdx.x < 8) {
    const int r = threadIdx.x, h = h0 + r;
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < K; ++j) {
      const int k = s_order[j];
      acc += s_w[k] * ys[r][k];
    }
    const float sh = s_gate * sh_raw[r];
    if (a.routed_sum) a.routed_sum[h] = acc;
    if (a.shared_out) a.shared_out[h] = sh;
    if (a.expert_raw) {
#pragma unroll
      for (int k = 0; k < K; ++k) a.expert_raw[(size_t)k * H + h] = ys[r][k];
    }
    a.out[h] = (a.residual ? a.residual[h] : 0.0f) + acc + sh;
  }
  // the last workgroup out advances the epoch for the next launch
  if (threadIdx.x == 0) {
    const int arrived = __hip_atomic_fetch_add(a.sync + 2, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (arrived == kG - 1) {
      __hip_atomic_store(a.sync + 2, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_fetch_add(a.sync + 1, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

}  // namespace moe

using namespace moe;

bool moe_layer_kernel_supported(int H, int I, int E, int K, int Is, int gu_fmt, int dn_fmt) {
  static int ncu = -1;
  if (ncu < 0) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      ncu = 0;
  }
  return ncu >= kG && H == 2048 && I == 512 && E == 256 && K == 8 && Is == 512 &&
         gu_fmt == MOE_FMT_Q4_K && dn_fmt == MOE_FMT_Q4_K;
}

size_t moe_layer_exchange_bytes() { return (size_t)XO_END * 8; }

int moe_launch_decode_layer(const MoeDecodeLaunch& L, int* sync, uint64_t* xch, hipStream_t st) {
  LayerArgs a;
  a.x = L.x; a.residual = L.residual; a.w_router = (const uint16_t*)L.w_router; a.bias = L.bias;
  a.gu = (const uint8_t*)L.gu; a.dn = (const uint8_t*)L.dn;
  a.sg = (const uint16_t*)L.sg; a.su = (const uint16_t*)L.su; a.sd = (const uint16_t*)L.sd;
  a.ssg = (const uint16_t*)L.ssg;
  a.sync = sync; a.xch = xch;
  a.logits_out = L.logits; a.ids_out = L.ids; a.w_f32_out = L.w_f32; a.w_bf16_out = L.w_bf16;
  a.gate_prob_out = L.gate_prob; a.out = L.out; a.routed_sum = L.routed_sum;
  a.shared_out = L.shared_out; a.expert_raw = L.expert_raw;
  a.exact_order = (L.ids_out_requested || L.expert_raw) ? 1 : 0;
  if (L.x_dtype == MOE_DT_F32)
    hipLaunchKernelGGL(k_dec_layer<MOE_DT_F32>, dim3(kG), dim3(kThreads), 0, st, a);
  else
    hipLaunchKernelGGL(k_dec_layer<MOE_DT_BF16>, dim3(kG), dim3(kThreads), 0, st, a);
  return moe_check_launch("decode_layer");
}
