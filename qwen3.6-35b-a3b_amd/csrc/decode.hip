// Fused single-token decode step of one MoE block: three launches instead of nine
// (engine/m3_forward.py:430-476 for one row; specification/11-moe-block.md §11.1-§11.6).
//
//  K1 k_dec_route_shared  router rows (one wave per expert logit, f64, certified bf16) ||
//                         shared gate/up rows || the scalar gate. The last router block to finish
//                         (device-scope atomic ticket) runs R2-R5 for the token.
//  K2 k_dec_gateup        8 routed experts' gate/up rows (fused Q4_K decode, f32) || shared down
//  K3 k_dec_down_combine  8 routed experts' down rows for 8 output rows per block, then the
//                         ascending-expert-id combine, the gated shared expert and an optional
//                         residual add, all in the block that produced the 8 x 8 dot products.
// Every routing value stays on the device; no float atomics (the output is deterministic).
#include "common.h"
#include "moe_internal.h"
#include "router_dev.h"
#include "gemv_dev.h"

namespace moe {

struct DecodeArgs {
  const void* x;
  const float* residual;
  const void* w_router;
  int router_dt;                // router weights: bf16 or f32
  const float* bias;
  const uint8_t* gu;            // gate rows of expert e at gu + e * gu_estride
  const uint8_t* gu_up;         // up rows likewise
  size_t gu_estride;
  const uint8_t* dn;
  const void* sg;               // shared expert rows: bf16, or Q8_0 when sfmt says so
  const void* su;
  const void* sd;
  int sfmt;
  const void* ssg;
  int ssg_dt;                   // scalar shared gate: bf16 or f32
  uint16_t* logits;
  int32_t* ids;
  float* w_f32;
  uint16_t* w_bf16;
  float* s_shared;
  float* gate_prob;
  float* shared_raw;
  float* s_routed;
  float* out;
  float* routed_sum;
  float* shared_out;
  float* expert_raw;
  int* counter;
  int H, I, E, K, Is;
};

// 8 router weights of row wr (bf16 or f32; f32 x f32 products are still exact in f64)
template <int WDT>
__device__ __forceinline__ void router_w8(const void* wr, int i, double* o) {
  if (WDT == MOE_DT_F32) {
    const float4 a = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(wr) + i);
    const float4 b = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(wr) + i + 4);
    o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w; o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
  } else {
    const uint4 v = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(wr) + i);
    const uint32_t ww[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) { o[2 * k] = bf16_to_f32(ww[k] & 0xFFFFu); o[2 * k + 1] = bf16_to_f32(ww[k] >> 16); }
  }
}

// One router logit (R1) for a single token, computed by one wave; returns the bf16 bits.
template <int XDT, int WDT>
__device__ __forceinline__ uint32_t router_logit_wave(const void* xv, const void* wr,
                                                      float bias, int H, int lane) {
  const int nchunk = H / 512;
  double acc = 0.0, xsq = 0.0, wsq = 0.0;
  for (int c = 0; c < nchunk; ++c) {
    double wd[8];
    router_w8<WDT>(wr, c * 512 + lane * 8, wd);
    float xf[8];
    load_x8<XDT>(xv, (size_t)c * 512 + lane * 8, xf);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const double x0 = xf[i];
      acc = fma(x0, wd[i], acc);
      xsq = fma(x0, x0, xsq);
      wsq = fma(wd[i], wd[i], wsq);
    }
  }
  acc = wave_sum_f64(acc);
  xsq = wave_sum_f64(xsq);
  wsq = wave_sum_f64(wsq);
  const double bval = bias;
  const double s = acc + bval;
  const double nrm = sqrt(xsq) * sqrt(wsq) + fabs(bval);
  uint32_t bits;
  if (round_bf16_certified(s, 4.0 * (double)(H + 3) * 0x1p-53 * nrm, &bits)) return bits;
  DD d = {0.0, 0.0};
  for (int c = 0; c < nchunk; ++c) {
    double wd[8];
    router_w8<WDT>(wr, c * 512 + lane * 8, wd);
    float xf[8];
    load_x8<XDT>(xv, (size_t)c * 512 + lane * 8, xf);
#pragma unroll
    for (int i = 0; i < 8; ++i) d = dd_add(d, DD{(double)xf[i] * wd[i], 0.0});
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    DD other = {__shfl_xor(d.hi, o, 64), __shfl_xor(d.lo, o, 64)};
    d = dd_add(d, other);
  }
  d = dd_add(d, DD{bval, 0.0});
  return round_bf16_dd(d, (double)(H + 64) * 0x1p-104 * 16.0 * nrm);
}

template <int XDT>
__global__ __launch_bounds__(256) void k_dec_route_shared(DecodeArgs a) {
  __shared__ TopkLds s;
  __shared__ int is_last;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int NR = (a.E + 3) / 4, NS = a.Is / 4;
  const int bid = blockIdx.x;
  if (bid < NR) {
    const int e = bid * 4 + wave;
    if (e < a.E) {
      const float bv = a.bias ? a.bias[e] : 0.0f;
      const uint32_t bits =
          a.router_dt == MOE_DT_F32
              ? router_logit_wave<XDT, MOE_DT_F32>(a.x, reinterpret_cast<const float*>(a.w_router) + (size_t)e * a.H, bv, a.H, lane)
              : router_logit_wave<XDT, MOE_DT_BF16>(a.x, reinterpret_cast<const uint16_t*>(a.w_router) + (size_t)e * a.H, bv, a.H, lane);
      if (lane == 0) a.logits[e] = (uint16_t)bits;
    }
    __threadfence();                       // publish this wave's logit device-wide
    __syncthreads();
    if (threadIdx.x == 0) is_last = (atomicAdd(a.counter, 1) == NR - 1);
    __syncthreads();
    if (!is_last) return;
    __threadfence();                       // acquire every block's logits
    if (wave == 0) {
      float p[4];
      route_softmax(a.logits, a.E, lane, p);
      route_select_and_write(s, p, a.E, a.K, lane, a.ids, a.w_f32, a.w_bf16, nullptr);
      if (lane == 0) atomicExch(a.counter, 0);   // ready for the next launch
    }
    return;
  }
  if (bid < NR + NS) {
    const int i = (bid - NR) * 4 + wave;
    float ag = 0.0f, au = 0.0f;
    for (int c = 0; c < a.H / 512; ++c) {
      float xv[8];
      load_x8<XDT>(a.x, (size_t)512 * c + 8 * lane, xv);
      if (a.sfmt == MOE_FMT_Q8_0) {
        ag += dot8_shared<MOE_FMT_Q8_0>(a.sg, i, a.H, 512 * c + 8 * lane, xv);
        au += dot8_shared<MOE_FMT_Q8_0>(a.su, i, a.H, 512 * c + 8 * lane, xv);
      } else {
        ag += dot8_shared<MOE_FMT_BF16>(a.sg, i, a.H, 512 * c + 8 * lane, xv);
        au += dot8_shared<MOE_FMT_BF16>(a.su, i, a.H, 512 * c + 8 * lane, xv);
      }
    }
    ag = wave_sum_f32(ag);
    au = wave_sum_f32(au);
    if (lane == 0) a.s_shared[i] = silu_f32(ag) * au;
    return;
  }
  if (wave == 0) {
    float g = 0.0f;
    for (int c = 0; c < a.H / 512; ++c) {
      float xv[8];
      load_x8<XDT>(a.x, (size_t)512 * c + 8 * lane, xv);
      g += dot8_w(a.ssg, (size_t)512 * c + 8 * lane, a.ssg_dt, xv);
    }
    g = wave_sum_f32(g);
    if (lane == 0) a.gate_prob[0] = 1.0f / (1.0f + expf(-g));
  }
}

// grid K*(I/16) routed blocks + H/16 shared-down blocks
template <int XDT>
__global__ __launch_bounds__(256) void k_dec_gateup(DecodeArgs a) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nchunk = a.I / 16;
  const int bid = blockIdx.x;
  if (bid < a.K * nchunk) {
    const int k = bid / nchunk;
    const int i0 = (bid % nchunk) * 16 + wave * 4;
    const int e = a.ids[k];
    const int b = lane >> 3, c = lane & 7, g = c >> 1, l0 = 16 * (c & 1);
    const size_t rowb = (size_t)(a.H / 256) * 144;
    const uint8_t* gbase = a.gu + (size_t)e * a.gu_estride;
    const uint8_t* ubase = a.gu_up + (size_t)e * a.gu_estride;
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int bg = 0; bg < a.H / 2048; ++bg) {
      const int blk = bg * 8 + b;
      uint4 hdr[8], qs[8];
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const uint8_t* p = ((r & 1) ? ubase : gbase) + (size_t)(i0 + (r >> 1)) * rowb + (size_t)blk * 144;
        hdr[r] = *reinterpret_cast<const uint4*>(p);
        qs[r] = *reinterpret_cast<const uint4*>(p + 16 + 16 * c);
      }
      float xl[16], xh[16];
      load_x32<XDT>(a.x, (size_t)256 * blk + 64 * g + l0, xl, xh);
      float sxl = 0.0f, sxh = 0.0f;
#pragma unroll
      for (int i = 0; i < 16; ++i) { sxl += xl[i]; sxh += xh[i]; }
#pragma unroll
      for (int r = 0; r < 8; ++r) acc[r] += q4k_chunk_dot(hdr[r], qs[r], g, xl, xh, sxl, sxh);
    }
#pragma unroll
    for (int r = 0; r < 8; ++r) acc[r] = wave_sum_f32(acc[r]);
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (lane == r) a.s_routed[(size_t)k * a.I + i0 + r] = silu_f32(acc[2 * r]) * acc[2 * r + 1];
    return;
  }
  const int l16 = lane & 15;
  const int row = (bid - a.K * nchunk) * 16 + wave * 4 + (lane >> 4);
  float acc = 0.0f;
  for (int c = 0; c < a.Is / 128; ++c) {
    float sv[8];
    load_x8<MOE_DT_F32>(a.s_shared, (size_t)128 * c + 8 * l16, sv);
    acc += a.sfmt == MOE_FMT_Q8_0 ? dot8_shared<MOE_FMT_Q8_0>(a.sd, row, a.Is, 128 * c + 8 * l16, sv)
                                  : dot8_shared<MOE_FMT_BF16>(a.sd, row, a.Is, 128 * c + 8 * l16, sv);
  }
  acc = row16_sum_f32(acc);
  if (l16 == 0) a.shared_raw[row] = acc;
}

// down-row dot for 16 lanes: (row of I elements of down weights) . s (I floats), lanes l16 of
// the group; Q4_K / Q5_K: lane = 8*block + chunk over a 512-element window; Q6_K: lane =
// 8*block + 4g + k
template <int DFMT>
__device__ __forceinline__ float down_dot16(const uint8_t* rowp, const float* sv, int I, int l16) {
  float acc = 0.0f;
  const int b = l16 >> 3, c = l16 & 7;
  if (DFMT == MOE_FMT_Q4_K || DFMT == MOE_FMT_Q5_K) {
    constexpr int kBB = DFMT == MOE_FMT_Q5_K ? 176 : 144, kQs = DFMT == MOE_FMT_Q5_K ? 48 : 16;
    const int g = c >> 1, l0 = 16 * (c & 1);
    for (int bg = 0; bg < I / 512; ++bg) {
      const int blk = bg * 2 + b;
      const uint8_t* p = rowp + (size_t)blk * kBB;
      const uint4 hdr = *reinterpret_cast<const uint4*>(p);
      const uint4 qs = *reinterpret_cast<const uint4*>(p + kQs + 16 * c);
      float xl[16], xh[16];
      load_x32<MOE_DT_F32>(sv, (size_t)256 * blk + 64 * g + l0, xl, xh);
      float sxl = 0.0f, sxh = 0.0f;
#pragma unroll
      for (int i = 0; i < 16; ++i) { sxl += xl[i]; sxh += xh[i]; }
      if (DFMT == MOE_FMT_Q5_K)
        acc += q5k_chunk_dot(hdr, qs, *reinterpret_cast<const uint4*>(p + 16 + l0), g, xl, xh, sxl, sxh);
      else
        acc += q4k_chunk_dot(hdr, qs, g, xl, xh, sxl, sxh);
    }
  } else {
    const int g = c >> 2, k = c & 3;
    for (int bg = 0; bg < I / 512; ++bg) {
      const int blk = bg * 2 + b;
      const uint16_t* p = reinterpret_cast<const uint16_t*>(rowp + (size_t)blk * 210);
      const uint16_t* ql = p + (64 * g + 32 * (k & 1)) / 2;
      const uint16_t* qh = p + (128 + 32 * g) / 2;
      const uint32_t scw = p[(192 + 8 * g + 2 * k) / 2];
      const float d = f16_to_f32(p[104]);
      const float* sp = sv + 256 * blk + 128 * g + 32 * k;
      const int sh_l = 4 * (k >> 1), sh_h = 2 * k;
      float d0 = 0.0f, d1 = 0.0f, s0 = 0.0f, s1 = 0.0f;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const uint32_t lw = ql[i], hw = qh[i];
        const float qa = (float)(((lw >> sh_l) & 15u) | (((hw >> sh_h) & 3u) << 4));
        const float qb = (float)((((lw >> 8) >> sh_l) & 15u) | ((((hw >> 8) >> sh_h) & 3u) << 4));
        const float va = sp[2 * i], vb = sp[2 * i + 1];
        if (i < 8) { d0 = fmaf(va, qa, fmaf(vb, qb, d0)); s0 += va + vb; }
        else { d1 = fmaf(va, qa, fmaf(vb, qb, d1)); s1 += va + vb; }
      }
      acc += d * (float)(int8_t)(scw & 0xFFu) * (d0 - 32.0f * s0) +
             d * (float)(int8_t)(scw >> 8) * (d1 - 32.0f * s1);
    }
  }
  return acc;
}

// grid H/8; wave w computes rows h0+2w, h0+2w+1 for all K = 8 slots (4 passes x 4 groups of 16)
template <int DFMT>
__global__ __launch_bounds__(256) void k_dec_down_combine(DecodeArgs a) {
  __shared__ float ys[8][8];
  __shared__ int order[8];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, l16 = lane & 15, g4 = lane >> 4;
  const int h0 = blockIdx.x * 8;
  const size_t rowb = (size_t)(a.I / 256) * (DFMT == MOE_FMT_Q4_K ? 144 : DFMT == MOE_FMT_Q5_K ? 176 : 210);
  if (threadIdx.x == 0) {
    // slots in ascending expert id (bubble sort on (id, slot) pairs, constant indices only)
    int id[8], sl[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) { id[k] = a.ids[k]; sl[k] = k; }
#pragma unroll
    for (int pass = 0; pass < 7; ++pass)
#pragma unroll
      for (int j = 0; j < 7; ++j)
        if (id[j] > id[j + 1]) {
          const int ti = id[j]; id[j] = id[j + 1]; id[j + 1] = ti;
          const int ts = sl[j]; sl[j] = sl[j + 1]; sl[j + 1] = ts;
        }
#pragma unroll
    for (int k = 0; k < 8; ++k) order[k] = sl[k];
  }
#pragma unroll
  for (int pass = 0; pass < 4; ++pass) {
    const int rl = 2 * wave + (g4 & 1);
    const int k = 2 * pass + (g4 >> 1);
    const int e = a.ids[k];
    const uint8_t* rowp = a.dn + ((size_t)e * a.H + h0 + rl) * rowb;
    float v = down_dot16<DFMT>(rowp, a.s_routed + (size_t)k * a.I, a.I, l16);
    v = row16_sum_f32(v);
    if (l16 == 0) ys[rl][k] = v;
  }
  __syncthreads();
  if (threadIdx.x < 8) {
    const int r = threadIdx.x, h = h0 + r;
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int k = order[j];
      acc = comb_madd(acc, bf16_to_f32(a.w_bf16[k]), ys[r][k]);
    }
    const float sh = a.gate_prob[0] * a.shared_raw[h];
    if (a.routed_sum) a.routed_sum[h] = acc;
    if (a.shared_out) a.shared_out[h] = sh;
    if (a.expert_raw) {
#pragma unroll
      for (int k = 0; k < 8; ++k) a.expert_raw[(size_t)k * a.H + h] = ys[r][k];
    }
    a.out[h] = comb_out(a.residual ? a.residual[h] : 0.0f, acc, a.gate_prob[0], a.shared_raw[h]);
  }
}

__global__ void k_zero_words(int* p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

// the status word, read and cleared in one device-scope exchange
__global__ void k_take_status(int* word, int32_t* out) {
  if (threadIdx.x == 0) out[0] = atomicExch(word, 0);
}

}  // namespace moe

using namespace moe;

int moe_launch_zero_words(int* p, int n, hipStream_t st) {
  hipLaunchKernelGGL(k_zero_words, dim3((n + 255) / 256), dim3(256), 0, st, p, n);
  return moe_check_launch("zero_words");
}

int moe_launch_take_status(int* word, int32_t* out, hipStream_t st) {
  hipLaunchKernelGGL(k_take_status, dim3(1), dim3(64), 0, st, word, out);
  return moe_check_launch("take_status");
}

int moe_launch_decode_fused(const MoeDecodeLaunch& L, hipStream_t st) {
  DecodeArgs a;
  a.x = L.x; a.residual = L.residual; a.w_router = L.w_router; a.router_dt = L.router_dt; a.bias = L.bias;
  a.gu = (const uint8_t*)L.gu; a.dn = (const uint8_t*)L.dn;
  {
    const size_t rowb = (size_t)(L.H / 256) * 144;
    a.gu_estride = L.gu_estride ? L.gu_estride : (size_t)2 * L.I * rowb;
    a.gu_up = L.gu_up ? (const uint8_t*)L.gu_up : a.gu + (size_t)L.I * rowb;
  }
  a.sg = L.sg; a.su = L.su; a.sd = L.sd; a.sfmt = L.sfmt;
  a.ssg = L.ssg; a.ssg_dt = L.ssg_dt;
  a.logits = L.logits; a.ids = L.ids; a.w_f32 = L.w_f32; a.w_bf16 = L.w_bf16;
  a.s_shared = L.s_shared; a.gate_prob = L.gate_prob; a.shared_raw = L.shared_raw;
  a.s_routed = L.s_routed; a.out = L.out; a.routed_sum = L.routed_sum; a.shared_out = L.shared_out;
  a.expert_raw = L.expert_raw; a.counter = L.counter;
  a.H = L.H; a.I = L.I; a.E = L.E; a.K = L.K; a.Is = L.Is;
  const int NR = (L.E + 3) / 4, NS = L.Is / 4;
  if (L.x_dtype == MOE_DT_F32) {
    hipLaunchKernelGGL(k_dec_route_shared<MOE_DT_F32>, dim3(NR + NS + 1), dim3(256), 0, st, a);
    hipLaunchKernelGGL(k_dec_gateup<MOE_DT_F32>, dim3(L.K * (L.I / 16) + L.H / 16), dim3(256), 0, st, a);
  } else {
    hipLaunchKernelGGL(k_dec_route_shared<MOE_DT_BF16>, dim3(NR + NS + 1), dim3(256), 0, st, a);
    hipLaunchKernelGGL(k_dec_gateup<MOE_DT_BF16>, dim3(L.K * (L.I / 16) + L.H / 16), dim3(256), 0, st, a);
  }
  if (L.dn_fmt == MOE_FMT_Q4_K)
    hipLaunchKernelGGL(k_dec_down_combine<MOE_FMT_Q4_K>, dim3(L.H / 8), dim3(256), 0, st, a);
  else if (L.dn_fmt == MOE_FMT_Q5_K)
    hipLaunchKernelGGL(k_dec_down_combine<MOE_FMT_Q5_K>, dim3(L.H / 8), dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL(k_dec_down_combine<MOE_FMT_Q6_K>, dim3(L.H / 8), dim3(256), 0, st, a);
  return moe_check_launch("decode_fused");
}
