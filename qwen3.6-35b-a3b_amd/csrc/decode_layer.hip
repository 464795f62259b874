// Single-token decode of one MoE block in ONE launch: a persistent grid of 256 workgroups of 8
// waves (one per CU on MI355X, all co-resident) runs the block's dependent phases and hands data
// between them through self-validating exchange words instead of kernel boundaries or
// device-wide fences.
//
//   start    every wg stages x in LDS, RMS-normalized when a post-attention norm weight is given
//            (Form A, engine/m3_forward.py:303-307; the f64 sum of squares is a block reduction)
//   phase 1  wg g: router logit e = g (f64, certified bf16) | shared gate/up rows i = 2g, 2g+1 |
//            (wg 0) the scalar shared gate                 -> logits[E], s_shared[I_s], gate
//   phase 2  every wg waits for the 256 logits and runs R2-R5 itself (same answer everywhere; the
//            fast top-k's slot order stands in for torch's when ties sit inside the top 8 and no
//            stage output is asked for: same experts, same weights);
//            wg g: routed gate/up rows of slot k = g/32, i in [16(g%32), +16) -> s_routed[k];
//            its down-projection weights are requested here, ahead of their use;
//            shared down rows 8g..8g+7 (one wave; waits for s_shared)
//   phase 3  wg g: down rows h in [64(g%32), +64) of slot k's expert (waits for the 512 words of
//            s_routed[k] only)                             -> y[k][h]
//   phase 4  wg g: ascending-expert-id combine of y[0..7][8g..8g+7], gated shared expert,
//            residual -> out[8g..8g+7]
// Each workgroup reads at most 2 KB of exchange words per phase: the words are hot (every
// workgroup polls the same few KB while the weights stream), so their volume sets the latency.
//
// Exchange words are 32-bit: a value is stored as the complement of its bit pattern (NaNs made
// canonical first), so 0 never encodes a value and means "not written yet". Each word is written
// once per launch by one dword store that bypasses the non-coherent L2 (agent-scope relaxed atomic
// store, sc1) and read the same way (sc1 loads, up to 16 bytes at a time); a reader re-polls, all
// of its missing words in parallel, until every word it needs is non-zero. Two buffers alternate
// by the launch's epoch parity, and each launch zeroes the buffer the next launch will use, so a
// zeroed workspace is a valid starting state and graph replays work. The epoch lives in the
// workspace's sync words: every workgroup reads it at the start, the last workgroup to finish
// (arrival counter) advances it. Every spin is bounded: on a timeout the workgroup records an
// error bit and carries on (no hang).
#include "common.h"
#include "moe_internal.h"
#include "router_dev.h"
#include "gemv_dev.h"

namespace moe {

constexpr int kG = 256;                 // workgroups (one per CU)
constexpr int kThreads = 512;           // 8 waves
constexpr int kSpinLimit = 1 << 20;     // polls (each a memory round trip) before giving up

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
  uint32_t* xch;                        // two exchange buffers of XW_BUF words
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
  const float* norm_w;                  // post-attention RMSNorm weight [H] f32, or NULL
  float norm_eps;
};

// exchange buffer layout (uint32 words; every region starts 16-byte aligned)
constexpr int XW_LOGITS = 0;            // 256 logits (bf16 bits)
constexpr int XW_GATE = 256;            // 4 copies of the sigmoid of the shared expert's gate
constexpr int XW_SSH = 260;             // 512 shared-expert activations
constexpr int XW_SR = 772;              // 8 x 512 routed activations, slot-major
constexpr int XW_Y = 772 + 4096;        // 8 x 2048 routed expert outputs, slot-major
constexpr int XW_BUF = XW_Y + 8 * 2048; // words per buffer
constexpr int kClearPerWg = (XW_BUF + kG - 1) / kG;

__device__ __forceinline__ uint32_t xenc(float v) {
  const uint32_t b = (v != v) ? 0x7FC00000u : __float_as_uint(v);
  return ~b;
}
__device__ __forceinline__ float xdec(uint32_t w) { return __uint_as_float(~w); }

__device__ __forceinline__ void xstore(uint32_t* p, uint32_t w) {
  __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t xload(uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// 16 bytes at byte offset `off` of the buffer, read past the non-coherent L2 (sc1)
__device__ __forceinline__ uint4 xload4(__amdgpu_buffer_rsrc_t r, int off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 16);
  return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ bool xfull(uint4 v) { return v.x && v.y && v.z && v.w; }

// N words p[j * stride]: every missing word is loaded again, in parallel, until all are written
template <int N>
__device__ __forceinline__ void xwait(uint32_t* p, int stride, int* err, uint32_t* v) {
#pragma unroll
  for (int j = 0; j < N; ++j) v[j] = xload(p + j * stride);
  for (int spins = 0;; ++spins) {
    bool ok = true;
#pragma unroll
    for (int j = 0; j < N; ++j) ok = ok && v[j] != 0u;
    if (ok) return;
    if (spins >= kSpinLimit) { atomicOr(err, 1); return; }
    __builtin_amdgcn_s_sleep(1);
#pragma unroll
    for (int j = 0; j < N; ++j)
      if (v[j] == 0u) v[j] = xload(p + j * stride);
  }
}
// N 16-byte groups at byte offsets off[j] of the buffer, same protocol
template <int N>
__device__ __forceinline__ void xwait4(__amdgpu_buffer_rsrc_t r, const int* off, int* err,
                                       uint4* v) {
#pragma unroll
  for (int j = 0; j < N; ++j) v[j] = xload4(r, off[j]);
  for (int spins = 0;; ++spins) {
    bool ok = true;
#pragma unroll
    for (int j = 0; j < N; ++j) ok = ok && xfull(v[j]);
    if (ok) return;
    if (spins >= kSpinLimit) { atomicOr(err, 1); return; }
    __builtin_amdgcn_s_sleep(1);
#pragma unroll
    for (int j = 0; j < N; ++j)
      if (!xfull(v[j])) v[j] = xload4(r, off[j]);
  }
}

template <int XDT>
__global__ __launch_bounds__(kThreads) void k_dec_layer(LayerArgs a) {
  constexpr int H = 2048, I = 512, E = 256, K = 8, IS = 512;
  __shared__ float s_x[H];
  __shared__ TopkLds tk;                 // the exact replay's scratch (ties only)
  __shared__ float s_k[I];               // this workgroup's slot's routed activations
  __shared__ float s_sh[IS];             // shared-expert activations (wave 4)
  __shared__ int s_ids[K];
  __shared__ float s_w[K];
  __shared__ float s_wf[K];
  __shared__ uint16_t s_wb[K];
  __shared__ int s_order[K];
  __shared__ float sh_raw[8];
  __shared__ float ys[K][8];
  __shared__ float s_gate;
  __shared__ double s_red[kThreads / 64];
  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int l16 = lane & 15;
  const int g = blockIdx.x;
  const int slot = g >> 5, blk = g & 31;
  int* err = a.sync + 3;
  const uint32_t epoch =
      (uint32_t)__hip_atomic_load(a.sync + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
  uint32_t* xb = a.xch + (epoch & 1u) * XW_BUF;          // this launch's words
  uint32_t* xn = a.xch + ((epoch & 1u) ^ 1u) * XW_BUF;   // the next launch's, zeroed here
  const __amdgpu_buffer_rsrc_t xr =
      __builtin_amdgcn_make_buffer_rsrc(xb, 0, XW_BUF * 4, 0x00020000);

  // x into LDS as f32 (RMS-normalized first when norm_w is given); the residual of this
  // workgroup's 8 output rows; the next buffer's slice
  {
    float4 v;
    if (XDT == MOE_DT_F32) {
      v = reinterpret_cast<const float4*>(a.x)[t];
    } else {
      const uint2 u = reinterpret_cast<const uint2*>(a.x)[t];
      v = make_float4(bf16_to_f32(u.x & 0xFFFFu), bf16_to_f32(u.x >> 16),
                      bf16_to_f32(u.y & 0xFFFFu), bf16_to_f32(u.y >> 16));
    }
    if (a.norm_w) {
      // r = f32(1 / sqrt(mean(x^2) + eps)) in f64: every square is exact, one final rounding
      const float4 nw = reinterpret_cast<const float4*>(a.norm_w)[t];
      double ss = (double)v.x * v.x + (double)v.y * v.y + (double)v.z * v.z + (double)v.w * v.w;
      ss = wave_sum_f64(ss);
      if (lane == 0) s_red[wave] = ss;
      __syncthreads();
      double tot = 0.0;
#pragma unroll
      for (int j = 0; j < kThreads / 64; ++j) tot += s_red[j];
      const float r = (float)(1.0 / sqrt(tot / (double)H + (double)a.norm_eps));
      v = make_float4((v.x * r) * nw.x, (v.y * r) * nw.y, (v.z * r) * nw.z, (v.w * r) * nw.w);
    }
    reinterpret_cast<float4*>(s_x)[t] = v;
  }
  const float resid = (t < 8 && a.residual) ? a.residual[8 * g + t] : 0.0f;
  if (t < kClearPerWg && kClearPerWg * g + t < XW_BUF) xstore(xn + kClearPerWg * g + t, 0u);
  // wave 4: shared-down weights, row 8g + (lane >> 3), cols 64 (lane & 7) + 0..63
  uint4 sdw[8];
  if (wave == 4) {
    const uint16_t* dr = a.sd + (size_t)(8 * g + (lane >> 3)) * IS + 64 * (lane & 7);
#pragma unroll
    for (int c = 0; c < 8; ++c) sdw[c] = reinterpret_cast<const uint4*>(dr)[c];
  }
  __syncthreads();

  // ------------------------------------------------------------------------------ phase 1 --
  if (wave < 4) {
    // x at cols 512c + 8 lane (c = 0..3)
    float xv[4][8];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float4 u0 = *reinterpret_cast<const float4*>(s_x + 512 * c + 8 * lane);
      const float4 u1 = *reinterpret_cast<const float4*>(s_x + 512 * c + 8 * lane + 4);
      xv[c][0] = u0.x; xv[c][1] = u0.y; xv[c][2] = u0.z; xv[c][3] = u0.w;
      xv[c][4] = u1.x; xv[c][5] = u1.y; xv[c][6] = u1.z; xv[c][7] = u1.w;
    }
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
      if (lane == 0) xstore(xb + XW_LOGITS + g, ~bits);
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
      if (lane == 0) xstore(xb + XW_SSH + i, xenc(silu_f32(ag) * au));
    } else if (g == 0) {
      float gs = 0.0f;
#pragma unroll
      for (int c = 0; c < 4; ++c)
        gs += dot8_bf16(*reinterpret_cast<const uint4*>(a.ssg + 512 * c + 8 * lane), xv[c]);
      gs = wave_sum_f32(gs);
      const float p = 1.0f / (1.0f + expf(-gs));
      if (lane < 4) xstore(xb + XW_GATE + lane, xenc(p));   // the whole 16-byte group
      if (lane == 0 && a.gate_prob_out) a.gate_prob_out[0] = p;
    }
  }

  // ------------------------------------------------------------------------------ phase 2 --
  if (wave == 0) {
    uint32_t lw[4];
    xwait<4>(xb + XW_LOGITS + lane, 64, err, lw);
    float lg[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) lg[j] = bf16_to_f32(~lw[j] & 0xFFFFu);
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
      for (int j = 0; j < 4; ++j) a.logits_out[64 * j + lane] = (uint16_t)(~lw[j] & 0xFFFFu);
    }
    int my_id;
    float my_val, tot;
    const int code = wave_topk32<K>(p, lane, my_id, my_val, tot);
    if (code == 0 || (code == 1 && !a.exact_order)) {
      if (lane < K) {
        const float wv = my_val / tot;
        s_ids[lane] = my_id;
        s_wf[lane] = wv;
        s_wb[lane] = (uint16_t)f32_to_bf16(wv);
      }
    } else {
      route_replay_and_write(tk, p, E, K, lane, s_ids, s_wf, s_wb, nullptr);
    }
    wave_sync();
    if (lane < K) {
      const int id = s_ids[lane];
      int rank = 0;
#pragma unroll
      for (int j = 0; j < K; ++j) rank += (s_ids[j] < id) ? 1 : 0;
      s_order[rank] = lane;              // ascending expert id (ids are distinct)
      s_w[lane] = bf16_to_f32(s_wb[lane]);
      if (g == 0) {
        if (a.ids_out) a.ids_out[lane] = id;
        if (a.w_f32_out) a.w_f32_out[lane] = s_wf[lane];
        if (a.w_bf16_out) a.w_bf16_out[lane] = s_wb[lane];
      }
    }
  }
  __syncthreads();
  const int e = s_ids[slot];
  // phase-3 weights: down rows h = 64 blk + 2 (t >> 4) + pass of expert e; 16 lanes per row,
  // lane: super-block b = l16 >> 3, 16-byte nibble chunk c = l16 & 7
  constexpr size_t drowb = (I / 256) * 144;
  uint4 dh[2], dq[2];
  {
    // routed gate/up: intermediate rows i0, i0+1 (gate and up) per wave
    const int i0 = 16 * blk + 2 * wave;
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
    {
      const int db = l16 >> 3, dc = l16 & 7;
#pragma unroll
      for (int pass = 0; pass < 2; ++pass) {
        const int h = 64 * blk + 2 * (t >> 4) + pass;
        const uint8_t* p = a.dn + ((size_t)e * H + h) * drowb + (size_t)db * 144;
        dh[pass] = *reinterpret_cast<const uint4*>(p);
        dq[pass] = *reinterpret_cast<const uint4*>(p + 16 + 16 * dc);
      }
    }
    float xl[16], xh[16];
    {
      const float* xp = s_x + 256 * b + 64 * gq + l0;
#pragma unroll
      for (int i = 0; i < 16; i += 4) {
        const float4 u0 = *reinterpret_cast<const float4*>(xp + i);
        const float4 u1 = *reinterpret_cast<const float4*>(xp + 32 + i);
        xl[i] = u0.x; xl[i + 1] = u0.y; xl[i + 2] = u0.z; xl[i + 3] = u0.w;
        xh[i] = u1.x; xh[i + 1] = u1.y; xh[i + 2] = u1.z; xh[i + 3] = u1.w;
      }
    }
    float sxl = 0.0f, sxh = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) { sxl += xl[i]; sxh += xh[i]; }
    float acc[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[r] = wave_sum_f32(q4k_chunk_dot(hdr[r], qs[r], gq, xl, xh, sxl, sxh));
#pragma unroll
    for (int r = 0; r < 2; ++r)
      if (lane == r) xstore(xb + XW_SR + slot * I + i0 + r, xenc(silu_f32(acc[2 * r]) * acc[2 * r + 1]));
  }
  if (wave == 4) {
    // shared down, rows 8g..8g+7: the 512 shared activations once into LDS, then 8 lanes a row
    uint4 sb[2];
    {
      const int off[2] = {4 * (XW_SSH + 8 * lane), 4 * (XW_SSH + 8 * lane) + 16};
      xwait4<2>(xr, off, err, sb);
    }
    reinterpret_cast<float4*>(s_sh)[2 * lane] = make_float4(xdec(sb[0].x), xdec(sb[0].y), xdec(sb[0].z), xdec(sb[0].w));
    reinterpret_cast<float4*>(s_sh)[2 * lane + 1] = make_float4(xdec(sb[1].x), xdec(sb[1].y), xdec(sb[1].z), xdec(sb[1].w));
    wave_sync();
    float acc = 0.0f;
    const float* sp = s_sh + 64 * (lane & 7);
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      float sv[8];
      const float4 u0 = *reinterpret_cast<const float4*>(sp + 8 * c);
      const float4 u1 = *reinterpret_cast<const float4*>(sp + 8 * c + 4);
      sv[0] = u0.x; sv[1] = u0.y; sv[2] = u0.z; sv[3] = u0.w;
      sv[4] = u1.x; sv[5] = u1.y; sv[6] = u1.z; sv[7] = u1.w;
      acc += dot8_bf16(sdw[c], sv);
    }
    acc += dpp_f32<0xB1>(acc);
    acc += dpp_f32<0x4E>(acc);
    acc += dpp_f32<0x141>(acc);          // sum over the 8 lanes of the row
    if ((lane & 7) == 0) sh_raw[lane >> 3] = acc;
  }

  // ------------------------------------------------------------------------------ phase 3 --
  if (t < I / 4) {
    const int off[1] = {4 * (XW_SR + slot * I) + 16 * t};
    uint4 sv[1];
    xwait4<1>(xr, off, err, sv);
    reinterpret_cast<float4*>(s_k)[t] = make_float4(xdec(sv[0].x), xdec(sv[0].y), xdec(sv[0].z), xdec(sv[0].w));
  }
  __syncthreads();
  {
    const int b = l16 >> 3, c = l16 & 7, gq = c >> 1, l0 = 16 * (c & 1);
    const float* sp = s_k + 256 * b + 64 * gq + l0;
    float xl[16], xh[16], sxl = 0.0f, sxh = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      xl[i] = sp[i];
      xh[i] = sp[32 + i];
      sxl += xl[i];
      sxh += xh[i];
    }
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {
      const float v = row16_sum_f32(q4k_chunk_dot(dh[pass], dq[pass], gq, xl, xh, sxl, sxh));
      if (l16 == 0) {
        const int h = 64 * blk + 2 * (t >> 4) + pass;
        xstore(xb + XW_Y + slot * H + h, xenc(v));
        if (a.expert_raw) a.expert_raw[(size_t)slot * H + h] = v;
      }
    }
  }

  // ------------------------------------------------------------------------------ phase 4 --
  // y[k][8g..8g+7] for the 8 slots (two 16-byte groups each) and the shared gate, polled together
  // by lanes 0..16 of wave 0
  if (t < 17) {
    const int off[1] = {t < 16 ? 4 * (XW_Y + (t >> 1) * H + 8 * g) + 16 * (t & 1) : 4 * XW_GATE};
    uint4 yv[1];
    xwait4<1>(xr, off, err, yv);
    if (t < 16) {
      float* yo = &ys[t >> 1][4 * (t & 1)];
      yo[0] = xdec(yv[0].x); yo[1] = xdec(yv[0].y); yo[2] = xdec(yv[0].z); yo[3] = xdec(yv[0].w);
    } else {
      s_gate = xdec(yv[0].x);
    }
  }
  wave_sync();
  if (t < 8) {
    const int h = 8 * g + t;
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < K; ++j) {
      const int k = s_order[j];
      acc += s_w[k] * ys[k][t];
    }
    const float sh = s_gate * sh_raw[t];
    if (a.routed_sum) a.routed_sum[h] = acc;
    if (a.shared_out) a.shared_out[h] = sh;
    a.out[h] = resid + acc + sh;
  }
  // the last workgroup out advances the epoch for the next launch
  if (t == 0) {
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

size_t moe_layer_exchange_bytes() { return (size_t)2 * XW_BUF * 4; }

int moe_launch_decode_layer(const MoeDecodeLaunch& L, int* sync, uint32_t* xch, hipStream_t st) {
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
  a.norm_w = L.norm_w;
  a.norm_eps = L.norm_eps;
  if (L.x_dtype == MOE_DT_F32)
    hipLaunchKernelGGL(k_dec_layer<MOE_DT_F32>, dim3(kG), dim3(kThreads), 0, st, a);
  else
    hipLaunchKernelGGL(k_dec_layer<MOE_DT_BF16>, dim3(kG), dim3(kThreads), 0, st, a);
  return moe_check_launch("decode_layer");
}
