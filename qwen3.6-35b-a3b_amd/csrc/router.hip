// Router R1-R5 on gfx950 (specification/11-moe-block.md §11.2-§11.3; speccheck/moe_ref.py:318-363;
// engine/block_forward.py:614-636).
//
// R1 is correctly rounded: each logit is summed in f64 (x*W products are exact in f64), the
// f64 sum is rounded straight to bf16 (never via f32), and a per-logit error bound
// (n+2) * 2^-53 * 4 * ||x|| * ||W_e|| (Cauchy-Schwarz bound on sum|x_j W_j|) certifies that
// no bf16 rounding midpoint lies between the computed and the exact sum. A logit that fails the
// certificate is recomputed in double-double (error-free TwoSum accumulation) and rounded from
// that, with ties to even only where the double-double value sits on the midpoint itself.
//
// R3 reproduces torch's CPU topk bit for bit, including its order among equal probabilities:
// torch runs std::nth_element(k-1) + std::sort(first k-1) (libstdc++ introselect) when
// k*64 > n. One wave replays that partition sequence with each unguarded Hoare partition done in
// parallel: with A = positions whose value is not greater than the pivot (left-scan stops) in
// ascending order and B = positions whose value is not less than it (right-scan stops) in
// descending order, the sequential partition swaps A[m] <-> B[m] for every m with A[m] < B[m]
// and returns min(A[M], B[M-1]) for the first M where that fails. Ranks come from ballots.
#include <type_traits>

#include "common.h"
#include "moe_internal.h"
#include "router_dev.h"
#include "shared_small.h"

namespace moe {

// Router weights are bf16 (the synthetic configs, HF checkpoints) or f32 (the shipped artifact's
// ffn_gate_inp, engine/block_forward.py:221-231). Either way every x * W product is exact in f64
// (at most 24 + 24 significant bits), so the certificate below holds unchanged.
template <int WDT>
__device__ __forceinline__ double w_at(const void* w, size_t i) {
  if constexpr (WDT == MOE_DT_F32) return (double)reinterpret_cast<const float*>(w)[i];
  else return (double)bf16_to_f32(reinterpret_cast<const uint16_t*>(w)[i]);
}
// 8 consecutive weights from element i (i % 8 == 0)
template <int WDT>
__device__ __forceinline__ void w_load8(const void* w, size_t i, double* o) {
  if constexpr (WDT == MOE_DT_F32) {
    const float4 a = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(w) + i);
    const float4 b = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(w) + i + 4);
    o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w; o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
  } else {
    const uint4 v = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(w) + i);
    const uint32_t ww[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      o[2 * k] = bf16_to_f32(ww[k] & 0xFFFFu);
      o[2 * k + 1] = bf16_to_f32(ww[k] >> 16);
    }
  }
}
// 4 consecutive weights from element i (i % 4 == 0)
template <int WDT>
__device__ __forceinline__ void w_load4(const void* w, size_t i, double* o) {
  if constexpr (WDT == MOE_DT_F32) {
    const float4 a = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(w) + i);
    o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
  } else {
    const uint2 a = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(w) + i);
    o[0] = bf16_to_f32(a.x & 0xFFFFu); o[1] = bf16_to_f32(a.x >> 16);
    o[2] = bf16_to_f32(a.y & 0xFFFFu); o[3] = bf16_to_f32(a.y >> 16);
  }
}

// ----------------------------------------------------------------- R1, small T (T <= 256) -------
// One wave per (expert row, 8-token slice): the row (H <= 2048) is loaded once into registers,
// then the slice's tokens go kGemvU at a time with every x load of the group issued before the
// first use, and the group's wave reductions (dot, |x|^2) interleaved. grid = (ceil(E/4), ceil(T/8)),
// block = 256 (4 waves). Each logit: f64 dot (products exact), certified bf16 rounding, the
// double-double recompute where the certificate does not hold.
constexpr int kGemvCh = 4;                            // 512-wide chunks: H <= 2048
constexpr int kGemvU = 2;                             // tokens whose loads go out together

template <int DT>
__device__ __forceinline__ void load8f(const void* p, size_t i, float* o) {
  if constexpr (DT == MOE_DT_F32) {
    const float4 a = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(p) + i);
    const float4 b = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(p) + i + 4);
    o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w; o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
  } else {
    const uint4 v = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(p) + i);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      o[2 * k] = bf16_to_f32(w[k] & 0xFFFFu);
      o[2 * k + 1] = bf16_to_f32(w[k] >> 16);
    }
  }
}

template <int XDT, int WDT>
__device__ __noinline__ uint32_t gemv_dd_logit(const void* __restrict__ xv, const void* __restrict__ w,
                                               int t, int e, int H, int lane, double bval,
                                               double xsq, double wsq) {
  // double-double recompute, error-free per lane, then across the wave
  DD d = {0.0, 0.0};
  for (int k = lane; k < H; k += 64) {
    const double xk = (XDT == MOE_DT_F32)
                          ? (double)reinterpret_cast<const float*>(xv)[(size_t)t * H + k]
                          : (double)bf16_to_f32(reinterpret_cast<const uint16_t*>(xv)[(size_t)t * H + k]);
    d = dd_add(d, DD{xk * w_at<WDT>(w, (size_t)e * H + k), 0.0});   // product exact in f64
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    DD other = {__shfl_xor(d.hi, o, 64), __shfl_xor(d.lo, o, 64)};
    d = dd_add(d, other);
  }
  d = dd_add(d, DD{bval, 0.0});
  const double ddb = (double)(H + 64) * 0x1p-104 * 16.0 * (sqrt(xsq) * sqrt(wsq) + fabs(bval));
  return round_bf16_dd(d, ddb);
}

template <int XDT, int WDT>
__global__ __launch_bounds__(256) void k_router_logits_gemv(
    const void* __restrict__ xv, const void* __restrict__ w, const float* __restrict__ bias,
    int T, int H, int E, uint16_t* __restrict__ logits) {
  const int lane = threadIdx.x & 63;
  const int e = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (e >= E) return;
  const size_t wr = (size_t)e * H;                    // the row's first element
  const int nchunk = H / 512;                         // 8 weights per lane per chunk
  float wf[kGemvCh][8];
#pragma unroll
  for (int c = 0; c < kGemvCh; ++c)
    if (c < nchunk) load8f<WDT>(w, wr + c * 512 + lane * 8, wf[c]);
  double wsq = 0.0;
#pragma unroll
  for (int c = 0; c < kGemvCh; ++c)
    if (c < nchunk) {
#pragma unroll
      for (int i = 0; i < 8; ++i) wsq = fma((double)wf[c][i], (double)wf[c][i], wsq);
    }
  wsq = wave_sum_f64(wsq);
  const double bval = bias ? (double)bias[e] : 0.0;
  const int t0 = 8 * (int)blockIdx.y, t_end = min(T, t0 + 8);
  for (int tb = t0; tb < t_end; tb += kGemvU) {
    float xf[kGemvU][kGemvCh][8];
#pragma unroll
    for (int u = 0; u < kGemvU; ++u) {
      const int t = min(tb + u, t_end - 1);           // a clamped token is computed, not stored
#pragma unroll
      for (int c = 0; c < kGemvCh; ++c)
        if (c < nchunk) load8f<XDT>(xv, (size_t)t * H + c * 512 + lane * 8, xf[u][c]);
    }
    double acc[kGemvU], xsq[kGemvU];
#pragma unroll
    for (int u = 0; u < kGemvU; ++u) {
      acc[u] = 0.0;
      xsq[u] = 0.0;
#pragma unroll
      for (int c = 0; c < kGemvCh; ++c)
        if (c < nchunk) {
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            acc[u] = fma((double)xf[u][c][i], (double)wf[c][i], acc[u]);
            xsq[u] = fma((double)xf[u][c][i], (double)xf[u][c][i], xsq[u]);
          }
        }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
#pragma unroll
      for (int u = 0; u < kGemvU; ++u) {
        acc[u] += __shfl_xor(acc[u], o, 64);
        xsq[u] += __shfl_xor(xsq[u], o, 64);
      }
    }
#pragma unroll
    for (int u = 0; u < kGemvU; ++u) {
      const int t = tb + u;
      if (t >= t_end) break;
      const double s = acc[u] + bval;
      const double bound = 4.0 * (double)(H + 3) * 0x1p-53 * (sqrt(xsq[u]) * sqrt(wsq) + fabs(bval));
      uint32_t bits;
      if (!round_bf16_certified(s, bound, &bits))
        bits = gemv_dd_logit<XDT, WDT>(xv, w, t, e, H, lane, bval, xsq[u], wsq);
      if (lane == 0) logits[(size_t)t * E + e] = (uint16_t)bits;
    }
  }
}

// One wave's share of a 16 x 16 f64 tile: x[t0 + .][k] . W[e0 + .][k] over k in [kb, kb + kw)
// (kw % 64 == 0) on v_mfma_f64_16x16x4f64 (A: lane l holds x[t0 + l%16][k], B: W[e0 + l%16][k],
// k = k0 + 4(l/16) + i for the step's MFMA i; D: lane l, register j holds D[4j + l/16][l%16]),
// written to s_d[wave] with the rows' partial squared norms (s_xsq / s_wsq[wave]).
template <int XDT, int WDT>
__device__ __forceinline__ void tile_f64_partial(const void* __restrict__ xv, const void* __restrict__ w,
                                                 int T, int H, int E, int t0, int e0, int kb, int kw,
                                                 double (*s_d)[256], double (*s_xsq)[16],
                                                 double (*s_wsq)[16]) {
  using d4 = double __attribute__((ext_vector_type(4)));
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int tr = min(t0 + r, T - 1), er = min(e0 + r, E - 1);   // clamped rows: never stored
  d4 acc = {0, 0, 0, 0}, acc2 = acc;                  // two chains of dependent MFMAs
  double xsq = 0.0, wsq = 0.0;
#pragma unroll 4
  for (int k0 = kb; k0 < kb + kw; k0 += 64) {
    double a[4][4], b[4][4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const size_t kx = (size_t)k0 + 16 * u + 4 * g;
      if constexpr (XDT == MOE_DT_F32) {
        const float4 v = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(xv) + (size_t)tr * H + kx);
        a[u][0] = v.x; a[u][1] = v.y; a[u][2] = v.z; a[u][3] = v.w;
      } else {
        const uint2 v = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(xv) + (size_t)tr * H + kx);
        a[u][0] = bf16_to_f32(v.x & 0xFFFFu); a[u][1] = bf16_to_f32(v.x >> 16);
        a[u][2] = bf16_to_f32(v.y & 0xFFFFu); a[u][3] = bf16_to_f32(v.y >> 16);
      }
      w_load4<WDT>(w, (size_t)er * H + kx, b[u]);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (u & 1) acc2 = __builtin_amdgcn_mfma_f64_16x16x4f64(a[u][i], b[u][i], acc2, 0, 0, 0);
        else acc = __builtin_amdgcn_mfma_f64_16x16x4f64(a[u][i], b[u][i], acc, 0, 0, 0);
        xsq = fma(a[u][i], a[u][i], xsq);
        wsq = fma(b[u][i], b[u][i], wsq);
      }
  }
  // row norms over this wave's k range: sum the four lane groups
  xsq += __shfl_xor(xsq, 16, 64);
  xsq += __shfl_xor(xsq, 32, 64);
  wsq += __shfl_xor(wsq, 16, 64);
  wsq += __shfl_xor(wsq, 32, 64);
  if (g == 0) { s_xsq[wv][r] = xsq; s_wsq[wv][r] = wsq; }
#pragma unroll
  for (int j = 0; j < 4; ++j) s_d[wv][16 * (4 * j + g) + r] = acc[j] + acc2[j];
}

// ------------------------------------------------- R1, 8 <= T <= 256: f64 MFMA, K split by wave --
// Block = 8 waves on one tile of 16 tokens x 16 experts; wave w sums k in [w H/8, (w+1) H/8) with
// v_mfma_f64_16x16x4f64 (A: lane l holds x[t0 + l%16][k], B: W[e0 + l%16][k], k = k0 + 4(l/16) + i
// for the step's MFMA i; D: lane l, register j holds D[4j + l/16][l%16]). The 8 partial tiles are
// added through LDS in wave order, so the f64 sum has a fixed order; any order stays inside the
// certificate's bound 4(H+3) 2^-53 (|x||W_e| + |b|). Logits the bound does not settle are
// recomputed in double-double by one wave. grid = (ceil(T/16), ceil(E/16)), block = 512.
template <int XDT, int WDT>
__global__ __launch_bounds__(512) void k_router_logits_small(
    const void* __restrict__ xv, const void* __restrict__ w, const float* __restrict__ bias,
    int T, int H, int E, uint16_t* __restrict__ logits) {
  __shared__ double s_d[8][256];
  __shared__ double s_xsq[8][16], s_wsq[8][16];
  __shared__ int s_fail[256];
  const int tid = threadIdx.x, wv = tid >> 6;
  const int lane = tid & 63;
  const int t0 = blockIdx.x * 16, e0 = blockIdx.y * 16;
  tile_f64_partial<XDT, WDT>(xv, w, T, H, E, t0, e0, wv * (H / 8), H / 8, s_d, s_xsq, s_wsq);
  __syncthreads();
  if (tid < 256) {
    const int tt = tid >> 4, ee = tid & 15;            // D[tt][ee]: token t0 + tt, expert e0 + ee
    const int t = t0 + tt, e = e0 + ee;
    int fail = 0;
    if (t < T && e < E) {
      double sum = 0.0, xs = 0.0, ws = 0.0;
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        sum += s_d[q][tid];
        xs += s_xsq[q][tt];
        ws += s_wsq[q][ee];
      }
      const double bval = bias ? (double)bias[e] : 0.0;
      const double sv = sum + bval;
      const double bound = 4.0 * (double)(H + 3) * 0x1p-53 * (sqrt(xs) * sqrt(ws) + fabs(bval));
      uint32_t bits;
      if (round_bf16_certified(sv, bound, &bits)) logits[(size_t)t * E + e] = (uint16_t)bits;
      else fail = 1;
    }
    s_fail[tid] = fail;
  }
  __syncthreads();
  // uncertified logits (rare): wave 0 recomputes each in double-double
  if (wv == 0) {
    for (int base = 0; base < 256; base += 64) {
      uint64_t m = __ballot(s_fail[base + lane] != 0);
      while (m) {
        const int idx = base + __builtin_ctzll(m);
        m &= m - 1;
        const int t = t0 + (idx >> 4), e = e0 + (idx & 15);
        double xs = 0.0, ws = 0.0;
        for (int q = 0; q < 8; ++q) { xs += s_xsq[q][idx >> 4]; ws += s_wsq[q][idx & 15]; }
        const double bval = bias ? (double)bias[e] : 0.0;
        const uint32_t bits = gemv_dd_logit<XDT, WDT>(xv, w, t, e, H, lane, bval, xs, ws);
        if (lane == 0) logits[(size_t)t * E + e] = (uint16_t)bits;
      }
    }
  }
}

// Rare path of the certificate: one logit recomputed sequentially in double-double (each
// product is exact in f64, TwoSum accumulation), then rounded to bf16.
template <int XDT, int WDT>
__device__ __noinline__ uint32_t logit_dd_recompute(const void* __restrict__ xv,
                                                    const void* __restrict__ w, int t, int e,
                                                    int H, double bval, double xsq, double wsq) {
  DD d = {0.0, 0.0};
  for (int k = 0; k < H; ++k) {
    const double xk = (XDT == MOE_DT_F32)
                          ? (double)reinterpret_cast<const float*>(xv)[(size_t)t * H + k]
                          : (double)bf16_to_f32(reinterpret_cast<const uint16_t*>(xv)[(size_t)t * H + k]);
    d = dd_add(d, DD{xk * w_at<WDT>(w, (size_t)e * H + k), 0.0});
  }
  d = dd_add(d, DD{bval, 0.0});
  const double ddb = (double)(H + 64) * 0x1p-104 * 16.0 * (sqrt(xsq) * sqrt(wsq) + fabs(bval));
  return round_bf16_dd(d, ddb);
}

// ------------------------------------------------------- R1, large T: f64 MFMA tile GEMM -----
// v_mfma_f64_16x16x4f64 (A 16x4: lane l holds A[l%16][l/16]; B 4x16: lane l holds B[l/16][l%16];
// D 16x16 in 4 f64 registers: lane l, register j holds D[4j + l/16][l%16]). The contraction
// index is free to permute as long as A and B agree, so in a 16-wide k step lane group g = l/16
// owns k = 4g..4g+3 and feeds one of them to each of the step's 4 MFMAs: one 16-byte (f32 x)
// or 8-byte (bf16 x / W) load per operand row per step.
// Block = 4 waves = 32 tokens x 128 experts; wave w owns experts 32w..32w+31 as 2 x 2 tiles.
// Operands come straight from global memory through a 4-step register ring (x rows are shared by
// the block's waves in L1; W, 1 MB at E=256, stays in L2). Each logit gets the same certificate
// as every R1 kernel here: f64 summation in any order stays within 4 (H+3) 2^-53 ||x|| ||W_e||
// of the exact sum.
template <int XDT, int WDT>
struct RouterRaw {
  using XT = typename std::conditional<XDT == MOE_DT_F32, float4, uint2>::type;
  using WT = typename std::conditional<WDT == MOE_DT_F32, float4, uint2>::type;
  XT a0, a1;
  WT b0, b1;
};

template <int XDT>
__device__ __forceinline__ void router_cvt_x(const typename RouterRaw<XDT, MOE_DT_BF16>::XT& v, double* o) {
  if constexpr (XDT == MOE_DT_F32) {
    o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
  } else {
    o[0] = bf16_to_f32(v.x & 0xFFFFu); o[1] = bf16_to_f32(v.x >> 16);
    o[2] = bf16_to_f32(v.y & 0xFFFFu); o[3] = bf16_to_f32(v.y >> 16);
  }
}
__device__ __forceinline__ void router_cvt_w(uint2 v, double* o) {
  o[0] = bf16_to_f32(v.x & 0xFFFFu); o[1] = bf16_to_f32(v.x >> 16);
  o[2] = bf16_to_f32(v.y & 0xFFFFu); o[3] = bf16_to_f32(v.y >> 16);
}
__device__ __forceinline__ void router_cvt_w(float4 v, double* o) {
  o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
}

template <int XDT, int WDT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void
k_router_logits_mfma(const void* __restrict__ xv, const void* __restrict__ w,
                     const float* __restrict__ bias, int T, int H, int E,
                     uint16_t* __restrict__ logits) {
  using XT = typename RouterRaw<XDT, WDT>::XT;
  using WT = typename RouterRaw<XDT, WDT>::WT;
  using d4 = double __attribute__((ext_vector_type(4)));
  constexpr int D = 4;                                  // ring depth in 16-wide k steps
  const int lane = threadIdx.x & 63;
  const int r = lane & 15, g = lane >> 4;
  const int t0 = blockIdx.x * 32;
  const int e0 = blockIdx.y * 128 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) * 32;
  if (e0 >= E) return;
  // operand rows (clamped into range; results of clamped rows are never stored)
  const XT* xa = reinterpret_cast<const XT*>(
      reinterpret_cast<const char*>(xv) + ((size_t)min(t0 + r, T - 1) * H + 4 * g) * sizeof(XT) / 4);
  const XT* xb = reinterpret_cast<const XT*>(
      reinterpret_cast<const char*>(xv) + ((size_t)min(t0 + 16 + r, T - 1) * H + 4 * g) * sizeof(XT) / 4);
  const WT* wa = reinterpret_cast<const WT*>(
      reinterpret_cast<const char*>(w) + ((size_t)min(e0 + r, E - 1) * H + 4 * g) * sizeof(WT) / 4);
  const WT* wb = reinterpret_cast<const WT*>(
      reinterpret_cast<const char*>(w) + ((size_t)min(e0 + 16 + r, E - 1) * H + 4 * g) * sizeof(WT) / 4);
  // one 16-wide k step is 4 XT / 4 WT further along each row
  auto load = [&](RouterRaw<XDT, WDT>& q, int step) {
    q.a0 = xa[4 * step]; q.a1 = xb[4 * step];
    q.b0 = wa[4 * step]; q.b1 = wb[4 * step];
  };
  d4 c00 = {0, 0, 0, 0}, c01 = c00, c10 = c00, c11 = c00;  // [token half][expert half]
  double xsa = 0, xsb = 0, wsa = 0, wsb = 0;
  const int nst = H / 16;
  RouterRaw<XDT, WDT> q[D];
#pragma unroll
  for (int s = 0; s < D; ++s) load(q[s], s);
  for (int it = 0; it < nst; it += D) {
#pragma unroll
    for (int s = 0; s < D; ++s) {
      double a0[4], a1[4], b0[4], b1[4];
      router_cvt_x<XDT>(q[s].a0, a0);
      router_cvt_x<XDT>(q[s].a1, a1);
      router_cvt_w(q[s].b0, b0);
      router_cvt_w(q[s].b1, b1);
      if (it + s + D < nst) load(q[s], it + s + D);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        c00 = __builtin_amdgcn_mfma_f64_16x16x4f64(a0[i], b0[i], c00, 0, 0, 0);
        c01 = __builtin_amdgcn_mfma_f64_16x16x4f64(a0[i], b1[i], c01, 0, 0, 0);
        c10 = __builtin_amdgcn_mfma_f64_16x16x4f64(a1[i], b0[i], c10, 0, 0, 0);
        c11 = __builtin_amdgcn_mfma_f64_16x16x4f64(a1[i], b1[i], c11, 0, 0, 0);
        xsa = fma(a0[i], a0[i], xsa);
        xsb = fma(a1[i], a1[i], xsb);
        wsa = fma(b0[i], b0[i], wsa);
        wsb = fma(b1[i], b1[i], wsb);
      }
    }
  }
  // squared norms: sum the four lane groups; lane r then holds row r's (and column r's) norm
#pragma unroll
  for (int o = 16; o <= 32; o <<= 1) {
    xsa += __shfl_xor(xsa, o, 64);
    xsb += __shfl_xor(xsb, o, 64);
    wsa += __shfl_xor(wsa, o, 64);
    wsb += __shfl_xor(wsb, o, 64);
  }
  const d4* acc[4] = {&c00, &c01, &c10, &c11};
#pragma unroll
  for (int q4 = 0; q4 < 4; ++q4) {
    const int th = q4 >> 1, eh = q4 & 1;
    const int e = e0 + 16 * eh + r;
    const double wsq = eh ? wsb : wsa;
    const double bval = (bias && e < E) ? (double)bias[e] : 0.0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int row = 4 * j + g;                       // token row within the 16-row half
      const double xsq = __shfl(th ? xsb : xsa, row, 64);
      const int t = t0 + 16 * th + row;
      if (t >= T || e >= E) continue;
      const double s = (*acc[q4])[j] + bval;
      const double bound = 4.0 * (double)(H + 3) * 0x1p-53 * (sqrt(xsq) * sqrt(wsq) + fabs(bval));
      uint32_t bits;
      if (!round_bf16_certified(s, bound, &bits))
        bits = logit_dd_recompute<XDT, WDT>(xv, w, t, e, H, bval, xsq, wsq);
      logits[(size_t)t * E + e] = (uint16_t)bits;
    }
  }
}

// ---------------------------------------------------------------- R1, large T: f64 tile GEMM --
// Shapes the MFMA kernel does not take (H % 64 != 0): 64 tokens x 64 experts per block of 256
// threads; each thread owns a 4x4 patch.
template <int XDT, int WDT>
__global__ __launch_bounds__(256) void k_router_logits_gemm(
    const void* __restrict__ xv, const void* __restrict__ w, const float* __restrict__ bias,
    int T, int H, int E, uint16_t* __restrict__ logits) {

  __shared__ double xs[16][64 + 2];
  __shared__ double wsm[16][64 + 2];
  const int tid = threadIdx.x;
  const int t0 = blockIdx.y * 64, e0 = blockIdx.x * 64;
  const int tx = tid & 15, ty = tid >> 4;             // experts tx*4.., tokens ty*4..
  double acc[4][4] = {};
  double xsq[4] = {}, wsq[4] = {};
  const int lrow = tid >> 2, lk = (tid & 3) * 4;      // loader: row 0..63, 4 k-values
  for (int k0 = 0; k0 < H; k0 += 16) {
    {
      const int t = t0 + lrow;
      double v[4] = {0, 0, 0, 0};
      if (t < T) {
        if (XDT == MOE_DT_F32) {
          float4 a = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(xv) + (size_t)t * H + k0 + lk);
          v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        } else {
          uint2 a = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(xv) + (size_t)t * H + k0 + lk);
          v[0] = bf16_to_f32(a.x & 0xFFFFu); v[1] = bf16_to_f32(a.x >> 16);
          v[2] = bf16_to_f32(a.y & 0xFFFFu); v[3] = bf16_to_f32(a.y >> 16);
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) xs[lk + i][lrow] = v[i];
      const int e = e0 + lrow;
      double u[4] = {0, 0, 0, 0};
      if (e < E) w_load4<WDT>(w, (size_t)e * H + k0 + lk, u);
#pragma unroll
      for (int i = 0; i < 4; ++i) wsm[lk + i][lrow] = u[i];
    }
    __syncthreads();
#pragma unroll 4
    for (int k = 0; k < 16; ++k) {
      double a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) { a[i] = xs[k][ty * 4 + i]; b[i] = wsm[k][tx * 4 + i]; }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        xsq[i] = fma(a[i], a[i], xsq[i]);
        wsq[i] = fma(b[i], b[i], wsq[i]);
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fma(a[i], b[j], acc[i][j]);
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = t0 + ty * 4 + i;
    if (t >= T) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = e0 + tx * 4 + j;
      if (e >= E) continue;
      const double bval = bias ? (double)bias[e] : 0.0;
      const double s = acc[i][j] + bval;
      const double bound = 4.0 * (double)(H + 3) * 0x1p-53 * (sqrt(xsq[i]) * sqrt(wsq[j]) + fabs(bval));
      uint32_t bits;
      if (!round_bf16_certified(s, bound, &bits))
        bits = logit_dd_recompute<XDT, WDT>(xv, w, t, e, H, bval, xsq[i], wsq[j]);
      logits[(size_t)t * E + e] = (uint16_t)bits;
    }
  }
}

// exact_order = 0 (the block forward when no routing output is asked for) accepts the fast path's
// slot order when equal probabilities sit only inside the top K: the same experts and weights, and
// the combine sums in ascending expert id, so the block output is the same bits.
__global__ __launch_bounds__(64) void k_route_topk(const uint16_t* __restrict__ logits, int T,
                                                   int E, int K, float* __restrict__ probs,
                                                   int32_t* __restrict__ ids,
                                                   float* __restrict__ w_f32,
                                                   uint16_t* __restrict__ w_bf16,
                                                   int32_t* __restrict__ heap_flag,
                                                   int exact_order) {
  __shared__ TopkLds s;
  const int t = blockIdx.x;
  const int lane = threadIdx.x;
  if (t >= T) return;
  float p[4];
  route_softmax(logits + (size_t)t * E, E, lane, p);
  if (probs) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (64 * j + lane < E) probs[(size_t)t * E + 64 * j + lane] = p[j];
  }
  route_select_and_write(s, p, E, K, lane, ids + (size_t)t * K, w_f32 + (size_t)t * K,
                         w_bf16 + (size_t)t * K, heap_flag, exact_order != 0);
}

// E = 256, K = 8, many tokens: one wave per token, four per block. The fast path settles a token
// (32-bit keys, rank r's id and weight written by lane r); a token it cannot settle (a tie at the
// K-th place, or any tie when the caller reads the slot order) is replayed exactly by its wave
// (FUSED: up to kFusedReplayMaxT tokens, where the launch the replay would otherwise take costs
// more than it saves), or marked by ids[t][0] = -1 and left to k_route_replay8, so that with many
// tokens the slow replays run in their own launch instead of beside three fast waves on a SIMD.
template <bool FUSED>
__global__ __launch_bounds__(256) void k_route_topk8(const uint16_t* __restrict__ logits, int T,
                                                     float* __restrict__ probs,
                                                     int32_t* __restrict__ ids,
                                                     float* __restrict__ w_f32,
                                                     uint16_t* __restrict__ w_bf16,
                                                     int32_t* __restrict__ heap_flag,
                                                     int exact_order) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (int)(threadIdx.x >> 6);
  if (t >= T) return;
  float p[4];
  route_softmax(logits + (size_t)t * 256, 256, lane, p);
  if (probs) {
#pragma unroll
    for (int j = 0; j < 4; ++j) probs[(size_t)t * 256 + 64 * j + lane] = p[j];
  }
  int my_id;
  float my_val, tot;
  const int code = wave_topk32<8>(p, lane, my_id, my_val, tot);
  const bool replay = code == 2 || (code == 1 && exact_order);
  if (replay) {
    if constexpr (FUSED) {
      __shared__ TopkLds s[4];
      route_replay_and_write(s[threadIdx.x >> 6], p, 256, 8, lane, ids + (size_t)t * 8,
                             w_f32 + (size_t)t * 8, w_bf16 + (size_t)t * 8, heap_flag);
    } else if (lane == 0) {
      ids[(size_t)t * 8] = -1;
    }
  } else if (lane < 8) {
    const float wv = my_val / tot;
    ids[(size_t)t * 8 + lane] = my_id;
    w_f32[(size_t)t * 8 + lane] = wv;
    w_bf16[(size_t)t * 8 + lane] = (uint16_t)f32_to_bf16(wv);
  }
}

// The exact replay of torch's CPU topk for the tokens k_route_topk8 marked; every other wave
// returns at once.
__global__ __launch_bounds__(256) void k_route_replay8(const uint16_t* __restrict__ logits, int T,
                                                       int32_t* __restrict__ ids,
                                                       float* __restrict__ w_f32,
                                                       uint16_t* __restrict__ w_bf16,
                                                       int32_t* __restrict__ heap_flag) {
  __shared__ TopkLds s[4];
  const int lane = threadIdx.x & 63, wave = (int)(threadIdx.x >> 6);
  const int t = blockIdx.x * 4 + wave;
  if (t >= T || ids[(size_t)t * 8] != -1) return;
  float p[4];
  route_softmax(logits + (size_t)t * 256, 256, lane, p);
  route_replay_and_write(s[wave], p, 256, 8, lane, ids + (size_t)t * 8, w_f32 + (size_t)t * 8,
                         w_bf16 + (size_t)t * 8, heap_flag);
}

constexpr int kChainKS = 4;       // blocks per tile (K splits)
constexpr int kChainPart = 288;   // doubles per partial: 256 tile sums, 16 + 16 row norms
constexpr int kChainTiles = 256;  // tile counters (T <= 256, E = 256); 16 group counters follow
constexpr int kChainSortCnt = kChainTiles + 16;   // then the count of groups routed (the fused sort)
static_assert((kRouterCntWord + kChainSortCnt + 1) * 4 <= (int)kSyncBytes, "router counters in the sync words");

// ------------------------------------------- R1-R5 in one launch, 8 <= T <= 256, E = 256, K = 8 --
// The small-T R1 above runs one 16 x 16 tile per block, so at T = 64 it keeps 64 CUs busy for the
// whole K; here each tile's K is split over kChainKS blocks (grid = tiles x kChainKS: 256 blocks at
// T = 64), and the launches of R2-R5 are folded in:
//   1. every block: the f64 partial tile of its K range (wave partials added in wave order), written
//      with its partial row norms to scratch; then an arrival count per tile;
//   2. the tile's last block to arrive: the kChainKS partials added in split order (a fixed order;
//      any order stays inside the certificate's bound), the certified bf16 rounding (double-double
//      recompute where it does not settle), the logits stored; then an arrival count per 16-token
//      group;
//   3. the group's last tile to arrive: R2-R5 for the group's 16 tokens, two per wave, as
//      k_route_topk8; then the exact replays of the tokens the fast path could not settle, one
//      per wave.
// What one block hands to another (partials, logits) goes through agent-scope stores and loads,
// which meet past the XCDs' L2s, and every thread waits for its stores before the block's arrival
// is counted. (Fences would write back and invalidate whole L2s, 256 times per launch, under the
// shared expert's concurrent GEMMs.) Each last arriver resets its counter, so the words are zero
// again for the next launch (also under graph replay). Counters: cnt[tile] for tiles <
// kChainTiles, cnt[kChainTiles + group], then the groups routed (kChainSortCnt, with the fused
// sort). An arrival that reads a count its launch cannot produce (at least the number of
// arrivals: a workspace never initialised, or two launches overlapping on one workspace) sets
// MOE_STATUS_SYNC_STATE in the status word; that launch's routing outputs are then unspecified,
// and moe_workspace_init restores the counters. The last arrival is recognised modulo the number
// of arrivals, so whatever a counter held, each stage still runs once per launch: the sort always
// writes a tile list consistent with its own positions, which the grouped GEMMs then read.
// agent-scope (cross-XCD) stores and loads of the single-launch router's hand-offs
__device__ __forceinline__ void st_agent(double* p, double v) {
  __hip_atomic_store(reinterpret_cast<unsigned long long*>(p), (unsigned long long)__double_as_longlong(v),
                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ double ld_agent(const double* p) {
  return __longlong_as_double((long long)__hip_atomic_load(reinterpret_cast<const unsigned long long*>(p),
                                                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}
__device__ __forceinline__ void st16_agent(uint16_t* p, uint16_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int ld32_agent(const int32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// this thread's stores complete (acknowledged) before what follows; the signal fence keeps the
// compiler from moving them past the wait
__device__ __forceinline__ void stores_done() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// The stable grouping of the P = T * 8 pairs by expert (E = 256) by one 512-thread block: the
// positions of moe_launch_sort (pairs p = t * 8 + k ordered by expert, equal experts in ascending
// p; a stable counting sort, so any correct one gives the same positions), the offsets, the hit
// list, and the bm-row tile list in build_tiles_block's order (by decreasing 32-row group count,
// then ascending expert; an expert's full tiles before its partial one). The ids come from other
// blocks of the launch, so they are read by agent-scope loads. P <= 2048, bm <= 160.
struct ChainSortLds {
  int h[256], start[256], run[256];
  int wcnt[8][256];
  uint32_t tmp[4][4];
};
// inclusive prefix sum over the wave on DPP moves: row shifts by 1, 2, 4, 8 inside each 16-lane
// row (lanes shifted in from outside the row read 0), then the row totals carried by the row
// broadcasts of lanes 15 and 31 (the wave_sum_f32 pattern)
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v) {
  v += dpp_u32<0x111>(v);
  v += dpp_u32<0x112>(v);
  v += dpp_u32<0x114>(v);
  v += dpp_u32<0x118>(v);
  v += dpp_u32<0x142, 0xA>(v);
  v += dpp_u32<0x143, 0xC>(v);
  return v;
}
__device__ void chain_sort(const int32_t* __restrict__ ids, const MoeSortJob& j, ChainSortLds& s) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int P = j.P;
  if (tid < 256) {
    s.h[tid] = 0;
    s.run[tid] = 0;
  }
  __syncthreads();
  // pair tid + 512 q (q < 4), read once
  int idv[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int p = tid + 512 * q;
    idv[q] = p < P ? ld32_agent(ids + p) : -1;
    if ((unsigned)idv[q] < 256u) atomicAdd(&s.h[idv[q]], 1);
  }
  __syncthreads();
  // thread e < 256: expert e's count; exclusive prefixes of the counts, of the hit flags and of
  // the tile counts per 32-row group count g (10-bit fields, at most 2048 / 32 + 256 = 320 tiles:
  // g = 1..3 in one word, g = 4..5 in another) over the 256 experts
  const int e = tid;
  const int tot = e < 256 ? s.h[e] : 0, hit = tot > 0 ? 1 : 0;
  const int ngmax = (j.bm + 31) / 32;
  const int nfull = tot / j.bm, rem = tot - nfull * j.bm;
  const int grem = rem > 0 ? (rem + 31) / 32 : 0;
  auto fbit = [](int g) { return 10 * ((g - 1) % 3); };
  const uint32_t pk0 = (ngmax <= 3 ? (uint32_t)nfull << fbit(ngmax) : 0u) + (grem && grem <= 3 ? 1u << fbit(grem) : 0u);
  const uint32_t pk1 = (ngmax > 3 ? (uint32_t)nfull << fbit(ngmax) : 0u) + (grem > 3 ? 1u << fbit(grem) : 0u);
  const uint32_t it = wave_incl_scan((uint32_t)tot), ih = wave_incl_scan((uint32_t)hit);
  const uint32_t ip0 = wave_incl_scan(pk0), ip1 = wave_incl_scan(pk1);
  if (lane == 63 && wave < 4) {
    s.tmp[0][wave] = it;
    s.tmp[1][wave] = ih;
    s.tmp[2][wave] = ip0;
    s.tmp[3][wave] = ip1;
  }
  __syncthreads();
  if (tid < 256) {
    uint32_t b[4] = {0u, 0u, 0u, 0u}, tt[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const uint32_t v = s.tmp[q][w];
        b[q] += w < wave ? v : 0u;
        tt[q] += v;
      }
    }
    const int base = (int)(b[0] + it) - tot, hidx = (int)(b[1] + ih) - hit;
    const uint32_t pre0 = b[2] + ip0 - pk0, pre1 = b[3] + ip1 - pk1;
    s.start[e] = base;
    j.offsets[e] = base;
    if (hit) j.hits[1 + hidx] = e;
    if (e == 0) {
      j.offsets[256] = (int)tt[0];
      j.hits[0] = (int)tt[1];
    }
    auto field = [&](uint32_t w0, uint32_t w1, int g) { return (int)(((g <= 3 ? w0 : w1) >> fbit(g)) & 1023u); };
    const uint32_t tp0 = tt[2], tp1 = tt[3];
    int gstart[6] = {0, 0, 0, 0, 0, 0};
    int acc = 0;
    for (int g = ngmax; g >= 1; --g) {
      gstart[g] = acc;
      acc += field(tp0, tp1, g);
    }
    const int p_full = gstart[ngmax] + field(pre0, pre1, ngmax);
    for (int i = 0; i < nfull; ++i) {
      j.tiles[1 + 2 * (p_full + i)] = e;
      j.tiles[2 + 2 * (p_full + i)] = base + i * j.bm;
    }
    if (grem) {
      const int pt = gstart[grem] + field(pre0, pre1, grem) + (grem == ngmax ? nfull : 0);
      j.tiles[1 + 2 * pt] = e;
      j.tiles[2 + 2 * pt] = base + nfull * j.bm;
    }
    if (e == 0) j.tiles[0] = acc;
  }
  // the scatter, 512 pairs a round: ranks inside a wave from id matching (8 ballots on the id
  // bits), across waves from per-wave counts, across rounds from run[]
  const uint64_t lt = lane == 0 ? 0ull : (~0ull) >> (64 - lane);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    if (512 * q >= P) break;
    for (int i = tid; i < 8 * 256; i += 512) (&s.wcnt[0][0])[i] = 0;
    __syncthreads();
    const int p = tid + 512 * q;
    const bool valid = (unsigned)idv[q] < 256u;
    const int id = valid ? idv[q] : 0;
    if (p < P && !valid) j.pos[p] = -1;
    uint64_t peers = __ballot(valid);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const bool bit = (id >> b) & 1;
      const uint64_t m = __ballot(bit);
      peers &= bit ? m : ~m;
    }
    const int rank_w = __popcll(peers & lt);
    const bool leader = valid && rank_w == 0;
    if (leader) s.wcnt[wave][id] = __popcll(peers);
    __syncthreads();
    if (valid) {
      int before = 0;
#pragma unroll
      for (int w2 = 0; w2 < 8; ++w2) before += w2 < wave ? s.wcnt[w2][id] : 0;
      const int dest = s.start[id] + s.run[id] + before + rank_w;
      j.sorted[dest] = p;
      j.pos[p] = dest;
    }
    __syncthreads();
    if (leader) atomicAdd(&s.run[id], __popcll(peers));
  }
}

template <int XDT, int WDT>
__global__ __launch_bounds__(512) void k_router_chain(
    const void* __restrict__ xv, const void* __restrict__ w, const float* __restrict__ bias, int T,
    int H, int E, uint16_t* __restrict__ logits, float* __restrict__ probs, int32_t* __restrict__ ids,
    float* __restrict__ w_f32, uint16_t* __restrict__ w_bf16, int32_t* __restrict__ heap_flag,
    int exact_order, double* __restrict__ part, int* __restrict__ cnt, int* __restrict__ status,
    uint16_t* __restrict__ x16, MoeShJob sh, MoeSortJob srt) {
  // the router blocks' arrays, or the shared-expert blocks' partial tiles, in one LDS region
  struct Chain {
    double d[8][256];
    double xsq[8][16], wsq[8][16];
    double xt[16], wt[16];
    int fail[256];
    int last, nrep;
    int rep[16];
    TopkLds tk[8];
    float prep[16][256];   // the probabilities of the group's tokens that the replays take
  };
  __shared__ __attribute__((aligned(16))) union {
    Chain c;
    float red[shs::red_floats<8>()];
    ChainSortLds srt;
  } sm;
  const int tid = threadIdx.x, wv = tid >> 6, lane = tid & 63;
  const int nr = (int)gridDim.x - sh.n;
  if ((int)blockIdx.x >= nr) {
    // the small-T shared expert's gate/up tile (32 token rows x 16 columns), x read as it is,
    // then the scalar gate of this block's share of the tokens
    const int b = (int)blockIdx.x - nr, nslab = sh.Is / 16;
    shs::gateup_tile<XDT, 8, 32>(xv, sh.w0, sh.w1, T, H, sh.Is, b % nslab, (b / nslab) * 32, sh.S, sm.red);
    shs::gate_rows<XDT>(xv, sh.wsg, sh.gdt, T, H, sh.gate_prob, b * 8 + wv, sh.n * 8);
    return;
  }
  auto& s_d = sm.c.d;
  auto& s_xsq = sm.c.xsq;
  auto& s_wsq = sm.c.wsq;
  auto& s_xt = sm.c.xt;
  auto& s_wt = sm.c.wt;
  auto& s_fail = sm.c.fail;
  auto& s_last = sm.c.last;
  auto& s_nrep = sm.c.nrep;
  auto& s_rep = sm.c.rep;
  auto& s_tk = sm.c.tk;
  const int nE = E / 16;
  const int ks = blockIdx.x % kChainKS, tile = blockIdx.x / kChainKS;
  const int et = tile % nE, tg = tile / nE;
  const int t0 = tg * 16, e0 = et * 16;
  const int kw = H / (8 * kChainKS);
  if (x16 && et == 0) {
    // the f16 copy of x (k_to_f16's conversion): rows t0 .. t0 + 15, this block's K quarter
    const int kq = H / kChainKS, upr = kq / 8;
    for (int u = tid; u < 16 * upr; u += 512) {
      const int t = t0 + u / upr;
      if (t >= T) break;
      const size_t i = (size_t)t * H + (size_t)ks * kq + (size_t)(u % upr) * 8;
      uint4 o;
      if constexpr (XDT == MOE_DT_BF16) {
        const uint4 v = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(xv) + i);
        o = make_uint4(shs::f16x2_sat(bf16_to_f32(v.x & 0xFFFFu), bf16_to_f32(v.x >> 16)),
                       shs::f16x2_sat(bf16_to_f32(v.y & 0xFFFFu), bf16_to_f32(v.y >> 16)),
                       shs::f16x2_sat(bf16_to_f32(v.z & 0xFFFFu), bf16_to_f32(v.z >> 16)),
                       shs::f16x2_sat(bf16_to_f32(v.w & 0xFFFFu), bf16_to_f32(v.w >> 16)));
      } else {
        const float4 a = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(xv) + i);
        const float4 b = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(xv) + i + 4);
        o = make_uint4(shs::f16x2_sat(a.x, a.y), shs::f16x2_sat(a.z, a.w), shs::f16x2_sat(b.x, b.y),
                       shs::f16x2_sat(b.z, b.w));
      }
      *reinterpret_cast<uint4*>(x16 + i) = o;
    }
  }
  tile_f64_partial<XDT, WDT>(xv, w, T, H, E, t0, e0, ks * (H / kChainKS) + wv * kw, kw, s_d, s_xsq, s_wsq);
  __syncthreads();
  double* my = part + ((size_t)tile * kChainKS + ks) * kChainPart;
  if (tid < 256) {
    double sum = 0.0;
#pragma unroll
    for (int q = 0; q < 8; ++q) sum += s_d[q][tid];
    st_agent(&my[tid], sum);
  } else if (tid < 288) {
    const int i = tid - 256;
    double n = 0.0;
#pragma unroll
    for (int q = 0; q < 8; ++q) n += i < 16 ? s_xsq[q][i] : s_wsq[q][i - 16];
    st_agent(&my[tid], n);
  }
  stores_done();
  __syncthreads();
  if (tid == 0) {
    const int c = atomicAdd(&cnt[tile], 1);
    if (c >= kChainKS) atomicOr(status, MOE_STATUS_SYNC_STATE);   // a start this launch cannot produce
    s_last = (unsigned)c % kChainKS == kChainKS - 1;
  }
  __syncthreads();
  if (!s_last) return;
  if (tid == 0) __hip_atomic_store(&cnt[tile], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const double* tp = part + (size_t)tile * kChainKS * kChainPart;
  if (tid < 32) {
    double n = 0.0;
#pragma unroll
    for (int q = 0; q < kChainKS; ++q) n += ld_agent(&tp[q * kChainPart + 256 + tid]);
    if (tid < 16) s_xt[tid] = n;
    else s_wt[tid - 16] = n;
  }
  __syncthreads();
  if (tid < 256) {
    const int tt = tid >> 4, ee = tid & 15;            // D[tt][ee]: token t0 + tt, expert e0 + ee
    const int t = t0 + tt, e = e0 + ee;
    int fail = 0;
    if (t < T) {
      double sum = 0.0;
#pragma unroll
      for (int q = 0; q < kChainKS; ++q) sum += ld_agent(&tp[q * kChainPart + tid]);
      const double bval = bias ? (double)bias[e] : 0.0;
      const double sv = sum + bval;
      const double bound = 4.0 * (double)(H + 3) * 0x1p-53 * (sqrt(s_xt[tt]) * sqrt(s_wt[ee]) + fabs(bval));
      uint32_t bits;
      if (round_bf16_certified(sv, bound, &bits)) st16_agent(&logits[(size_t)t * E + e], (uint16_t)bits);
      else fail = 1;
    }
    s_fail[tid] = fail;
  }
  __syncthreads();
  if (wv == 0) {
    for (int base = 0; base < 256; base += 64) {
      uint64_t m = __ballot(s_fail[base + lane] != 0);
      while (m) {
        const int idx = base + __builtin_ctzll(m);
        m &= m - 1;
        const int t = t0 + (idx >> 4), e = e0 + (idx & 15);
        const double bval = bias ? (double)bias[e] : 0.0;
        const uint32_t bits = gemv_dd_logit<XDT, WDT>(xv, w, t, e, H, lane, bval, s_xt[idx >> 4], s_wt[idx & 15]);
        if (lane == 0) st16_agent(&logits[(size_t)t * E + e], (uint16_t)bits);
      }
    }
  }
  stores_done();
  __syncthreads();
  if (tid == 0) {
    const int c = atomicAdd(&cnt[kChainTiles + tg], 1);
    if (c >= nE) atomicOr(status, MOE_STATUS_SYNC_STATE);
    s_last = (unsigned)c % (unsigned)nE == (unsigned)nE - 1;
  }
  __syncthreads();
  if (!s_last) return;
  if (tid == 0) {
    __hip_atomic_store(&cnt[kChainTiles + tg], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_nrep = 0;
  }
  __syncthreads();
  // the fast path for the group's 16 tokens, two per wave; the tokens it cannot settle are listed
  // and replayed afterwards, one per wave, so that no wave runs two replays while others idle
  // both tokens' logits requested before either is used
  uint32_t raw[2][4];
#pragma unroll
  for (int j = 0; j < 2; ++j)
    route_logits_load<true>(logits + (size_t)min(t0 + 2 * wv + j, T - 1) * 256, 256, lane, raw[j]);
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int t = t0 + 2 * wv + j;
    if (t >= T) break;
    float p[4];
    route_softmax_raw(raw[j], 256, lane, p);
    if (probs) {
#pragma unroll
      for (int q = 0; q < 4; ++q) probs[(size_t)t * 256 + 64 * q + lane] = p[q];
    }
    int my_id;
    float my_val, tot;
    const int code = wave_topk32<8>(p, lane, my_id, my_val, tot);
    if (code == 2 || (code == 1 && exact_order)) {
#pragma unroll
      for (int q = 0; q < 4; ++q) sm.c.prep[t - t0][64 * q + lane] = p[q];
      if (lane == 0) s_rep[atomicAdd(&s_nrep, 1)] = t;
    } else if (lane < 8) {
      const float wv8 = my_val / tot;
      // read by the fused sort's block (another XCD) in this launch
      if (srt.P) __hip_atomic_store(&ids[(size_t)t * 8 + lane], my_id, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      else ids[(size_t)t * 8 + lane] = my_id;
      w_f32[(size_t)t * 8 + lane] = wv8;
      w_bf16[(size_t)t * 8 + lane] = (uint16_t)f32_to_bf16(wv8);
    }
  }
  __syncthreads();
#pragma unroll 1
  for (int i = wv; i < s_nrep; i += 8) {
    const int t = s_rep[i];
    // the fast path's probabilities (route_softmax's values: the same logits, the same arithmetic)
    float p[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) p[q] = sm.c.prep[t - t0][64 * q + lane];
    if (srt.P)
      route_replay_and_write<true>(s_tk[wv], p, 256, 8, lane, ids + (size_t)t * 8, w_f32 + (size_t)t * 8,
                                   w_bf16 + (size_t)t * 8, heap_flag);
    else
      route_replay_and_write(s_tk[wv], p, 256, 8, lane, ids + (size_t)t * 8, w_f32 + (size_t)t * 8,
                             w_bf16 + (size_t)t * 8, heap_flag);
  }
  if (!srt.P) return;
  // 4. the last group to finish its routing: the sort (every group's ids stored and acknowledged
  // before its arrival is counted)
  stores_done();
  __syncthreads();
  if (tid == 0) {
    const int ng = (T + 15) / 16;
    const int c = atomicAdd(&cnt[kChainSortCnt], 1);
    if (c >= ng) atomicOr(status, MOE_STATUS_SYNC_STATE);
    s_last = (unsigned)c % (unsigned)ng == (unsigned)ng - 1;
    if (s_last) __hip_atomic_store(&cnt[kChainSortCnt], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!s_last) return;
  chain_sort(ids, srt, sm.srt);
}

}  // namespace moe

using namespace moe;

template <int XDT, int WDT>
static void launch_router_logits(const void* x, const void* w, const float* bias, int T, int H,
                                 int E, uint16_t* logits, hipStream_t st) {
  if (T >= 8 && T <= 256 && H % 512 == 0) {
    hipLaunchKernelGGL((k_router_logits_small<XDT, WDT>), dim3((T + 15) / 16, (E + 15) / 16), dim3(512), 0,
                       st, x, w, bias, T, H, E, logits);
  } else if (T <= 256 && H <= 512 * kGemvCh) {
    hipLaunchKernelGGL((k_router_logits_gemv<XDT, WDT>), dim3((E + 3) / 4, (T + 7) / 8), dim3(256), 0, st,
                       x, w, bias, T, H, E, logits);
  } else if (H % 64 == 0) {
    hipLaunchKernelGGL((k_router_logits_mfma<XDT, WDT>), dim3((T + 31) / 32, (E + 127) / 128), dim3(256), 0, st,
                       x, w, bias, T, H, E, logits);
  } else {
    hipLaunchKernelGGL((k_router_logits_gemm<XDT, WDT>), dim3((E + 63) / 64, (T + 63) / 64), dim3(256), 0, st,
                       x, w, bias, T, H, E, logits);
  }
}

bool moe_router_chain_supported(int T, int H, int E, int K) {
  return T >= 8 && T <= 256 && E == 256 && K == 8 && H % (64 * 8 * kChainKS) == 0;
}

size_t moe_router_chain_scratch_bytes(int T, int E) {
  return (size_t)((T + 15) / 16) * (size_t)((E + 15) / 16) * kChainKS * kChainPart * sizeof(double);
}

size_t moe_router_scratch_bytes(int T, int H, int E) {
  const size_t a = moe_router_i8_scratch_bytes(T, H, E), b = moe_router_chain_scratch_bytes(T, E);
  return a > b ? a : b;
}

int moe_launch_router_chain(const void* x, int x_dtype, const void* w, int w_dtype, const float* bias,
                            int T, int H, int E, uint16_t* logits, float* probs, int32_t* ids,
                            float* w_f32, uint16_t* w_bf16, int32_t* heap_flag, bool exact_order,
                            void* scratch, int* sync, hipStream_t st, uint16_t* x16,
                            const MoeShJob* sh, const MoeSortJob* srt) {
  if (!moe_router_chain_supported(T, H, E, 8) || !scratch || !sync)
    return moe_set_error(MOE_E_UNSUPPORTED, "router_chain: needs 8 <= T <= 256, E = 256, K = 8, H %% 2048 == 0");
  const MoeShJob job = sh ? *sh : MoeShJob{};
  if (job.n) {
    if (job.T != T || job.H != H || job.Is % 256 || !job.w0 || !job.w1 || !job.S || !job.wsg || !job.gate_prob)
      return moe_set_error(MOE_E_UNSUPPORTED, "router_chain: shared-expert blocks need I_s %% 256 == 0 and every pointer");
    if (job.n != moe_shjob_gateup_blocks(T, job.Is))
      return moe_set_error(MOE_E_ARG, "router_chain: %d shared-expert blocks given, %d needed", job.n,
                           moe_shjob_gateup_blocks(T, job.Is));
  }
  const MoeSortJob sj = srt ? *srt : MoeSortJob{};
  if (sj.P) {
    if (sj.P != T * 8 || !sj.offsets || !sj.sorted || !sj.pos || !sj.hits || !sj.tiles || sj.bm < 32 || sj.bm > 160)
      return moe_set_error(MOE_E_ARG, "router_chain: the fused sort needs P = 8 T, 32 <= bm <= 160 and every output");
  }
  dim3 grid(((T + 15) / 16) * (E / 16) * kChainKS);
  grid.x += (unsigned)job.n;
  double* part = reinterpret_cast<double*>(scratch);
  int* cnt = sync + kRouterCntWord;
  const int eo = exact_order ? 1 : 0;
#define MOE_CHAIN(XD, WD)                                                                          \
  hipLaunchKernelGGL((k_router_chain<XD, WD>), grid, dim3(512), 0, st, x, w, bias, T, H, E, logits, \
                     probs, ids, w_f32, w_bf16, heap_flag, eo, part, cnt, sync + MOE_STATUS_WORD, x16, job, sj)
  if (x_dtype == MOE_DT_F32 && w_dtype == MOE_DT_F32) MOE_CHAIN(MOE_DT_F32, MOE_DT_F32);
  else if (x_dtype == MOE_DT_F32) MOE_CHAIN(MOE_DT_F32, MOE_DT_BF16);
  else if (w_dtype == MOE_DT_F32) MOE_CHAIN(MOE_DT_BF16, MOE_DT_F32);
  else MOE_CHAIN(MOE_DT_BF16, MOE_DT_BF16);
#undef MOE_CHAIN
  return moe_check_launch("router_chain");
}

int moe_launch_router_logits(const void* x, int x_dtype, const void* w, int w_dtype, const float* bias,
                             int T, int H, int E, uint16_t* logits, void* scratch,
                             size_t scratch_bytes, hipStream_t st) {
  if (scratch && moe_router_i8_supported(T, H, E) && scratch_bytes >= moe_router_i8_scratch_bytes(T, H, E))
    return moe_launch_router_logits_i8(x, x_dtype, w, w_dtype, bias, T, H, E, logits, scratch, st);
  if (x_dtype == MOE_DT_F32 && w_dtype == MOE_DT_F32)
    launch_router_logits<MOE_DT_F32, MOE_DT_F32>(x, w, bias, T, H, E, logits, st);
  else if (x_dtype == MOE_DT_F32)
    launch_router_logits<MOE_DT_F32, MOE_DT_BF16>(x, w, bias, T, H, E, logits, st);
  else if (w_dtype == MOE_DT_F32)
    launch_router_logits<MOE_DT_BF16, MOE_DT_F32>(x, w, bias, T, H, E, logits, st);
  else
    launch_router_logits<MOE_DT_BF16, MOE_DT_BF16>(x, w, bias, T, H, E, logits, st);
  return moe_check_launch("router_logits");
}

// up to this many tokens the exact replays run inside the top-k launch (measured at 4096 tokens:
// 3 µs per block step faster than the replays in their own launch)
constexpr int kFusedReplayMaxT = 4096;

int moe_launch_route_topk(const uint16_t* logits, int T, int E, int K, float* probs, int32_t* ids,
                          float* w_f32, uint16_t* w_bf16, int32_t* heap_flag, hipStream_t st,
                          bool exact_order) {
  if (E == 256 && K == 8 && T >= 16) {
    const dim3 grid((T + 3) / 4);
    if (T <= kFusedReplayMaxT) {
      hipLaunchKernelGGL(k_route_topk8<true>, grid, dim3(256), 0, st, logits, T, probs, ids, w_f32, w_bf16,
                         heap_flag, exact_order ? 1 : 0);
      return moe_check_launch("route_topk");
    }
    hipLaunchKernelGGL(k_route_topk8<false>, grid, dim3(256), 0, st, logits, T, probs, ids, w_f32, w_bf16,
                       heap_flag, exact_order ? 1 : 0);
    hipLaunchKernelGGL(k_route_replay8, grid, dim3(256), 0, st, logits, T, ids, w_f32, w_bf16, heap_flag);
    return moe_check_launch("route_topk");
  }
  hipLaunchKernelGGL(k_route_topk, dim3(T), dim3(64), 0, st, logits, T, E, K, probs, ids, w_f32,
                     w_bf16, heap_flag, exact_order ? 1 : 0);
  return moe_check_launch("route_topk");
}
