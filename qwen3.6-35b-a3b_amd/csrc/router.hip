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
#include "common.h"
#include "moe_internal.h"
#include "router_dev.h"

namespace moe {

// ------------------------------------------------------------------ R1, small T (T <= 8) -------
// One wave per expert row; the row (H bf16) is read once and applied to every token.
// grid.x = ceil(E/4), block = 256 (4 waves).
template <int XDT>
__global__ __launch_bounds__(256) void k_router_logits_gemv(
    const void* __restrict__ xv, const uint16_t* __restrict__ w, const float* __restrict__ bias,
    int T, int H, int E, uint16_t* __restrict__ logits) {
  const int lane = threadIdx.x & 63;
  const int e = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (e >= E) return;
  const uint16_t* wr = w + (size_t)e * H;
  const int nchunk = H / 512;                         // 8 bf16 per lane per chunk
  double wsq = 0.0;
  for (int c = 0; c < nchunk; ++c) {
    uint4 wv = *reinterpret_cast<const uint4*>(wr + c * 512 + lane * 8);
    const uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      double a = bf16_to_f32(ww[i] & 0xFFFFu), b = bf16_to_f32(ww[i] >> 16);
      wsq = fma(a, a, wsq);
      wsq = fma(b, b, wsq);
    }
  }
  wsq = wave_sum_f64(wsq);
  for (int t = 0; t < T; ++t) {
    double acc = 0.0, xsq = 0.0;
    for (int c = 0; c < nchunk; ++c) {
      uint4 wv = *reinterpret_cast<const uint4*>(wr + c * 512 + lane * 8);
      const uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w};
      float xf[8];
      if (XDT == MOE_DT_F32) {
        const float* xp = reinterpret_cast<const float*>(xv) + (size_t)t * H + c * 512 + lane * 8;
        float4 a = *reinterpret_cast<const float4*>(xp);
        float4 b = *reinterpret_cast<const float4*>(xp + 4);
        xf[0] = a.x; xf[1] = a.y; xf[2] = a.z; xf[3] = a.w;
        xf[4] = b.x; xf[5] = b.y; xf[6] = b.z; xf[7] = b.w;
      } else {
        const uint16_t* xp = reinterpret_cast<const uint16_t*>(xv) + (size_t)t * H + c * 512 + lane * 8;
        uint4 a = *reinterpret_cast<const uint4*>(xp);
        const uint32_t aa[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          xf[2 * i] = bf16_to_f32(aa[i] & 0xFFFFu);
          xf[2 * i + 1] = bf16_to_f32(aa[i] >> 16);
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const double w0 = bf16_to_f32(ww[i] & 0xFFFFu), w1 = bf16_to_f32(ww[i] >> 16);
        acc = fma((double)xf[2 * i], w0, acc);
        acc = fma((double)xf[2 * i + 1], w1, acc);
        xsq = fma((double)xf[2 * i], (double)xf[2 * i], xsq);
        xsq = fma((double)xf[2 * i + 1], (double)xf[2 * i + 1], xsq);
      }
    }
    acc = wave_sum_f64(acc);
    xsq = wave_sum_f64(xsq);
    double bval = bias ? (double)bias[e] : 0.0;
    const double s = acc + bval;
    const double bound = 4.0 * (double)(H + 3) * 0x1p-53 * (sqrt(xsq) * sqrt(wsq) + fabs(bval));
    uint32_t bits;
    bool ok = round_bf16_certified(s, bound, &bits);
    if (!ok) {
      // double-double recompute, error-free per lane, then across the wave
      DD d = {0.0, 0.0};
      for (int c = 0; c < nchunk; ++c) {
        uint4 wv = *reinterpret_cast<const uint4*>(wr + c * 512 + lane * 8);
        const uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          double xv_;
          if (XDT == MOE_DT_F32)
            xv_ = reinterpret_cast<const float*>(xv)[(size_t)t * H + c * 512 + lane * 8 + i];
          else
            xv_ = bf16_to_f32(reinterpret_cast<const uint16_t*>(xv)[(size_t)t * H + c * 512 + lane * 8 + i]);
          const double wv_ = bf16_to_f32((i & 1) ? (ww[i >> 1] >> 16) : (ww[i >> 1] & 0xFFFFu));
          d = dd_add(d, DD{xv_ * wv_, 0.0});          // product exact in f64
        }
      }
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) {
        DD other = {__shfl_xor(d.hi, o, 64), __shfl_xor(d.lo, o, 64)};
        d = dd_add(d, other);
      }
      d = dd_add(d, DD{bval, 0.0});
      const double ddb = (double)(H + 64) * 0x1p-104 * 16.0 * (sqrt(xsq) * sqrt(wsq) + fabs(bval));
      bits = round_bf16_dd(d, ddb);
    }
    if (lane == 0) logits[(size_t)t * E + e] = (uint16_t)bits;
  }
}

// ---------------------------------------------------------------- R1, large T: f64 tile GEMM --
// 64 tokens x 64 experts per block of 256 threads; each thread owns a 4x4 patch.
template <int XDT>
__global__ __launch_bounds__(256) void k_router_logits_gemm(
    const void* __restrict__ xv, const uint16_t* __restrict__ w, const float* __restrict__ bias,
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
      if (e < E) {
        uint2 a = *reinterpret_cast<const uint2*>(w + (size_t)e * H + k0 + lk);
        u[0] = bf16_to_f32(a.x & 0xFFFFu); u[1] = bf16_to_f32(a.x >> 16);
        u[2] = bf16_to_f32(a.y & 0xFFFFu); u[3] = bf16_to_f32(a.y >> 16);
      }
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
      if (!round_bf16_certified(s, bound, &bits)) {
        // rare: sequential double-double recompute of this one logit
        DD d = {0.0, 0.0};
        for (int k = 0; k < H; ++k) {
          double xk = (XDT == MOE_DT_F32)
                          ? (double)reinterpret_cast<const float*>(xv)[(size_t)t * H + k]
                          : (double)bf16_to_f32(reinterpret_cast<const uint16_t*>(xv)[(size_t)t * H + k]);
          d = dd_add(d, DD{xk * (double)bf16_to_f32(w[(size_t)e * H + k]), 0.0});
        }
        d = dd_add(d, DD{bval, 0.0});
        const double ddb = (double)(H + 64) * 0x1p-104 * 16.0 * (sqrt(xsq[i]) * sqrt(wsq[j]) + fabs(bval));
        bits = round_bf16_dd(d, ddb);
      }
      logits[(size_t)t * E + e] = (uint16_t)bits;
    }
  }
}

__global__ __launch_bounds__(64) void k_route_topk(const uint16_t* __restrict__ logits, int T,
                                                   int E, int K, float* __restrict__ probs,
                                                   int32_t* __restrict__ ids,
                                                   float* __restrict__ w_f32,
                                                   uint16_t* __restrict__ w_bf16,
                                                   int32_t* __restrict__ heap_flag) {
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
                         w_bf16 + (size_t)t * K, heap_flag);
}

}  // namespace moe

using namespace moe;

int moe_launch_router_logits(const void* x, int x_dtype, const void* w, const float* bias, int T,
                             int H, int E, uint16_t* logits, hipStream_t st) {
  const uint16_t* wr = reinterpret_cast<const uint16_t*>(w);
  if (T <= 8) {
    dim3 grid((E + 3) / 4);
    if (x_dtype == MOE_DT_F32)
      hipLaunchKernelGGL(k_router_logits_gemv<MOE_DT_F32>, grid, dim3(256), 0, st, x, wr, bias, T, H, E, logits);
    else
      hipLaunchKernelGGL(k_router_logits_gemv<MOE_DT_BF16>, grid, dim3(256), 0, st, x, wr, bias, T, H, E, logits);
  } else {
    dim3 grid((E + 63) / 64, (T + 63) / 64);
    if (x_dtype == MOE_DT_F32)
      hipLaunchKernelGGL(k_router_logits_gemm<MOE_DT_F32>, grid, dim3(256), 0, st, x, wr, bias, T, H, E, logits);
    else
      hipLaunchKernelGGL(k_router_logits_gemm<MOE_DT_BF16>, grid, dim3(256), 0, st, x, wr, bias, T, H, E, logits);
  }
  return moe_check_launch("router_logits");
}

int moe_launch_route_topk(const uint16_t* logits, int T, int E, int K, float* probs, int32_t* ids,
                          float* w_f32, uint16_t* w_bf16, int32_t* heap_flag, hipStream_t st) {
  hipLaunchKernelGGL(k_route_topk, dim3(T), dim3(64), 0, st, logits, T, E, K, probs, ids, w_f32,
                     w_bf16, heap_flag);
  return moe_check_launch("route_topk");
}
