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

namespace moe {

// ------------------------------------------------------------------------- certified rounding --
struct DD { double hi, lo; };

__device__ __forceinline__ DD two_sum(double a, double b) {
  double s = a + b;
  double bb = s - a;
  double e = (a - (s - bb)) + (b - bb);
  return {s, e};
}
__device__ __forceinline__ DD dd_add(DD a, DD b) {
  DD s = two_sum(a.hi, b.hi);
  double lo = s.lo + a.lo + b.lo;
  return two_sum(s.hi, lo);
}

// exponent e with 2^e <= |v| < 2^(e+1), v != 0, v finite
__device__ __forceinline__ int exp2_floor(double v) { return ilogb(v); }

// Round the f64 value s (|s - exact| <= bound) to bf16. Returns false if not certified.
__device__ __forceinline__ bool round_bf16_certified(double s, double bound, uint32_t* out) {
  if (s == 0.0) {
    if (bound > 0.0) {
      // the exact value may be a tiny non-zero: certify only if every value within the bound
      // rounds to zero, i.e. the bound is below half the smallest bf16 subnormal
      if (bound >= ldexp(1.0, -134)) return false;
    }
    *out = 0u;
    return true;
  }
  const double a = fabs(s);
  const int e = exp2_floor(a);
  const int qe = max(e - 7, -133);
  const double r = ldexp(a, -qe);                     // exact
  const double fl = floor(r);
  const double dist = fabs((r - fl) - 0.5);          // in units of the quantum, exact
  if (ldexp(dist, qe) <= bound) return false;
  const double rounded = ldexp(rint(r), qe);          // rint: ties-to-even
  float f = (float)rounded;                           // exact (or inf on overflow)
  if (s < 0) f = -f;
  *out = __float_as_uint(f) >> 16;
  return true;
}

// Decide the bf16 rounding of hi+lo (double-double) whose error is below ddbound.
__device__ uint32_t round_bf16_dd(DD v, double ddbound) {
  uint32_t bits;
  if (round_bf16_certified(v.hi, fabs(v.lo) + ddbound, &bits)) return bits;
  // hi is within |lo| + ddbound of a midpoint: compare against that midpoint exactly.
  const double s = v.hi;
  if (s == 0.0 && v.lo == 0.0) return 0u;
  const double sref = (s != 0.0) ? s : v.lo;
  const double a = fabs(sref);
  const int qe = max(exp2_floor(a) - 7, -133);
  const double r = ldexp(a, -qe);
  const double fl = floor(r);
  const double mid_abs = ldexp(fl + 0.5, qe);
  const double mid = (sref < 0) ? -mid_abs : mid_abs;
  const double diff = (v.hi - mid) + v.lo;            // hi - mid is exact (close values)
  double n;                                           // magnitude in quanta after rounding
  if (fabs(diff) <= ddbound) {
    n = (fmod(fl, 2.0) == 0.0) ? fl : fl + 1.0;       // tie: to even
  } else {
    const bool above = (sref < 0) ? (diff < 0) : (diff > 0);
    n = above ? fl + 1.0 : fl;
  }
  float f = (float)ldexp(n, qe);
  if (sref < 0) f = -f;
  return __float_as_uint(f) >> 16;
}

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

// ------------------------------------------------------------- R2-R5 with torch's tie order --
// One 64-thread block (one wave) per token. Queue positions 0..E-1 live in LDS; lane l owns
// positions l, l+64, l+128, l+192.
struct TopkLds {
  float v[256];
  int i[256];
  int pa[256];
  int pb[256];
  int cell[2];
};

__device__ __forceinline__ void qswap(TopkLds& s, int a, int b) {
  float tv = s.v[a]; s.v[a] = s.v[b]; s.v[b] = tv;
  int ti = s.i[a]; s.i[a] = s.i[b]; s.i[b] = ti;
}

// greater-than on queue positions (values only; NaN does not occur on this path)
__device__ __forceinline__ bool qgt(const TopkLds& s, int a, int b) { return s.v[a] > s.v[b]; }

// stable insertion sort, descending, of positions [lo, hi) — lane 0 only
__device__ void q_insertion_sort(TopkLds& s, int lo, int hi) {
  for (int i = lo + 1; i < hi; ++i) {
    float v = s.v[i];
    int id = s.i[i];
    int j = i;
    while (j > lo && v > s.v[j - 1]) {
      s.v[j] = s.v[j - 1];
      s.i[j] = s.i[j - 1];
      --j;
    }
    s.v[j] = v;
    s.i[j] = id;
  }
}

// libstdc++ heap helpers, comparator "greater" — lane 0 only
__device__ void q_push_heap(TopkLds& s, int base, int hole, int top, float v, int id) {
  int parent = (hole - 1) / 2;
  while (hole > top && s.v[base + parent] > v) {
    s.v[base + hole] = s.v[base + parent];
    s.i[base + hole] = s.i[base + parent];
    hole = parent;
    parent = (hole - 1) / 2;
  }
  s.v[base + hole] = v;
  s.i[base + hole] = id;
}
__device__ void q_adjust_heap(TopkLds& s, int base, int hole, int len, float v, int id) {
  const int top = hole;
  int child = hole;
  while (child < (len - 1) / 2) {
    child = 2 * (child + 1);
    if (s.v[base + child] > s.v[base + child - 1]) child--;
    s.v[base + hole] = s.v[base + child];
    s.i[base + hole] = s.i[base + child];
    hole = child;
  }
  if ((len & 1) == 0 && child == (len - 2) / 2) {
    child = 2 * (child + 1);
    s.v[base + hole] = s.v[base + child - 1];
    s.i[base + hole] = s.i[base + child - 1];
    hole = child - 1;
  }
  q_push_heap(s, base, hole, top, v, id);
}
__device__ void q_heap_select(TopkLds& s, int lo, int mid, int hi) {
  const int n = mid - lo;
  if (n >= 2) {
    for (int parent = (n - 2) / 2;; --parent) {
      q_adjust_heap(s, lo, parent, n, s.v[lo + parent], s.i[lo + parent]);
      if (parent == 0) break;
    }
  }
  for (int i = mid; i < hi; ++i) {
    if (s.v[i] > s.v[lo]) {
      float v = s.v[i];
      int id = s.i[i];
      s.v[i] = s.v[lo];
      s.i[i] = s.i[lo];
      q_adjust_heap(s, lo, 0, n, v, id);
    }
  }
}

// Unguarded Hoare partition of [a, b) around the pivot at a-1, done by the whole wave.
__device__ int wave_partition(TopkLds& s, int a, int b, int lane) {
  const float pv = s.v[a - 1];
  const uint64_t lt = (lane == 0) ? 0ull : ((~0ull) >> (64 - lane));
  const uint64_t gt = (lane == 63) ? 0ull : ((~0ull) << (lane + 1));
  bool isA[4], isB[4];
  uint64_t mA[4], mB[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int pos = 64 * j + lane;
    const bool in = pos >= a && pos < b;
    const float v = in ? s.v[pos] : 0.0f;
    isA[j] = in && !(v > pv);
    isB[j] = in && !(pv > v);
    mA[j] = __ballot(isA[j]);
    mB[j] = __ballot(isB[j]);
  }
  int cA[5], cB[5];
  cA[0] = 0; cB[0] = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    cA[j + 1] = cA[j] + __popcll(mA[j]);
    cB[j + 1] = cB[j] + __popcll(mB[j]);
  }
  const int totB = cB[4];
  int rankA[4], rankB[4];
  bool swA[4], swB[4];
  int M = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    rankA[j] = cA[j] + __popcll(mA[j] & lt);                 // # A positions < pos
    rankB[j] = (totB - cB[j + 1]) + __popcll(mB[j] & gt);    // # B positions > pos
    swA[j] = isA[j] && rankB[j] > rankA[j];
    swB[j] = isB[j] && rankA[j] > rankB[j];
    M += __popcll(__ballot(swA[j]));
  }
  if (lane == 0) { s.cell[0] = 0x7FFFFFFF; s.cell[1] = 0x7FFFFFFF; }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int pos = 64 * j + lane;
    if (swA[j]) s.pa[rankA[j]] = pos;
    if (swB[j]) s.pb[rankB[j]] = pos;
    if (isA[j] && rankA[j] == M) s.cell[0] = pos;            // A[M]
    if (isB[j] && rankB[j] == M - 1) s.cell[1] = pos;        // B[M-1]
  }
  __syncthreads();
  float nv[4];
  int ni[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    int partner = -1;
    if (swA[j]) partner = s.pb[rankA[j]];
    if (swB[j]) partner = s.pa[rankB[j]];
    if (partner >= 0) { nv[j] = s.v[partner]; ni[j] = s.i[partner]; }
  }
  // min(A[M], B[M-1]); the median-of-three guarantees A[0] exists, the clamp only keeps a broken
  // invariant from indexing outside the range
  const int cut = min(min(s.cell[0], s.cell[1]), b);
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (swA[j] || swB[j]) { s.v[64 * j + lane] = nv[j]; s.i[64 * j + lane] = ni[j]; }
  }
  __syncthreads();
  return cut;
}

// torch CPU topk(values, k) for k*64 > n: nth_element(k-1) then sort of the first k-1.
// Returns 1 if the heap-select branch ran (reported for tests), 0 otherwise.
__device__ int wave_torch_topk(TopkLds& s, int n, int k, int lane) {
  int lo = 0, hi = n;
  const int nth = k - 1;
  int depth = 2 * (31 - __clz(n));
  int heap = 0;
  while (hi - lo > 3) {
    if (depth == 0) {
      if (lane == 0) {
        q_heap_select(s, lo, nth + 1, hi);
        qswap(s, lo, nth);
      }
      __syncthreads();
      heap = 1;
      break;
    }
    --depth;
    const int mid = lo + (hi - lo) / 2;
    if (lane == 0) {
      // move_median_to_first(lo, lo+1, mid, hi-1)
      const int a = lo + 1, b = mid, c = hi - 1;
      int pick;
      if (qgt(s, a, b)) {
        if (qgt(s, b, c)) pick = b;
        else if (qgt(s, a, c)) pick = c;
        else pick = a;
      } else if (qgt(s, a, c)) pick = a;
      else if (qgt(s, b, c)) pick = c;
      else pick = b;
      qswap(s, lo, pick);
    }
    __syncthreads();
    const int cut = wave_partition(s, lo + 1, hi, lane);
    if (cut <= nth) lo = cut;
    else hi = cut;
  }
  if (lane == 0) {
    if (!heap) q_insertion_sort(s, lo, hi);
    q_insertion_sort(s, 0, k - 1);
  }
  __syncthreads();
  return heap;
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
  float lv[4];
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int pos = 64 * j + lane;
    lv[j] = pos < E ? bf16_to_f32(logits[(size_t)t * E + pos]) : -INFINITY;
    m = fmaxf(m, lv[j]);
  }
  m = wave_max_f32(m);
  float ex[4], sum = 0.0f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int pos = 64 * j + lane;
    ex[j] = pos < E ? expf(lv[j] - m) : 0.0f;
    sum += ex[j];
  }
  sum = wave_sum_f32(sum);
  const float rs = 1.0f / sum;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int pos = 64 * j + lane;
    if (pos < E) {
      const float p = ex[j] * rs;
      s.v[pos] = p;
      s.i[pos] = pos;
      if (probs) probs[(size_t)t * E + pos] = p;
    }
  }
  __syncthreads();
  const int heap = wave_torch_topk(s, E, K, lane);
  if (lane == 0) {
    float tot = 0.0f;
    for (int k = 0; k < K; ++k) tot += s.v[k];
    for (int k = 0; k < K; ++k) {
      const float wv = s.v[k] / tot;
      ids[(size_t)t * K + k] = s.i[k];
      w_f32[(size_t)t * K + k] = wv;
      w_bf16[(size_t)t * K + k] = (uint16_t)f32_to_bf16(wv);
    }
    if (heap && heap_flag) atomicAdd(heap_flag, 1);
  }
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
