// Router device helpers shared by the standalone and the fused decode kernels:
// certified f64 -> bf16 rounding of R1 and the wave-parallel replay of torch's CPU topk.
#pragma once
#include "common.h"

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
__host__ __device__ __forceinline__ int exp2_floor(double v) { return ilogb(v); }

// The bf16 rounding of the f64 value s (|s - exact| <= bound) into bits, and whether it is
// certified, i.e. no bf16 rounding midpoint lies within `bound` of s. Straight-line (selects, no early exits or
// conditional writes), so that a wave finishing many logits interleaves their dependency chains.
// bits is the bf16 rounding of s whether or not it is certified.
__host__ __device__ __forceinline__ bool round_bf16_sel(double s, double bound, uint32_t& bits) {
  const double a = fabs(s);
  const bool zero = a == 0.0;
  // zero: certified only if every value within the bound rounds to zero, i.e. the bound is below
  // half the smallest bf16 subnormal (the exact value may be a tiny non-zero)
  const bool ok_zero = !(bound > 0.0 && bound >= 0x1p-134);
  const int e = zero ? 0 : exp2_floor(a);
  const int qe = max(e - 7, -133);
  const double r = ldexp(a, -qe);                     // exact
  const double fl = floor(r);
  double dist = fabs((r - fl) - 0.5);                // in units of the quantum, exact
  // just above a power of two (fl == 128) the quantum below 2^e is half as wide, so the nearest
  // midpoint may be 2^e - q/4, at (r - 128) + 1/4 quanta, rather than 2^e + q/2; in the subnormal
  // range (qe == -133 below and above 2^e) the quantum does not change
  dist = (fl == 128.0 && qe > -133) ? fmin(dist, (r - fl) + 0.25) : dist;
  const double rounded = ldexp(rint(r), qe);          // rint: ties-to-even
  float f = (float)rounded;                           // exact (or inf on overflow)
  f = s < 0 ? -f : f;
  uint32_t fb;
  __builtin_memcpy(&fb, &f, 4);
  bits = zero ? 0u : fb >> 16;
  return zero ? ok_zero : !(ldexp(dist, qe) <= bound);
}

// round_bf16_sel with the bits written only when certified. (Host-callable, so the host tests can
// check it.)
__host__ __device__ __forceinline__ bool round_bf16_certified(double s, double bound, uint32_t* out) {
  uint32_t bits;
  const bool ok = round_bf16_sel(s, bound, bits);
  if (ok) *out = bits;
  return ok;
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
  // the nearest midpoint: fl + 1/2, or 2^e - q/4 (127.75 quanta) just above a power of two
  const bool below_pow2 = fl == 128.0 && qe > -133 && (r - fl) + 0.25 < fabs((r - fl) - 0.5);
  const double mq = below_pow2 ? 127.75 : fl + 0.5;
  // its two neighbours in quanta (127.5 = the largest bf16 below 2^e) and whether the upper
  // one is the even one (2^e is; so is fl + 1 when fl is odd)
  const double lo_n = below_pow2 ? 127.5 : fl, hi_n = below_pow2 ? 128.0 : fl + 1.0;
  const bool hi_even = below_pow2 || fmod(fl, 2.0) != 0.0;
  const double mid_abs = ldexp(mq, qe);
  const double mid = (sref < 0) ? -mid_abs : mid_abs;
  const double diff = (v.hi - mid) + v.lo;            // hi - mid is exact (close values)
  double n;                                           // magnitude in quanta after rounding
  if (fabs(diff) <= ddbound) {
    n = hi_even ? hi_n : lo_n;                        // tie: to even
  } else {
    const bool above = (sref < 0) ? (diff < 0) : (diff > 0);
    n = above ? hi_n : lo_n;
  }
  float f = (float)ldexp(n, qe);
  if (sref < 0) f = -f;
  return __float_as_uint(f) >> 16;
}

// ------------------------------------------------------------- R2-R5 with torch's tie order --
// One 64-thread block (one wave) per token. Queue positions 0..E-1 live in LDS; lane l owns
// positions l, l+64, l+128, l+192.
// LDS ordering among the lanes of one wave (the topk replay runs on a single wave, also inside
// larger workgroups, so it must not use a workgroup barrier).
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

struct __attribute__((aligned(16))) TopkLds {
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

// Stable descending insertion sort (libstdc++ __insertion_sort with greater) of positions
// [lo, lo + n), n <= 64, done by the wave:
// an element's final position is its rank, the number of elements greater than it plus the
// number of equal ones before it (insertion sort moves an element only past strictly smaller
// ones, so equal values keep their order).
__device__ void wave_stable_sort_small(TopkLds& s, int lo, int n, int lane) {
  float v = 0.0f;
  int id = 0;
  if (lane < n) { v = s.v[lo + lane]; id = s.i[lo + lane]; }
  int rank = 0;
  for (int j = 0; j < n; ++j) {
    const float vj = readlane_f32(v, j);
    rank += (vj > v || (vj == v && j < lane)) ? 1 : 0;
  }
  wave_sync();
  if (lane < n) { s.v[lo + rank] = v; s.i[lo + rank] = id; }
  wave_sync();
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

// ---- torch CPU topk(values, k) for k*64 > n: nth_element(k-1) then sort of the first k-1 ----
// (libstdc++ introselect: median-of-three pivot to the front, unguarded Hoare partition, until at
// most 3 elements remain or the depth limit 2 floor(log2 n) sends it to heap-select; then the
// insertion sorts). The partition rounds run on registers: lane l holds positions l + 64 j, as
// the f32 bits of the probabilities, which are >= +0, so their unsigned order is the float order
// and every comparison is an integer one (scalar where the operands are wave-uniform).
// value (or id bits) at position p: register p >> 6 (wave-uniform) of lane p & 63
__device__ __forceinline__ uint32_t reg_at(const uint32_t (&r)[4], int p) {
  // four reads and scalar selects: no branches
  const int l = p & 63, j = p >> 6;
  const uint32_t x0 = (uint32_t)__builtin_amdgcn_readlane((int)r[0], l);
  const uint32_t x1 = (uint32_t)__builtin_amdgcn_readlane((int)r[1], l);
  const uint32_t x2 = (uint32_t)__builtin_amdgcn_readlane((int)r[2], l);
  const uint32_t x3 = (uint32_t)__builtin_amdgcn_readlane((int)r[3], l);
  const uint32_t lo = (j & 1) ? x1 : x0, hi = (j & 1) ? x3 : x2;
  return (j & 2) ? hi : lo;
}
// number of set bits of m below this lane
__device__ __forceinline__ int lanes_below(uint64_t m) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// One unguarded Hoare partition of [a, b) around pv (the pivot, at a - 1), by rank pairing: the
// i-th stop of the left scan (an A position, !(v > pv)) trades places with the i-th stop of the
// right scan (a B position, !(pv > v)) while it lies to the left of it, which is the sequence of
// swaps the sequential scans make. Partners meet through LDS slots indexed by the rank (value and
// id as one 64-bit word; a swapping A element writes slot r of X and reads slot r of Y, a
// swapping B element the reverse), with no position lookup. Every register is processed under
// its in-range mask, without branches. Returns the cut, min(A[M], B[M-1], b) for M swaps.
__device__ int reg_partition(TopkLds& s, uint32_t (&v)[4], uint32_t (&id)[4], int a, int b,
                             uint32_t pv, int lane) {
  bool isA[4], isB[4];
  uint64_t mA[4], mB[4];
  int cA[5], cB[5];
  cA[0] = 0;
  cB[0] = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int pos = 64 * j + lane;
    const bool in = pos >= a && pos < b;
    isA[j] = in && v[j] <= pv;
    isB[j] = in && v[j] >= pv;
    mA[j] = __ballot(isA[j]);
    mB[j] = __ballot(isB[j]);
    cA[j + 1] = cA[j] + __popcll(mA[j]);
    cB[j + 1] = cB[j] + __popcll(mB[j]);
  }
  const int totB = cB[4];
  int rankA[4], rankB[4];
  bool swA[4], swB[4];
  int M = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    rankA[j] = cA[j] + lanes_below(mA[j]);                              // # A positions < pos
    rankB[j] = totB - cB[j] - lanes_below(mB[j]) - (isB[j] ? 1 : 0);   // # B positions > pos
    swA[j] = isA[j] && rankB[j] > rankA[j];
    swB[j] = isB[j] && rankA[j] > rankB[j];
    M += __popcll(__ballot(swA[j]));
  }
  // A[M] and B[M-1]: the positions holding those ranks (none: past the range)
  int cut = b;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint64_t fa = __ballot(isA[j] && rankA[j] == M);
    const uint64_t fb = __ballot(isB[j] && rankB[j] == M - 1);
    const int pa = fa ? 64 * j + (int)__builtin_ctzll(fa) : b;
    const int pb = fb ? 64 * j + (int)__builtin_ctzll(fb) : b;
    cut = min(cut, min(pa, pb));
  }
  if (M > 0) {
    // X = slots 0..191 and Y = slots 192..383 over s.v .. s.pb (ranks < M <= 128; lanes that do not
    // swap use slot 128 + lane of X, which no rank reaches); indices, not pointers, are selected,
    // so the exchange has no branches
    uint2* XY = reinterpret_cast<uint2*>(&s.v[0]);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int slot = swA[j] ? rankA[j] : (swB[j] ? 192 + rankB[j] : 128 + lane);
      XY[slot] = make_uint2(v[j], id[j]);
    }
    wave_sync();
    // all four reads issued by every lane before any result is used (the empty asm keeps the
    // compiler from turning them into reads under each lane's swap condition, one at a time)
    uint2 got[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int slot = swA[j] ? 192 + rankA[j] : (swB[j] ? rankB[j] : 128 + lane);
      got[j] = XY[slot];
    }
    asm volatile("" ::"v"(got[0].x), "v"(got[0].y), "v"(got[1].x), "v"(got[1].y), "v"(got[2].x),
                 "v"(got[2].y), "v"(got[3].x), "v"(got[3].y));
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool sw = swA[j] || swB[j];
      v[j] = sw ? got[j].x : v[j];
      id[j] = sw ? got[j].y : id[j];
    }
    wave_sync();
  }
  return cut;
}

// The same partition when [a - 1, b) lies in one register: x / xi hold positions base + lane.
__device__ int reg_partition1(TopkLds& s, uint32_t& x, uint32_t& xi, int a, int b, uint32_t pv,
                              int lane, int base) {
  const int pos = base + lane;
  const bool in = pos >= a && pos < b;
  const bool isA = in && x <= pv, isB = in && x >= pv;
  const uint64_t mA = __ballot(isA), mB = __ballot(isB);
  const int rankA = lanes_below(mA);
  const int rankB = __popcll(mB) - lanes_below(mB) - (isB ? 1 : 0);
  const bool swA = isA && rankB > rankA, swB = isB && rankA > rankB;
  const int M = __popcll(__ballot(swA));
  const uint64_t fa = __ballot(isA && rankA == M);
  const uint64_t fb = __ballot(isB && rankB == M - 1);
  int cut = b;
  if (fa) cut = min(cut, base + (int)__builtin_ctzll(fa));
  if (fb) cut = min(cut, base + (int)__builtin_ctzll(fb));
  if (M > 0) {
    uint2* XY = reinterpret_cast<uint2*>(&s.v[0]);
    XY[swA ? rankA : (swB ? 192 + rankB : 128 + lane)] = make_uint2(x, xi);
    wave_sync();
    const uint2 got = XY[swA ? 192 + rankA : (swB ? rankB : 128 + lane)];
    asm volatile("" ::"v"(got.x), "v"(got.y));
    const bool sw = swA || swB;
    x = sw ? got.x : x;
    xi = sw ? got.y : xi;
    wave_sync();
  }
  return cut;
}

// p holds the n values (lane + 64 j); the array goes to s.v / s.i (positions 0..n-1) when the
// rounds end, for the heap-select fallback and the final insertion sorts, which run on LDS.
// Returns 1 if the heap-select branch ran (reported for tests), 0 otherwise.
__device__ int wave_torch_topk_reg(TopkLds& s, const float* p, int n, int k, int lane) {
  uint32_t v[4], id[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    v[j] = __float_as_uint(p[j]);
    id[j] = (uint32_t)(64 * j + lane);
  }
  int lo = 0, hi = n;
  const int nth = k - 1;
  int depth = 2 * (31 - __clz(n));
  bool deep = false;
  while (hi - lo > 3) {
    if (depth == 0) { deep = true; break; }
    // once the range sits in one register it stays there: the rounds below work on that register
    if ((lo >> 6) == ((hi - 1) >> 6)) break;
    --depth;
    const int mid = lo + (hi - lo) / 2;
    // move_median_to_first(lo, lo+1, mid, hi-1) with comp = greater
    const int a = lo + 1, b = mid, c = hi - 1;
    const uint32_t va = reg_at(v, a), vb = reg_at(v, b), vc = reg_at(v, c);
    int pick;
    if (va > vb) {
      if (vb > vc) pick = b;
      else if (va > vc) pick = c;
      else pick = a;
    } else if (va > vc) pick = a;
    else if (vb > vc) pick = c;
    else pick = b;
    const uint32_t vlo = reg_at(v, lo), ilo = reg_at(id, lo);
    const uint32_t vpk = reg_at(v, pick), ipk = reg_at(id, pick);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int pos = 64 * j + lane;
      const bool at_lo = pos == lo, at_pk = pos == pick;
      v[j] = at_lo ? vpk : (at_pk ? vlo : v[j]);
      id[j] = at_lo ? ipk : (at_pk ? ilo : id[j]);
    }
    const int cut = reg_partition(s, v, id, lo + 1, hi, vpk, lane);
    if (cut <= nth) lo = cut;
    else hi = cut;
  }
  if (!deep && hi - lo > 3) {
    const int j0 = lo >> 6, base = 64 * j0;
    uint32_t x = j0 == 0 ? v[0] : (j0 == 1 ? v[1] : (j0 == 2 ? v[2] : v[3]));
    uint32_t xi = j0 == 0 ? id[0] : (j0 == 1 ? id[1] : (j0 == 2 ? id[2] : id[3]));
    while (hi - lo > 3) {
      if (depth == 0) { deep = true; break; }
      --depth;
      const int mid = lo + (hi - lo) / 2;
      const int a = lo + 1, b = mid, c = hi - 1;
      const uint32_t va = (uint32_t)__builtin_amdgcn_readlane((int)x, a - base);
      const uint32_t vb = (uint32_t)__builtin_amdgcn_readlane((int)x, b - base);
      const uint32_t vc = (uint32_t)__builtin_amdgcn_readlane((int)x, c - base);
      int pick;
      if (va > vb) {
        if (vb > vc) pick = b;
        else if (va > vc) pick = c;
        else pick = a;
      } else if (va > vc) pick = a;
      else if (vb > vc) pick = c;
      else pick = b;
      const uint32_t vlo = (uint32_t)__builtin_amdgcn_readlane((int)x, lo - base);
      const uint32_t ilo = (uint32_t)__builtin_amdgcn_readlane((int)xi, lo - base);
      const uint32_t vpk = (uint32_t)__builtin_amdgcn_readlane((int)x, pick - base);
      const uint32_t ipk = (uint32_t)__builtin_amdgcn_readlane((int)xi, pick - base);
      const bool at_lo = base + lane == lo, at_pk = base + lane == pick;
      x = at_lo ? vpk : (at_pk ? vlo : x);
      xi = at_lo ? ipk : (at_pk ? ilo : xi);
      const int cut = reg_partition1(s, x, xi, lo + 1, hi, vpk, lane, base);
      if (cut <= nth) lo = cut;
      else hi = cut;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[j] = j == j0 ? x : v[j];
      id[j] = j == j0 ? xi : id[j];
    }
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int pos = 64 * j + lane;
    if (pos < n) { s.v[pos] = __uint_as_float(v[j]); s.i[pos] = (int)id[j]; }
  }
  wave_sync();
  int heap = 0;
  if (deep) {
    if (lane == 0) {
      q_heap_select(s, lo, nth + 1, hi);
      qswap(s, lo, nth);
    }
    wave_sync();
    heap = 1;
  }
  if (!heap) wave_stable_sort_small(s, lo, hi - lo, lane);
  wave_stable_sort_small(s, 0, k - 1, lane);
  return heap;
}



// 64-bit unsigned wave max, every lane ends with the maximum (DPP inside rows, readlane across)
__device__ __forceinline__ uint64_t dpp_u64_max_step_b1(uint64_t v) {
  const uint64_t o = (uint64_t)dpp_u32<0xB1>((uint32_t)v) | ((uint64_t)dpp_u32<0xB1>((uint32_t)(v >> 32)) << 32);
  return o > v ? o : v;
}
template <int CTRL>
__device__ __forceinline__ uint64_t u64_max_step(uint64_t v) {
  const uint64_t o = (uint64_t)dpp_u32<CTRL>((uint32_t)v) | ((uint64_t)dpp_u32<CTRL>((uint32_t)(v >> 32)) << 32);
  return o > v ? o : v;
}
__device__ __forceinline__ uint64_t readlane_u64(uint64_t v, int l) {
  return (uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, l) |
         ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), l) << 32);
}
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
  v = u64_max_step<0xB1>(v);
  v = u64_max_step<0x4E>(v);
  v = u64_max_step<0x141>(v);
  v = u64_max_step<0x140>(v);
  const uint64_t r0 = readlane_u64(v, 15), r1 = readlane_u64(v, 31);
  const uint64_t r2 = readlane_u64(v, 47), r3 = readlane_u64(v, 63);
  const uint64_t a = r0 > r1 ? r0 : r1, b = r2 > r3 ? r2 : r3;
  return a > b ? a : b;
}

// Fast R3. Each lane holds positions lane, lane+64, lane+128, lane+192 (p[j] >= 0). Keys are
// (f32 bits << 8 | position): non-negative floats order like their bit patterns. K+1 rounds of a
// wave max pull the largest remaining key, giving the top min(K+1, E) in descending order.
// Returns 0 if those are all distinct (then this is exactly torch's answer), 1 if ties occur only
// inside the top K (the selected set and every weight are exact; only the slot order among equal
// probabilities may differ from torch's), 2 if the K-th and (K+1)-th are equal (the set itself
// depends on torch's tie order: the caller must run the full replay).
template <int KMAX>
__device__ __forceinline__ int wave_topk_fast(const float* p, int E, int K, int lane, int* ids,
                                              float* vals) {
  uint64_t k0, k1, k2, k3;
  {
    uint64_t kk[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int pos = 64 * j + lane;
      kk[j] = pos < E ? (((uint64_t)__float_as_uint(p[j])) << 8) | (uint64_t)pos : 0ull;
    }
    // sort the lane's four keys descending (5 compare-exchanges)
#define MOE_CX(a, b) { if (kk[a] < kk[b]) { uint64_t t_ = kk[a]; kk[a] = kk[b]; kk[b] = t_; } }
    MOE_CX(0, 1) MOE_CX(2, 3) MOE_CX(0, 2) MOE_CX(1, 3) MOE_CX(1, 2)
#undef MOE_CX
    k0 = kk[0]; k1 = kk[1]; k2 = kk[2]; k3 = kk[3];
  }
  const int rounds = min(K + 1, E);
  uint64_t prev = 0;
  bool inner_tie = false, boundary_tie = false;
#pragma unroll
  for (int r = 0; r < KMAX + 1; ++r) {
    if (r < rounds) {
      const uint64_t m = wave_max_u64(k0);
      if (k0 == m) { k0 = k1; k1 = k2; k2 = k3; k3 = 0ull; }
      if (r > 0 && (m >> 8) == (prev >> 8)) {
        if (r == K) boundary_tie = true;
        else inner_tie = true;
      }
      prev = m;
      if (r < K) {
        ids[r] = (int)(m & 255u);
        vals[r] = __uint_as_float((uint32_t)(m >> 8));
      }
    }
  }
  return boundary_tie ? 2 : (inner_tie ? 1 : 0);
}

// R2's exp, correctly rounded to f32 (the f64 exp's error is far below an f32 half-ulp, so one
// rounding of it lands on the nearest f32 except for arguments within ~2^-29 relative of an f32
// midpoint, none of which an exact f32 argument other than 0 reaches in practice). torch's CPU
// softmax evaluates its exps within one ulp of this; hipcc's expf is further off near zero, where
// distinct logits' probabilities sit within an ulp of each other and the last bit decides ties.
__device__ __forceinline__ float r2_exp(float a) { return (float)exp((double)a); }

// R2: softmax over E bf16 logits in f32 (max-subtracted, sum, multiply by the reciprocal — the
// same form as torch's CPU kernel); lane holds positions lane + 64j. AGENT: the logits were
// written by other workgroups of this launch through agent-scope stores, and are read likewise.
// (route_logits_load and route_softmax_raw: the same in two halves, so that a wave can have
// several tokens' loads in flight)
template <bool AGENT = false>
__device__ __forceinline__ void route_logits_load(const uint16_t* lg, int E, int lane, uint32_t* raw) {
  // clamped loads, all four in flight at once (guarded loads would each wait for the last)
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint16_t* a = lg + min(64 * j + lane, E - 1);
    if constexpr (AGENT) raw[j] = __hip_atomic_load(a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else raw[j] = *a;
  }
}
__device__ __forceinline__ void route_softmax_raw(const uint32_t* raw, int E, int lane, float* p) {
  float lv[4];
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    lv[j] = (64 * j + lane) < E ? bf16_to_f32(raw[j]) : -INFINITY;
    m = fmaxf(m, lv[j]);
  }
  m = wave_max_f32(m);
  float sum = 0.0f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    p[j] = (64 * j + lane) < E ? r2_exp(lv[j] - m) : 0.0f;
    sum += p[j];
  }
  sum = wave_sum_f32(sum);
  const float rs = 1.0f / sum;
#pragma unroll
  for (int j = 0; j < 4; ++j) p[j] *= rs;
}
template <bool AGENT = false>
__device__ __forceinline__ void route_softmax(const uint16_t* lg, int E, int lane, float* p) {
  uint32_t raw[4];
  route_logits_load<AGENT>(lg, E, lane, raw);
  route_softmax_raw(raw, E, lane, p);
}

// R3-R5 by the exact replay of torch's CPU topk (for ties that the fast paths cannot settle),
// then w = p_k / sum_k p_k (rank order) and its bf16 cast. Writes ids/w_f32/w_bf16[0..K) from
// lane 0. p: lane's probabilities at positions lane + 64j. AGENT_IDS: the ids by agent-scope
// stores, for a reader in another XCD during the same launch.
template <bool AGENT_IDS = false>
__device__ __forceinline__ void route_replay_and_write(TopkLds& s, const float* p, int E, int K,
                                                       int lane, int32_t* ids, float* w_f32,
                                                       uint16_t* w_bf16, int32_t* heap_flag) {
  const int heap = wave_torch_topk_reg(s, p, E, K, lane);
  if (lane == 0) {
    float tot = 0.0f;
    for (int k = 0; k < K; ++k) tot += s.v[k];
    for (int k = 0; k < K; ++k) {
      const float wv = s.v[k] / tot;
      if (AGENT_IDS) __hip_atomic_store(&ids[k], (int32_t)s.i[k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      else ids[k] = s.i[k];
      w_f32[k] = wv;
      w_bf16[k] = (uint16_t)f32_to_bf16(wv);
    }
    if (heap && heap_flag) atomicAdd(heap_flag, 1);
  }
  wave_sync();
}

// R3-R5 for one token by one wave: fast path, else the exact replay of torch's CPU topk; then
// w = p_k / sum_k p_k (rank order) and its bf16 cast. Writes ids/w_f32/w_bf16[0..K) from lane 0.
// exact_order = false accepts the fast path's slot order when ties sit only inside the top K
// (same set, same weights; used where only the block output is consumed).
__device__ __forceinline__ void route_select_and_write(TopkLds& s, const float* p, int E, int K,
                                                       int lane, int32_t* ids, float* w_f32,
                                                       uint16_t* w_bf16, int32_t* heap_flag,
                                                       bool exact_order = true) {
  int fid[16];
  float fval[16];
  const int code = wave_topk_fast<16>(p, E, K, lane, fid, fval);
  if (code == 0 || (code == 1 && !exact_order)) {
    if (lane == 0) {
      float tot = 0.0f;
#pragma unroll
      for (int k = 0; k < 16; ++k)
        if (k < K) tot += fval[k];
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        if (k < K) {
          const float wv = fval[k] / tot;
          ids[k] = fid[k];
          w_f32[k] = wv;
          w_bf16[k] = (uint16_t)f32_to_bf16(wv);
        }
      }
    }
    return;
  }
  route_replay_and_write(s, p, E, K, lane, ids, w_f32, w_bf16, heap_flag);
}

// Fast top-K over E = 256 probabilities (lane holds positions lane + 64j) with 32-bit keys: the
// lane sorts its four values, then K + 1 rounds each take the wave maximum (DPP row maxima + four
// readlanes) and pop it from the lowest lane that holds it. p >= 0, so the f32 bit patterns order
// like the values. Lane r < K ends with the rank-r id and value; *tot gets sum_k p_k in rank order.
// Returns 0 (no equal values among the first K + 1: torch's answer), 1 (equal values only inside
// the top K: same set and weights, slot order among equals may differ), 2 (the K-th and (K+1)-th
// are equal: the set depends on torch's tie order).
template <int K>
__device__ __forceinline__ int wave_topk32(const float* p, int lane, int& my_id, float& my_val,
                                           float& tot) {
  uint32_t k0 = __float_as_uint(p[0]), k1 = __float_as_uint(p[1]);
  uint32_t k2 = __float_as_uint(p[2]), k3 = __float_as_uint(p[3]);
  int p0 = lane, p1 = lane + 64, p2 = lane + 128, p3 = lane + 192;
#define MOE_CX32(a, b)                                     \
  {                                                        \
    const bool sw_ = k##a < k##b;                          \
    const uint32_t tk_ = sw_ ? k##b : k##a;                \
    k##b = sw_ ? k##a : k##b; k##a = tk_;                  \
    const int tp_ = sw_ ? p##b : p##a;                     \
    p##b = sw_ ? p##a : p##b; p##a = tp_;                  \
  }
  MOE_CX32(0, 1) MOE_CX32(2, 3) MOE_CX32(0, 2) MOE_CX32(1, 3) MOE_CX32(1, 2)
#undef MOE_CX32
  int code = 0;
  uint32_t prev = 0;
  float sum = 0.0f;
  my_id = 0;
  my_val = 0.0f;
#pragma unroll
  for (int r = 0; r <= K; ++r) {
    uint32_t m = k0;
    m = max(m, dpp_u32<0xB1>(m));
    m = max(m, dpp_u32<0x4E>(m));
    m = max(m, dpp_u32<0x141>(m));
    m = max(m, dpp_u32<0x140>(m));
    const uint32_t r0 = (uint32_t)__builtin_amdgcn_readlane((int)m, 15);
    const uint32_t r1 = (uint32_t)__builtin_amdgcn_readlane((int)m, 31);
    const uint32_t r2 = (uint32_t)__builtin_amdgcn_readlane((int)m, 47);
    const uint32_t r3 = (uint32_t)__builtin_amdgcn_readlane((int)m, 63);
    m = max(max(r0, r1), max(r2, r3));
    const uint64_t own = __ballot(k0 == m);
    const int owner = __builtin_ctzll(own);
    if (r > 0 && m == prev) code = (r == K) ? 2 : max(code, 1);
    prev = m;
    if (r < K) {
      const int id = __builtin_amdgcn_readlane(p0, owner);
      const float v = __uint_as_float(m);
      sum += v;
      if (lane == r) { my_id = id; my_val = v; }
      if (lane == owner) {
        k0 = k1; k1 = k2; k2 = k3; k3 = 0u;
        p0 = p1; p1 = p2; p2 = p3;
      }
    }
  }
  tot = sum;
  return code;
}

}  // namespace moe
