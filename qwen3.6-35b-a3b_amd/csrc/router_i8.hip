// R1 for large T on the int8 matrix cores (gfx950 v_mfma_i32_32x32x32_i8), correctly rounded to
// bf16 like every other R1 kernel here (speccheck/moe_ref.py:318-326: logits = bf16 of the exact
// sum x . W_e + b_e).
//
// Method: error-free splitting into integer digits (Ozaki, Ogita, Oishi, "Error-free
// transformations of matrix multiplication by using fast routines of matrix multiplication",
// Numer. Algorithms 59, 2012; integer form as in Ootomo, Ozaki, Yokota, "DGEMM on integer matrix
// multiplication unit", IJHPCA 2024).
//   * Every row v (an x row or a router row) gets its exponent E = floor(log2 max|v|) and the
//     integers N_k = rint(v_k 2^(S-E)), S = 8D - 3, so |N_k| < 2^(8D-2); v^_k = N_k 2^(E-S).
//   * N = sum_a d_a 256^(D-1-a) with balanced digits d_a in [-128, 127] (the bytes of
//     (N + 0x80..80) ^ 0x80..80); the top digit lies in [-64, 64].
//   * x^ . w^ = sum over digit pairs (a, b) of 2^(Ex+Ew-10-8(a+b)) * sum_k dx_a,k dw_b,k. Each
//     pair sum is an exact int32 (|d d'| <= 2^14, H <= 4096, at most 4 pairs share a level's
//     accumulator), so level l = a + b holds an exact integer.
//   * The levels are combined in f64 (Horner from the least significant level), scaled by
//     2^(Ex+Ew-10) (exact) and the bias is added. The distance to the exact sum x . w + b is at most
//       sum|x^-x| max|w^| + max|x| sum|w^-w|        (the rows' rounding to the digit grid)
//     + 2^-52 (sum of the Horner partials' magnitudes) 2^(Ex+Ew-10) + 2^-52 |s|  (f64 roundings),
//     and that bound certifies the bf16 rounding exactly as the f64 kernels' bound does. bf16
//     rows (x or router) use D = 3 digits (S = 21: a bf16 element is on the grid when within 2^14
//     of its row maximum), f32 x rows D = 4 (within 2^6), f32 router rows D = 5 (within 2^14);
//     what is left over is rare and bounded.
//   * A logit the bound does not certify is recomputed by its wave in double-double (the whole
//     wave sums the row in parallel) and rounded from that, ties to even on the midpoint itself.
//
// Kernels: k_router_prep (one wave per row: the row metadata and digit planes of the router rows
// and of the x rows), then k_router_i8 (64 tokens x 64 experts per block of 8 waves: two waves per
// 32 x 32 tile, each summing one k half of every 64-wide LDS stage, their int32 partial sums
// added through LDS at the end; digit planes staged global -> registers -> LDS one stage ahead).
#include <algorithm>
#include <type_traits>

#include "common.h"
#include "lds_dma.h"
#include "moe_internal.h"
#include "router_dev.h"

namespace moe {
namespace ri8 {

constexpr int kXDMax = 4;              // digits per x element, at most (scratch sizing)
constexpr int kKC = 64;                // k per LDS stage
constexpr int kRS = 80;                // LDS row stride (bytes): 16-byte slots of 8 rows distinct
constexpr int kMaxCh = 8;              // prep: 8-element chunks per lane, so H <= 4096

template <int XDT> struct XDig { static constexpr int D = (XDT == MOE_DT_F32) ? 4 : 3; };
template <int WDT> struct WDig { static constexpr int D = (WDT == MOE_DT_F32) ? 5 : 3; };
static_assert(XDig<MOE_DT_F32>::D <= kXDMax && XDig<MOE_DT_BF16>::D <= kXDMax, "x digit planes");

struct alignas(32) RowMeta {
  int e;          // row exponent E (0 for an all-zero row)
  int pad;
  double dsum;    // sum_k |v^_k - v_k|
  double vmax;    // max_k |v_k|
  double qmax;    // max_k |v^_k|
};

typedef int v4i __attribute__((ext_vector_type(4)));
// staging registers: vector types, so SROA keeps arrays of them in VGPRs (arrays of the struct
// type uint4 are left as allocas, which the backend then places in LDS)
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// Three digits on both sides (bf16 x, bf16 router rows): the digit planes are stored
// fragment-tiled, so that every MFMA operand (32 rows x 32 k of one plane, lane l holding row
// l % 32, k 16 (l / 32) .. + 15) is one contiguous kilobyte with lane l's 16 bytes at 16 l,
// operands ordered [row group r / 32][k chunk k / 32][digit]. Row groups run to a multiple of 64
// rows; the rows past T (or E) are never written and their sums never stored.
constexpr int kTD = 3;
template <int XDT, int WDT> constexpr bool tiled() {
  return XDig<XDT>::D == kTD && WDig<WDT>::D == kTD;
}
__host__ __device__ __forceinline__ size_t tiled_off(int r, int k, int C) {
  const size_t frag = ((size_t)(r >> 5) * C + (k >> 5)) * kTD;
  return (frag << 10) + ((size_t)((((k >> 4) & 1) << 5) | (r & 31)) << 4) + (k & 15);
}

template <int DT>
__device__ __forceinline__ float elt(const void* p, size_t i) {
  if constexpr (DT == MOE_DT_F32) return reinterpret_cast<const float*>(p)[i];
  else return bf16_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
}

// 8 consecutive elements from element i (i % 8 == 0)
template <int DT>
__device__ __forceinline__ void load8(const void* p, size_t i, float* o) {
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

__device__ __forceinline__ double wave_max_f64(double v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmax(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// ------------------------------------------------------------------------------ row metadata --
// Digits of 8 consecutive elements (n8: the integers N, |N| < 2^(8D-2)) into D planes, 8 bytes
// each: byte j of plane a = digit a of element j (plane 0 the most significant).
template <int D>
__device__ __forceinline__ void store_digits8(const double* n8, int8_t* dst, size_t plane) {
  if constexpr (D == 4) {
    // u = (N + 0x80808080) ^ 0x80808080 holds digit a in byte 3 - a; a 4 x 4 byte transpose per
    // group of four elements
    uint32_t u[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) u[j] = ((uint32_t)(int)n8[j] + 0x80808080u) ^ 0x80808080u;
    uint32_t p[4][2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const uint32_t* w = u + 4 * q;
      // t = [w0.b3 w1.b3 w0.b2 w1.b2], t2 = [w0.b1 w1.b1 w0.b0 w1.b0]; s, s2 likewise for w2, w3
      const uint32_t t = __builtin_amdgcn_perm(w[1], w[0], 0x06020703u);
      const uint32_t t2 = __builtin_amdgcn_perm(w[1], w[0], 0x04000501u);
      const uint32_t s = __builtin_amdgcn_perm(w[3], w[2], 0x06020703u);
      const uint32_t s2 = __builtin_amdgcn_perm(w[3], w[2], 0x04000501u);
      p[0][q] = __builtin_amdgcn_perm(s, t, 0x05040100u);
      p[1][q] = __builtin_amdgcn_perm(s, t, 0x07060302u);
      p[2][q] = __builtin_amdgcn_perm(s2, t2, 0x05040100u);
      p[3][q] = __builtin_amdgcn_perm(s2, t2, 0x07060302u);
    }
#pragma unroll
    for (int a = 0; a < 4; ++a) *reinterpret_cast<uint2*>(dst + a * plane) = make_uint2(p[a][0], p[a][1]);
  } else {
    uint64_t u[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      u[j] = ((uint64_t)(int64_t)n8[j] + 0x8080808080ull) ^ 0x8080808080ull;
#pragma unroll
    for (int a = 0; a < D; ++a) {
      const int b = 8 * (D - 1 - a);
      uint32_t lo = 0, hi = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) lo |= (uint32_t)((u[j] >> b) & 0xFF) << (8 * j);
#pragma unroll
      for (int j = 0; j < 4; ++j) hi |= (uint32_t)((u[4 + j] >> b) & 0xFF) << (8 * j);
      *reinterpret_cast<uint2*>(dst + a * plane) = make_uint2(lo, hi);
    }
  }
}

// One wave per row: rows 0..E-1 are the router rows (D = WD; planes [WD][E][H] in wdig), rows
// E..E+T-1 the x rows (D = XD; planes [XD][T][H] in xdig); the metadata goes to meta[t] for
// x rows and meta[T + e] for router rows. The router rows come first so that their longer
// digit work starts with the launch. grid = ceil((T+E)/4), block = 256.
template <int RD, int DT, bool TILED>
__device__ __forceinline__ void prep_row(const void* __restrict__ base, int r, int nrows, int H,
                                         int lane, RowMeta* __restrict__ m_out,
                                         int8_t* __restrict__ dig) {
  const size_t off = (size_t)r * H;
  const int nch = H / 512;                          // 8-element chunks per lane (<= kMaxCh)
  float v[kMaxCh][8];                               // the whole row stays in registers
#pragma unroll
  for (int c = 0; c < kMaxCh; ++c) {
    if (c >= nch) break;
    load8<DT>(base, off + (size_t)(c * 64 + lane) * 8, v[c]);
  }
  double vmax = 0.0;
#pragma unroll
  for (int c = 0; c < kMaxCh; ++c) {
    if (c >= nch) break;
#pragma unroll
    for (int j = 0; j < 8; ++j) vmax = fmax(vmax, (double)fabsf(v[c][j]));
  }
  vmax = wave_max_f64(vmax);
  const int e = vmax > 0.0 ? ilogb(vmax) : 0;
  const int sh = 8 * RD - 3 - e;
  double dsum = 0.0, qmax = 0.0;
  const size_t plane = (size_t)nrows * H;
#pragma unroll
  for (int c = 0; c < kMaxCh; ++c) {
    if (c >= nch) break;
    double n8[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const double y = ldexp((double)v[c][j], sh);  // exact
      const double n = rint(y);                     // ties to even
      dsum += fabs(y - n);
      qmax = fmax(qmax, fabs(n));
      n8[j] = n;
    }
    const int k = (c * 64 + lane) * 8;
    if constexpr (TILED) store_digits8<RD>(n8, dig + tiled_off(r, k, H >> 5), 1024);
    else store_digits8<RD>(n8, dig + off + k, plane);
  }
  dsum = wave_sum_f64(dsum);
  qmax = wave_max_f64(qmax);
  if (lane == 0) {
    RowMeta m;
    m.e = e;
    m.pad = 0;
    m.dsum = ldexp(dsum, -sh);
    m.vmax = vmax;
    m.qmax = ldexp(qmax, -sh);
    *m_out = m;
  }
}

template <int XDT, int WDT>
__global__ __launch_bounds__(256) void k_router_prep(const void* __restrict__ xv,
                                                     const void* __restrict__ w, int T, int H,
                                                     int E, RowMeta* __restrict__ meta,
                                                     int8_t* __restrict__ xdig,
                                                     int8_t* __restrict__ wdig) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= T + E) return;
  constexpr bool kTiled = tiled<XDT, WDT>();
  if (row < E) prep_row<WDig<WDT>::D, WDT, kTiled>(w, row, E, H, lane, meta + T + row, wdig);
  else prep_row<XDig<XDT>::D, XDT, kTiled>(xv, row - E, T, H, lane, meta + (row - E), xdig);
}

// ------------------------------------------------------------------------------ digit GEMM --
// Nothing moves across this: no memory access (a compiler memory barrier) and no instruction
// (a scheduling barrier).
__device__ __forceinline__ void fence_sched() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// One wave recomputes logit (t, e) in double-double: lane l sums k = 512 c + 8 l .. + 7 over the
// H / 512 chunks c (every x*W product is exact in f64) into four interleaved double-doubles, all
// of its elements loaded before the first add (the chunk index clamped, so the loads do not
// depend on H); the partial sums then meet in a butterfly. Bound as logit_dd_recompute's (at most
// H + 64 double-double adds on any path, whatever their order).
template <int XDT, int WDT>
__device__ uint32_t wave_dd_logit(const void* __restrict__ xv, const void* __restrict__ w, int t,
                                  int e, int H, double bval, int lane) {
  const int nch = H / 512;
  float xa[kMaxCh][8], wa[kMaxCh][8];
#pragma unroll
  for (int c = 0; c < kMaxCh; ++c) {
    const size_t k = (size_t)(min(c, nch - 1) * 64 + lane) * 8;
    load8<XDT>(xv, (size_t)t * H + k, xa[c]);
    load8<WDT>(w, (size_t)e * H + k, wa[c]);
  }
  DD d[4] = {{0.0, 0.0}, {0.0, 0.0}, {0.0, 0.0}, {0.0, 0.0}};
  double xsq = 0.0, wsq = 0.0;
#pragma unroll
  for (int c = 0; c < kMaxCh; ++c) {
    if (c >= nch) break;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const double xk = xa[c][j], wk = wa[c][j];
      d[j & 3] = dd_add(d[j & 3], DD{xk * wk, 0.0});
      xsq = fma(xk, xk, xsq);
      wsq = fma(wk, wk, wsq);
    }
  }
  DD s = dd_add(dd_add(d[0], d[1]), dd_add(d[2], d[3]));
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const DD p = {__shfl_xor(s.hi, o, 64), __shfl_xor(s.lo, o, 64)};
    s = dd_add(s, p);
    xsq += __shfl_xor(xsq, o, 64);
    wsq += __shfl_xor(wsq, o, 64);
  }
  s = dd_add(s, DD{bval, 0.0});
  const double ddb = (double)(H + 64) * 0x1p-104 * 16.0 * (sqrt(xsq) * sqrt(wsq) + fabs(bval));
  return round_bf16_dd(s, ddb);
}

// Row metadata of a block's 64 tokens (from t0) and 64 experts (from e0) into LDS (indices
// clamped; rows past T or E are never finished). Read after the block's next barrier.
__device__ __forceinline__ void stage_meta(RowMeta* sm, const RowMeta* __restrict__ meta, int t0,
                                           int e0, int T, int E, int tid) {
  if (tid < 64) sm[tid] = meta[min(t0 + tid, T - 1)];
  else if (tid < 128) sm[tid] = meta[T + min(e0 + tid - 64, E - 1)];
}

// The certified bf16 logits of one wave's 32 x 32 tile from its exact level sums (level l =
// the digit pairs a + b = l): register r of lane l holds token tb + 8 (r / 4) + 4 (l / 32) + r % 4
// and expert eb + l % 32; registers [r0, r1) are this wave's to finish. xm / wm: the row metadata
// of the block's tokens t0 .. t0 + 63 and experts e0 .. e0 + 63 (in LDS, tb - t0 and eb - e0 the
// tile's offsets in them). A logit the bound does not certify is recomputed by the whole wave in
// double-double (rare).
template <int XDT, int WDT, int NL>
__device__ __forceinline__ void finish_tile(const v16i (&acc)[NL], int r0, int r1, int t0, int tl,
                                            int e0, int el, const RowMeta* xm, const RowMeta* wm,
                                            const void* __restrict__ xv,
                                            const void* __restrict__ w,
                                            const float* __restrict__ bias, int T, int H, int E,
                                            int lane, uint16_t* __restrict__ logits) {
  const int tb = t0 + tl, eb = e0 + el;
  const int e = eb + (lane & 31);
  const bool e_ok = e < E;
  const RowMeta mw = wm[el + (lane & 31)];
  const double bval = (bias && e_ok) ? (double)bias[e] : 0.0;
  // every register's chain is computed first (no branches) so that the wave interleaves them;
  // the stores follow
  uint32_t fail = 0, okm = 0, bits[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int tr = tl + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
    const int t = t0 + tr;
    const bool live = r >= r0 && r < r1 && t < T && e_ok;
    const RowMeta mx = xm[tr];
    double v = (double)acc[NL - 1][r], cb = 0.0;
#pragma unroll
    for (int l = NL - 2; l >= 0; --l) {
      v = fma(v, 0x1p-8, (double)acc[l][r]);
      cb += fabs(v);
    }
    const int sc = mx.e + mw.e - 10;
    const double s = ldexp(v, sc) + bval;
    const double bound = (mx.dsum * mw.qmax + mx.vmax * mw.dsum) * (1.0 + 0x1p-32) +
                         ldexp(cb, sc) * 0x1p-52 + fabs(s) * 0x1p-52;
    const bool ok = round_bf16_sel(s, bound, bits[r]);
    okm |= (live && ok) ? 1u << r : 0u;
    fail |= (live && !ok) ? 1u << r : 0u;
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int t = t0 + tl + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
    if (okm >> r & 1) logits[(size_t)t * E + e] = (uint16_t)bits[r];
  }
  for (;;) {
    const uint64_t m = __ballot(fail != 0);
    if (m == 0) break;
    const int l0 = __builtin_ctzll(m);
    const int r = __builtin_ctz((uint32_t)__builtin_amdgcn_readlane((int)fail, l0));
    const int t = tb + 8 * (r >> 2) + 4 * (l0 >> 5) + (r & 3);
    const int ee = eb + (l0 & 31);
    const double bv = bias ? (double)bias[ee] : 0.0;
    const uint32_t bits = wave_dd_logit<XDT, WDT>(xv, w, t, ee, H, bv, lane);
    if (lane == l0) {
      logits[(size_t)t * E + ee] = (uint16_t)bits;
      fail &= ~(1u << r);
    }
  }
}

// grid = 8 * nE * ceil(nT / 8) blocks (nT = ceil(T/64) token tiles, nE = ceil(E/64) expert
// tiles), block = 256 (4 waves, 2 x 2 of 32 x 32). Blocks are dealt to the 8 XCDs round-robin;
// the nE blocks of one token tile share an XCD, so its x rows are fetched into one L2.
template <int XDT, int WDT>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void
k_router_i8(const void* __restrict__ xv, const void* __restrict__ w,
            const int8_t* __restrict__ xdig, const int8_t* __restrict__ wdig,
            const RowMeta* __restrict__ meta, const float* __restrict__ bias, int T, int H, int E,
            uint16_t* __restrict__ logits) {
  constexpr int WD = WDig<WDT>::D;
  constexpr int XD = XDig<XDT>::D;
  constexpr int NL = XD + WD - 1;                  // accumulator levels
  __shared__ __attribute__((aligned(16))) int8_t sx[2][XD][64 * kRS];
  __shared__ __attribute__((aligned(16))) int8_t sw[2][WD][64 * kRS];
  __shared__ RowMeta smeta[128];
  const int nT = (T + 63) / 64, nE = (E + 63) / 64;
  const int b = blockIdx.x, xcd = b & 7, jb = b >> 3;
  const int tt = xcd + 8 * (jb / nE), et = jb % nE;
  if (tt >= nT) return;
  const int t0 = tt * 64, e0 = et * 64;
  // 8 waves: wave (kh, q) owns the 32 x 32 tile q (2 x 2) for the k half kh of every stage
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  stage_meta(smeta, meta, t0, e0, T, E, tid);
  const int kh = wv >> 2, q4 = wv & 3;
  const int wm = q4 >> 1, wn = q4 & 1;
  // staging role: waves 0-3 copy the x planes, waves 4-7 the router planes; row (tid%256)/4 of
  // the tile, 16 bytes at 16 * (tid % 4) of each plane's stage slice
  const int st = tid & 255;
  const int srow = st >> 2, sseg = st & 3;
  const bool stage_x = kh == 0;
  const int8_t* src = stage_x ? xdig + (size_t)min(t0 + srow, T - 1) * H + 16 * sseg
                              : wdig + (size_t)min(e0 + srow, E - 1) * H + 16 * sseg;
  const size_t plane = stage_x ? (size_t)T * H : (size_t)E * H;
  const int soff = srow * kRS + 16 * sseg;

  // one register set: stage s + 1's digits (loaded during stage s - 1) go into the idle LDS
  // buffer at the start of stage s, the same registers then take stage s + 2's loads, then the
  // MFMAs of stage s run; one barrier per stage
  constexpr int NP = WD > XD ? WD : XD;
  u32x4 q[NP];
  auto gload = [&](int k0) {
    if (stage_x) {
#pragma unroll
      for (int a = 0; a < XD; ++a) q[a] = *reinterpret_cast<const u32x4*>(src + a * plane + k0);
    } else {
#pragma unroll
      for (int a = 0; a < WD; ++a) q[a] = *reinterpret_cast<const u32x4*>(src + a * plane + k0);
    }
  };
  auto lstore = [&](int buf) {
    if (stage_x) {
#pragma unroll
      for (int a = 0; a < XD; ++a) *reinterpret_cast<u32x4*>(&sx[buf][a][soff]) = q[a];
    } else {
#pragma unroll
      for (int a = 0; a < WD; ++a) *reinterpret_cast<u32x4*>(&sw[buf][a][soff]) = q[a];
    }
  };

  v16i acc[NL];
#pragma unroll
  for (int l = 0; l < NL; ++l) acc[l] = (v16i){};
  const int ar = (wm * 32 + (lane & 31)) * kRS + 16 * (lane >> 5);
  const int br = (wn * 32 + (lane & 31)) * kRS + 16 * (lane >> 5);
  auto mma = [&](int buf) {
    {
      const int ks = 32 * kh;
      v4i a[XD], bq[WD];
#pragma unroll
      for (int p = 0; p < XD; ++p) a[p] = *reinterpret_cast<const v4i*>(&sx[buf][p][ar + ks]);
#pragma unroll
      for (int q = 0; q < WD; ++q) bq[q] = *reinterpret_cast<const v4i*>(&sw[buf][q][br + ks]);
#pragma unroll
      for (int p = 0; p < XD; ++p)
#pragma unroll
        for (int q = 0; q < WD; ++q)
          acc[p + q] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[p], bq[q], acc[p + q], 0, 0, 0);
    }
  };
  const int nst = H / kKC;
  gload(0);
  lstore(0);
  if (nst > 1) gload(kKC);
  __syncthreads();
  for (int s = 0; s < nst; ++s) {
    const int buf = s & 1;
    if (s + 1 < nst) lstore(buf ^ 1);
    if (s + 2 < nst) gload((s + 2) * kKC);
    fence_sched();
    mma(buf);
    __syncthreads();
  }

  // the two k halves meet: wave (kh, q) keeps registers 8 kh .. 8 kh + 7 of every level and
  // takes the partner's partial sums for them through LDS (integer adds, exact)
  int32_t* xch = reinterpret_cast<int32_t*>(&sx[0][0][0]);
#pragma unroll
  for (int l = 0; l < NL; ++l) {
    if (kh == 0) {
#pragma unroll
      for (int j = 0; j < 8; ++j) xch[((q4 * 2 + 0) * 8 + j) * 64 + lane] = acc[l][8 + j];
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) xch[((q4 * 2 + 1) * 8 + j) * 64 + lane] = acc[l][j];
    }
    __syncthreads();
    if (kh == 0) {
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[l][j] += xch[((q4 * 2 + 1) * 8 + j) * 64 + lane];
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[l][8 + j] += xch[((q4 * 2 + 0) * 8 + j) * 64 + lane];
    }
    __syncthreads();
  }

  finish_tile<XDT, WDT, NL>(acc, 8 * kh, 8 * kh + 8, t0, wm * 32, e0, wn * 32, smeta, smeta + 64, xv,
                            w, bias, T, H, E, lane, logits);
}

// Tiled operands (bf16 x, bf16 router rows): grid as k_router_i8's, block = 256 (4 waves, one
// per SIMD; no LDS in the main loop). Wave (kh, n) = (w / 2, w % 2) sums the k chunks kh,
// kh + 2, ... of the block's 64 tokens x experts 32 n .. 32 n + 31 (two 32 x 32 tiles), its
// operands streamed straight into registers, nine kilobyte operands per chunk with two chunks in
// flight (the x operands are fetched by both waves of a k half, the second time from L1). The
// two k halves then meet through LDS: each wave keeps the tile of token half kh and hands the
// other one to its partner (w ^ 2); integer adds, exact.
template <int XDT, int WDT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 2))) void
k_router_i8t(const void* __restrict__ xv, const void* __restrict__ w,
             const int8_t* __restrict__ xdig, const int8_t* __restrict__ wdig,
             const RowMeta* __restrict__ meta, const float* __restrict__ bias, int T, int H, int E,
             uint16_t* __restrict__ logits) {
  static_assert(tiled<XDT, WDT>(), "three digits on both sides");
  constexpr int D = kTD, NL = 2 * D - 1;
  constexpr int kOps = 3 * D;                             // operands per chunk
  __shared__ __attribute__((aligned(16))) u32x4 xch[4][NL][4][64];
  __shared__ RowMeta smeta[128];
  const int nT = (T + 63) / 64, nE = (E + 63) / 64;
  const int b = blockIdx.x, xcd = b & 7, jb = b >> 3;
  const int tt = xcd + 8 * (jb / nE), et = jb % nE;
  if (tt >= nT) return;
  stage_meta(smeta, meta, 64 * tt, 64 * et, T, E, threadIdx.x);
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kh = wv >> 1, cg = wv & 1;
  const int C = H >> 5;                                   // k chunks
  const uint32_t gb = (uint32_t)C * D * 1024;             // bytes per 32-row group
  const auto rx = dma::rsrc(xdig, (int)(2u * nT * gb));
  const auto rw = dma::rsrc(wdig, (int)(2u * nE * gb));
  // local tile j covers token half j ^ kh: tile 0 is the one this wave keeps
  const uint32_t xo0 = (2u * tt + kh) * gb, xo1 = (2u * tt + (kh ^ 1)) * gb;
  const uint32_t wo = (2u * et + cg) * gb;
  const uint32_t voff = 16u * lane;
  // operands of chunk c: x tile 0 digits 0..2, x tile 1 digits 0..2, expert digits 0..2
  auto load = [&](u32x4 (&g)[kOps], int c) {
    const uint32_t co = (uint32_t)c * (D * 1024);
#pragma unroll
    for (int a = 0; a < D; ++a) {
      g[a] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, voff, xo0 + co + a * 1024, 0));
      g[D + a] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, voff, xo1 + co + a * 1024, 0));
      g[2 * D + a] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, voff, wo + co + a * 1024, 0));
    }
  };
  v16i acc[2][NL];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int l = 0; l < NL; ++l) acc[j][l] = (v16i){};
  auto mma = [&](const u32x4 (&g)[kOps]) {
#pragma unroll
    for (int a = 0; a < D; ++a)
#pragma unroll
      for (int c = 0; c < D; ++c)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[j][a + c] = __builtin_amdgcn_mfma_i32_32x32x32_i8(
              __builtin_bit_cast(v4i, g[D * j + a]), __builtin_bit_cast(v4i, g[2 * D + c]),
              acc[j][a + c], 0, 0, 0);
  };
  const int n = C >> 1;                                   // chunks per wave (a multiple of 8)
  // three chunks in flight: chunk i + 3 is loaded into the registers chunk i has just freed. The
  // fences keep each chunk's loads behind those MFMAs (the scheduler would otherwise gather the
  // loads and wait for all of them at once); the loads past the last chunk repeat it (in bounds,
  // unused) so every step waits for the same count.
  u32x4 f0[kOps], f1[kOps], f2[kOps];
  load(f0, kh);
  fence_sched();
  load(f1, kh + 2);
  fence_sched();
  load(f2, kh + 4);
  fence_sched();
  auto step = [&](u32x4 (&g)[kOps], int i) {
    if (i < n) mma(g);
    fence_sched();
    load(g, kh + 2 * min(i + 3, n - 1));
    fence_sched();
  };
  for (int i = 0; i < n; i += 3) {
    step(f0, i);
    step(f1, i + 1);
    step(f2, i + 2);
  }

  // the partner (other k half, same experts) takes tile 1, which is its tile 0
#pragma unroll
  for (int l = 0; l < NL; ++l)
#pragma unroll
    for (int q = 0; q < 4; ++q)
      xch[wv][l][q][lane] = (u32x4){(unsigned)acc[1][l][4 * q], (unsigned)acc[1][l][4 * q + 1],
                                    (unsigned)acc[1][l][4 * q + 2], (unsigned)acc[1][l][4 * q + 3]};
  __syncthreads();
#pragma unroll
  for (int l = 0; l < NL; ++l)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const u32x4 v = xch[wv ^ 2][l][q][lane];
      acc[0][l][4 * q] += (int)v.x;
      acc[0][l][4 * q + 1] += (int)v.y;
      acc[0][l][4 * q + 2] += (int)v.z;
      acc[0][l][4 * q + 3] += (int)v.w;
    }
  finish_tile<XDT, WDT, NL>(acc[0], 0, 16, 64 * tt, 32 * kh, 64 * et, 32 * cg, smeta, smeta + 64, xv,
                            w, bias, T, H, E, lane, logits);
}

// scratch: RowMeta[T + E] | x digit planes [XD][T][H] | router digit planes [WD][E][H] (sized
// for the most digits)
inline size_t meta_bytes(int T, int E) { return ((size_t)(T + E) * sizeof(RowMeta) + 255) / 256 * 256; }
inline size_t pad64(int n) { return (size_t)(n + 63) / 64 * 64; }
inline size_t xdig_bytes(int T, int H) {
  const size_t n = std::max((size_t)kXDMax * T, kTD * pad64(T)) * H;
  return (n + 255) / 256 * 256;
}
inline size_t wdig_bytes(int E, int H) {
  const size_t n = std::max((size_t)WDig<MOE_DT_F32>::D * E, kTD * pad64(E)) * H;
  return (n + 255) / 256 * 256;
}

template <int XDT, int WDT>
void launch(const void* x, const void* w, const float* bias, int T, int H, int E, uint16_t* logits,
            void* scratch, hipStream_t st) {
  RowMeta* meta = reinterpret_cast<RowMeta*>(scratch);
  int8_t* xdig = reinterpret_cast<int8_t*>(scratch) + meta_bytes(T, E);
  int8_t* wdig = xdig + xdig_bytes(T, H);
  hipLaunchKernelGGL((k_router_prep<XDT, WDT>), dim3((T + E + 3) / 4), dim3(256), 0, st, x, w, T, H,
                     E, meta, xdig, wdig);
  const int nT = (T + 63) / 64, nE = (E + 63) / 64;
  if constexpr (tiled<XDT, WDT>())
    hipLaunchKernelGGL((k_router_i8t<XDT, WDT>), dim3(8 * nE * ((nT + 7) / 8)), dim3(256), 0, st, x,
                       w, xdig, wdig, meta, bias, T, H, E, logits);
  else
    hipLaunchKernelGGL((k_router_i8<XDT, WDT>), dim3(8 * nE * ((nT + 7) / 8)), dim3(512), 0, st, x,
                       w, xdig, wdig, meta, bias, T, H, E, logits);
}

}  // namespace ri8
}  // namespace moe

using namespace moe;

size_t moe_router_i8_scratch_bytes(int T, int H, int E) {
  return ri8::meta_bytes(T, E) + ri8::xdig_bytes(T, H) + ri8::wdig_bytes(E, H);
}

bool moe_router_i8_supported(int T, int H, int E) {
  return T > 256 && H % 512 == 0 && H <= 512 * ri8::kMaxCh && E >= 1;
}

int moe_launch_router_logits_i8(const void* x, int x_dtype, const void* w, int w_dtype,
                                const float* bias, int T, int H, int E, uint16_t* logits,
                                void* scratch, hipStream_t st) {
  if (x_dtype == MOE_DT_F32 && w_dtype == MOE_DT_F32)
    ri8::launch<MOE_DT_F32, MOE_DT_F32>(x, w, bias, T, H, E, logits, scratch, st);
  else if (x_dtype == MOE_DT_F32)
    ri8::launch<MOE_DT_F32, MOE_DT_BF16>(x, w, bias, T, H, E, logits, scratch, st);
  else if (w_dtype == MOE_DT_F32)
    ri8::launch<MOE_DT_BF16, MOE_DT_F32>(x, w, bias, T, H, E, logits, scratch, st);
  else
    ri8::launch<MOE_DT_BF16, MOE_DT_BF16>(x, w, bias, T, H, E, logits, scratch, st);
  return moe_check_launch("router_logits_i8");
}
