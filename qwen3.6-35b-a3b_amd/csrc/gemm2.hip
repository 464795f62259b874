// Prefill-path grouped GEMM, register-fed form (gfx950, v_mfma_f32_32x32x16_f16, f32 accumulate).
//
// Work: one tile of up to 128 sorted (token, slot) rows of one expert (the device built list of
// k_build_tiles with 128-row tiles) times one output-column slab per block (XCD-aware order, see
// tile_rows). Block = 8 waves, two per SIMD so one wave's MFMAs overlap the other's decode and
// memory waits; wave w owns rows [64 (w >> 2), +64) of the tile and column group w & 3:
//   gate_up: gate rows n0 + 32 (w & 3) + (0..31) and the matching up rows; 2 x 32-row groups x
//            {gate, up} = 4 accumulator tiles; epilogue s = silu(gate) * up -> f16 S.
//   down:    down rows n0 + 64 (w & 3) + (0..63); 2 x 2 accumulator tiles; epilogue y in f32.
// Activations (f16 rows: x converted once, or S) go through LDS, double buffered, one barrier per
// 64-wide K step. Weights never touch LDS: each lane loads the bytes of its own MFMA B fragment
// (8 consecutive k of one weight row) and decodes them in registers, so a decoded weight feeds
// 64 rows of MFMA work. Row groups past the tile's last row skip their MFMAs.
//
// Q4_K decode to f16 (mantissa trick): a low nibble q placed in the low mantissa bits of the f16
// 0x6400 (= 1024) gives 1024 + q exactly, a high nibble left at bits 4-7 under 0x5400 (= 64, ulp
// 1/16) gives 64 + q; subtracting 1024 / 64 leaves q exactly, and one packed f16 FMA gives
// q * f16(d * sc) - f16(dmin * m). Against decoding in f32 and rounding once this adds
// the f16 rounding of the two per-sub-block factors (relative 2^-11 each); the block output stays
// far inside its tolerance (tests/test_gpu_experts.py, tests/test_gpu_block.py). bf16 weights
// (the shared expert) are converted to f16 exactly (every bf16 in f16's normal range is an f16).
// Element order inside a fragment is the natural k order, so the activations need no shuffle.
#include "common.h"
#include "moe_internal.h"

namespace moe {

typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kBM = MOE_GEMM2_BM;       // 128 rows per tile
constexpr int kBK = 64;                 // K per step
constexpr int kAS = 72;                 // LDS row stride in f16 (144 B: 16-B aligned rows)

struct Frag {                           // one MFMA operand: 8 f16
  uint32_t d[4];
};

__device__ __forceinline__ f32x16_t mfma(const uint4 a, const Frag& b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                               __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

// ------------------------------------------------------------------------------- Q4_K fragments --
struct Q4Scale {                        // packed f16x2 splats of (d*sc) and -(dmin*m)
  f16x2_t ds, ndm;
};

__device__ __forceinline__ Q4Scale q4_scale(uint4 hdr, int j) {
  uint32_t sc, m;
  q4k_scale_min(hdr.y, hdr.z, hdr.w, j, sc, m);
  const _Float16 ds = (_Float16)(f16_to_f32(hdr.x & 0xFFFFu) * (float)sc);
  const _Float16 dm = (_Float16)(-(f16_to_f32(hdr.x >> 16) * (float)m));
  Q4Scale r;
  r.ds = (f16x2_t){ds, ds};
  r.ndm = (f16x2_t){dm, dm};
  return r;
}

// One v_and_or_b32, the mask in a scalar register and the magic in a (loop-invariant) vector
// register: a gfx9 VOP3 takes no literal and at most one scalar operand, so the compiler would
// otherwise split it into v_and + v_or.
__device__ __forceinline__ uint32_t and_or_s(uint32_t p, uint32_t mask, uint32_t magic) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(p), "s"(mask), "v"(magic));
  return r;
}

// Low nibble q in mantissa bits 0-3 under 0x6400 (1024.0, ulp 1): 1024 + q. High nibble left in
// bits 4-7 under 0x5400 (64.0, ulp 1/16): 64 + q. Both exact; the subtraction leaves q exactly.
template <bool HIGH>
__device__ __forceinline__ uint32_t q4_pair(uint32_t w, uint32_t sel, const Q4Scale& s) {
  // bytes (b_a, b_b) of w -> f16x2 (off + nibble(b_a), off + nibble(b_b))
  const uint32_t p = __builtin_amdgcn_perm(0u, w, sel);
  const uint32_t magic = HIGH ? and_or_s(p, 0x00F000F0u, 0x54005400u)
                              : and_or_s(p, 0x000F000Fu, 0x64006400u);
  const _Float16 off = HIGH ? (_Float16)64.0f : (_Float16)1024.0f;
  const f16x2_t q = __builtin_bit_cast(f16x2_t, magic) - (f16x2_t){off, off};
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(q, s.ds, s.ndm));
}

// the 8 low (HIGH = false) or high nibbles of bytes w.x (b0..b3), w.y (b4..b7)
template <bool HIGH>
__device__ __forceinline__ Frag q4_frag(uint2 w, const Q4Scale& s) {
  Frag f;
  f.d[0] = q4_pair<HIGH>(w.x, 0x0C010C00u, s);
  f.d[1] = q4_pair<HIGH>(w.x, 0x0C030C02u, s);
  f.d[2] = q4_pair<HIGH>(w.y, 0x0C010C00u, s);
  f.d[3] = q4_pair<HIGH>(w.y, 0x0C030C02u, s);
  return f;
}

// ------------------------------------------------------------------------------- bf16 fragments --
__device__ __forceinline__ uint32_t bf2_to_f16x2(uint32_t w) {
  const f16x2_t v = {(_Float16)__uint_as_float(w << 16), (_Float16)__uint_as_float(w & 0xFFFF0000u)};
  return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ Frag bf_frag(uint4 w) {
  Frag f;
  f.d[0] = bf2_to_f16x2(w.x);
  f.d[1] = bf2_to_f16x2(w.y);
  f.d[2] = bf2_to_f16x2(w.z);
  f.d[3] = bf2_to_f16x2(w.w);
  return f;
}

// Raw bytes of one weight row for one K step, as one lane needs them (khalf h = lane >> 5).
//   Q4_K: hdr (16 B, the step's super-block) + bytes [8h, 8h+8) and [16+8h, 16+8h+8) of the
//         step's 32-byte nibble group; fragments s = 0,1 from the low nibbles, 2,3 from the high.
//   BF16: 4 x 16 B, fragment s = elements 16s + 8h .. +8.
template <int WFMT>
struct RowRaw;
template <>
struct RowRaw<MOE_FMT_Q4_K> {
  uint4 hdr;
  uint2 p0, p1;
  __device__ __forceinline__ void load(const uint8_t* row, int k0, int h) {
    const uint8_t* b = row + (size_t)(k0 >> 8) * 144;
    const int g = (k0 >> 6) & 3;
    hdr = *reinterpret_cast<const uint4*>(b);          // every step: the sets rotate mod 3
    p0 = *reinterpret_cast<const uint2*>(b + 16 + 32 * g + 8 * h);
    p1 = *reinterpret_cast<const uint2*>(b + 16 + 32 * g + 16 + 8 * h);
  }
  __device__ __forceinline__ void decode(int k0, Frag* f) const {
    const int g = (k0 >> 6) & 3;
    const Q4Scale lo = q4_scale(hdr, 2 * g), hi = q4_scale(hdr, 2 * g + 1);
    f[0] = q4_frag<false>(p0, lo);
    f[1] = q4_frag<false>(p1, lo);
    f[2] = q4_frag<true>(p0, hi);
    f[3] = q4_frag<true>(p1, hi);
  }
};
template <>
struct RowRaw<MOE_FMT_BF16> {
  uint4 q[4];
  __device__ __forceinline__ void load(const uint8_t* row, int k0, int h) {
    const uint16_t* r = reinterpret_cast<const uint16_t*>(row) + k0 + 8 * h;
#pragma unroll
    for (int s = 0; s < 4; ++s) q[s] = *reinterpret_cast<const uint4*>(r + 16 * s);
  }
  __device__ __forceinline__ void decode(int, Frag* f) const {
#pragma unroll
    for (int s = 0; s < 4; ++s) f[s] = bf_frag(q[s]);
  }
};

__device__ __forceinline__ size_t row_bytes2(int fmt, int cols) {
  return fmt == MOE_FMT_Q4_K ? (size_t)(cols / 256) * 144 : (size_t)cols * 2;
}

// ------------------------------------------------------------------------------ A tile (LDS) --
// Thread t stages row t / TPR, k columns [(64 / TPR) (t % TPR), +64 / TPR) of the step (TPR = 2:
// 4 x 16-byte loads; TPR = 4: 2). Rows past the tile's end read a valid row instead (their
// outputs are never stored), so the loads carry no branch.
template <int TPR>
struct ARaw {
  static constexpr int NV = 8 / TPR;
  uint4 v[NV];
  __device__ __forceinline__ void load(const uint16_t* src, int k0, int t) {
    const uint4* s = reinterpret_cast<const uint4*>(src + k0 + (64 / TPR) * (t % TPR));
#pragma unroll
    for (int j = 0; j < NV; ++j) v[j] = s[j];
  }
  __device__ __forceinline__ void store(uint16_t* As, int t) const {
    uint4* d = reinterpret_cast<uint4*>(As + (t / TPR) * kAS + (64 / TPR) * (t % TPR));
#pragma unroll
    for (int j = 0; j < NV; ++j) d[j] = v[j];
  }
};

__device__ __forceinline__ uint4 a_frag(const uint16_t* As, int mg, int s, int lane) {
  return *reinterpret_cast<const uint4*>(As + (32 * mg + (lane & 31)) * kAS + 16 * s + 8 * (lane >> 5));
}

// Block -> (tile, column slab), XCD-aware. Workgroups are dispatched round-robin over the 8 XCDs
// (block b runs on XCD b % 8), and each XCD has its own L2. XCD x takes a contiguous range of the
// tile list (tiles of one expert are adjacent in it) and walks each tile's column slabs
// consecutively: a tile's activation rows and an expert's weight slab are fetched once per XCD and
// then served from its L2. The tile count is read on the device; blocks past it exit.
constexpr int kXcd = 8;
__device__ __forceinline__ int tile_rows(const int32_t* tiles, const int32_t* offsets, int T,
                                         int ncol, int& e, int& m0, int& mend, int& col) {
  const int count = tiles ? tiles[0] : (T + kBM - 1) / kBM;
  const int per = (count + kXcd - 1) / kXcd;
  const int xcd = blockIdx.x % kXcd, slot = blockIdx.x / kXcd;
  const int tl = slot / ncol;
  col = slot % ncol;
  const int tile = xcd * per + tl;
  if (tl >= per || tile >= count) return 0;
  if (tiles) {
    e = tiles[1 + 2 * tile];
    m0 = tiles[2 + 2 * tile];
    mend = min(m0 + kBM, offsets[e + 1]);
  } else {
    e = 0;
    m0 = tile * kBM;
    mend = min(m0 + kBM, T);
  }
  return 1;
}

// ------------------------------------------------------------------------------- main loop --
// Block = NW waves (NW = 4: 1 wave per SIMD, each wave all 128 rows; NW = 8: 2 per SIMD, each
// wave 64 rows). NG = this wave's active 32-row groups (fixed per wave, so the loop has no row
// branch; every variant runs the same barriers). Raw bytes (weights in registers, activations in
// registers until stored to LDS) are loaded PD steps ahead through a ring of 4 register sets;
// step k+1's weights are decoded into the other fragment set after step k's MFMAs are issued;
// activations go through two LDS buffers with one barrier per step.
// Named ring slots reached through compile-time accessors: no array is ever indexed at run time,
// so every slot stays in registers.
template <class T>
struct Ring4 {
  T s0, s1, s2, s3;
  template <int N>
  __device__ __forceinline__ T& get() {
    if constexpr (N % 4 == 0) return s0;
    else if constexpr (N % 4 == 1) return s1;
    else if constexpr (N % 4 == 2) return s2;
    else return s3;
  }
};
struct FragSet {
  Frag g[4], u[4];
};
template <int WFMT, int NW>
struct Gemm2State {
  static constexpr int TPR = NW * 64 / kBM;
  Ring4<ARaw<TPR>> ar;                                // raw sets, prefetch distance <= 3
  Ring4<RowRaw<WFMT>> q0, q1;
  FragSet f[2];
  template <int N>
  __device__ __forceinline__ FragSet& frag() {
    if constexpr (N % 2 == 0) return f[0];
    else return f[1];
  }
};

// one K step; J = step index mod 4 (compile time, so every ring slot is static)
template <int WFMT, int NW, int NG, int PD, int J>
__device__ __forceinline__ void gemm2_step(Gemm2State<WFMT, NW>& st, int ks, int nk,
                                           const uint16_t* asrc, const uint8_t* w0,
                                           const uint8_t* w1, int g0, uint16_t (*As)[kBM * kAS],
                                           f32x16_t (&acc)[4][2]) {
  const int t = threadIdx.x, lane = t & 63, h = lane >> 5;
  const int kl = min(ks + PD, nk - 1) * kBK;          // loads past the end reload the last step
  st.ar.template get<J + PD>().load(asrc, kl, t);
  if (NG) {
    st.q0.template get<J + PD>().load(w0, kl, h);
    st.q1.template get<J + PD>().load(w1, kl, h);
  }
  FragSet& fc = st.template frag<J>();
#pragma unroll
  for (int s2 = 0; s2 < 4; ++s2) {
#pragma unroll
    for (int mg = 0; mg < NG; ++mg) {
      const uint4 a = a_frag(As[J & 1], g0 + mg, s2, lane);
      acc[mg][0] = mfma(a, fc.g[s2], acc[mg][0]);
      acc[mg][1] = mfma(a, fc.u[s2], acc[mg][1]);
    }
  }
  const int kn = min(ks + 1, nk - 1) * kBK;
  FragSet& fn = st.template frag<J + 1>();
  if (NG) {
    st.q0.template get<J + 1>().decode(kn, fn.g);
    st.q1.template get<J + 1>().decode(kn, fn.u);
  }
  st.ar.template get<J + 1>().store(As[(J + 1) & 1], t);
  __syncthreads();
}

template <int WFMT, int NW, int NG, int PD>
__device__ __forceinline__ void gemm2_loop(const uint16_t* asrc, const uint8_t* w0,
                                           const uint8_t* w1, int nk, int g0,
                                           uint16_t (*As)[kBM * kAS], f32x16_t (&acc)[4][2]) {
  const int t = threadIdx.x, lane = t & 63, h = lane >> 5;
  Gemm2State<WFMT, NW> st;
  st.ar.template get<0>().load(asrc, 0, t);
  if (NG) {
    st.q0.template get<0>().load(w0, 0, h);
    st.q1.template get<0>().load(w1, 0, h);
  }
  if (PD > 1) {
    const int k1 = min(1, nk - 1) * kBK;
    st.ar.template get<1>().load(asrc, k1, t);
    if (NG) {
      st.q0.template get<1>().load(w0, k1, h);
      st.q1.template get<1>().load(w1, k1, h);
    }
  }
  if (PD > 2) {
    const int k2 = min(2, nk - 1) * kBK;
    st.ar.template get<2>().load(asrc, k2, t);
    if (NG) {
      st.q0.template get<2>().load(w0, k2, h);
      st.q1.template get<2>().load(w1, k2, h);
    }
  }
  st.ar.template get<0>().store(As[0], t);
  if (NG) {
    st.q0.template get<0>().decode(0, st.f[0].g);
    st.q1.template get<0>().decode(0, st.f[0].u);
  }
  __syncthreads();
  for (int kq = 0; kq < nk; kq += 4) {
    gemm2_step<WFMT, NW, NG, PD, 0>(st, kq, nk, asrc, w0, w1, g0, As, acc);
    gemm2_step<WFMT, NW, NG, PD, 1>(st, kq + 1, nk, asrc, w0, w1, g0, As, acc);
    gemm2_step<WFMT, NW, NG, PD, 2>(st, kq + 2, nk, asrc, w0, w1, g0, As, acc);
    gemm2_step<WFMT, NW, NG, PD, 3>(st, kq + 3, nk, asrc, w0, w1, g0, As, acc);
  }
}

// ------------------------------------------------------------- super-block pipeline (PD = 0) --
// A weight row's raw bytes for a whole super-block (256 k = 4 steps) are fetched one super-block
// ahead into the other of two named register sets: four steps of MFMA time cover each load.
template <int WFMT>
struct RowSB;
template <>
struct RowSB<MOE_FMT_Q4_K> {
  uint4 hdr;
  uint4 q[4];                                         // per group: bytes [8h, +8) and [16+8h, +8)
  __device__ __forceinline__ void load(const uint8_t* row, int sb, int h) {
    const uint8_t* b = row + (size_t)sb * 144;
    hdr = *reinterpret_cast<const uint4*>(b);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const uint2 a = *reinterpret_cast<const uint2*>(b + 16 + 32 * g + 8 * h);
      const uint2 c = *reinterpret_cast<const uint2*>(b + 16 + 32 * g + 16 + 8 * h);
      q[g] = make_uint4(a.x, a.y, c.x, c.y);
    }
  }
  template <int G>
  __device__ __forceinline__ void decode(Frag* f) const {
    const Q4Scale lo = q4_scale(hdr, 2 * G), hi = q4_scale(hdr, 2 * G + 1);
    const uint2 p0 = make_uint2(q[G].x, q[G].y), p1 = make_uint2(q[G].z, q[G].w);
    f[0] = q4_frag<false>(p0, lo);
    f[1] = q4_frag<false>(p1, lo);
    f[2] = q4_frag<true>(p0, hi);
    f[3] = q4_frag<true>(p1, hi);
  }
  // the step's two sub-block scales, then fragment S alone (so decode can interleave with MFMAs)
  template <int G>
  __device__ __forceinline__ void scales(Q4Scale& lo, Q4Scale& hi) const {
    lo = q4_scale(hdr, 2 * G);
    hi = q4_scale(hdr, 2 * G + 1);
  }
  template <int G, int S>
  __device__ __forceinline__ Frag frag(const Q4Scale& lo, const Q4Scale& hi) const {
    const uint2 p = (S & 1) ? make_uint2(q[G].z, q[G].w) : make_uint2(q[G].x, q[G].y);
    return (S >> 1) ? q4_frag<true>(p, hi) : q4_frag<false>(p, lo);
  }
};
template <>
struct RowSB<MOE_FMT_BF16> {
  const uint8_t* row;                                 // bf16 rows stream from cache: no staging
  int sb, h;
  __device__ __forceinline__ void load(const uint8_t* r, int sb_, int h_) { row = r; sb = sb_; h = h_; }
  template <int G>
  __device__ __forceinline__ void decode(Frag* f) const {
    RowRaw<MOE_FMT_BF16> raw;
    raw.load(row, 256 * sb + 64 * G, h);
    raw.decode(0, f);
  }
};

template <int WFMT, int NW>
struct SBState {
  static constexpr int TPR = NW * 64 / kBM;
  ARaw<TPR> ar[2];
  RowSB<WFMT> r0a, r1a, r0b, r1b;                     // super-block sets a (even), b (odd)
  FragSet f0, f1;
};

// step g of a super-block (EVEN: the even super-block, raw set a; the next one's in set b). The
// next step's weight fragments are decoded one fragment at a time between this step's MFMA
// groups, so the decode VALU work issues while the MFMAs run.
// Loads retire in issue order, so the next step's activations are requested first and the next
// super-block's weights (step 0 only, sbn >= 0) after them: waiting for the activations then does
// not wait for the weight prefetch, which has the whole super-block to arrive.
template <int WFMT, int NW, int NG, int G, bool EVEN>
__device__ __forceinline__ void sb_step(SBState<WFMT, NW>& st, int ks, int nk, const uint16_t* asrc,
                                        int g0, uint16_t (*As)[kBM * kAS], f32x16_t (&acc)[4][2],
                                        const uint8_t* w0 = nullptr, const uint8_t* w1 = nullptr,
                                        int sbn = -1) {
  const int t = threadIdx.x, lane = t & 63;
  constexpr int J = G & 1;                            // step parity (As buffer, fragment set)
  constexpr int GN = (G + 1) & 3;                     // the next step's group
  const int kn = min(ks + 1, nk - 1) * kBK;
  st.ar[J ^ 1].load(asrc, kn, t);
  if (G == 0 && NG && sbn >= 0) {
    (EVEN ? st.r0b : st.r0a).load(w0, sbn, lane >> 5);
    (EVEN ? st.r1b : st.r1a).load(w1, sbn, lane >> 5);
  }
  FragSet& fc = J ? st.f1 : st.f0;
  FragSet& fn = J ? st.f0 : st.f1;
  const RowSB<WFMT>& n0 = (G < 3) == EVEN ? st.r0a : st.r0b;
  const RowSB<WFMT>& n1 = (G < 3) == EVEN ? st.r1a : st.r1b;
  if constexpr (WFMT == MOE_FMT_Q4_K) {
    Q4Scale l0, h0, l1, h1;
    if (NG) {
      n0.template scales<GN>(l0, h0);
      n1.template scales<GN>(l1, h1);
    }
    // activation fragments one sub-step ahead: the LDS reads of sub-step s2 + 1 are in flight
    // while sub-step s2's MFMAs run
    uint4 ac[4], an[4];
#pragma unroll
    for (int mg = 0; mg < NG; ++mg) ac[mg] = a_frag(As[J], g0 + mg, 0, lane);
#pragma unroll
    for (int s2 = 0; s2 < 4; ++s2) {
      if (s2 < 3) {
#pragma unroll
        for (int mg = 0; mg < NG; ++mg) an[mg] = a_frag(As[J], g0 + mg, s2 + 1, lane);
      }
#pragma unroll
      for (int mg = 0; mg < NG; ++mg) {
        acc[mg][0] = mfma(ac[mg], fc.g[s2], acc[mg][0]);
        acc[mg][1] = mfma(ac[mg], fc.u[s2], acc[mg][1]);
      }
#pragma unroll
      for (int mg = 0; mg < NG; ++mg) ac[mg] = an[mg];
      if (NG) {
        if (s2 == 0) { fn.g[0] = n0.template frag<GN, 0>(l0, h0); fn.u[0] = n1.template frag<GN, 0>(l1, h1); }
        if (s2 == 1) { fn.g[1] = n0.template frag<GN, 1>(l0, h0); fn.u[1] = n1.template frag<GN, 1>(l1, h1); }
        if (s2 == 2) { fn.g[2] = n0.template frag<GN, 2>(l0, h0); fn.u[2] = n1.template frag<GN, 2>(l1, h1); }
        if (s2 == 3) { fn.g[3] = n0.template frag<GN, 3>(l0, h0); fn.u[3] = n1.template frag<GN, 3>(l1, h1); }
      }
    }
  } else {
#pragma unroll
    for (int s2 = 0; s2 < 4; ++s2) {
#pragma unroll
      for (int mg = 0; mg < NG; ++mg) {
        const uint4 a = a_frag(As[J], g0 + mg, s2, lane);
        acc[mg][0] = mfma(a, fc.g[s2], acc[mg][0]);
        acc[mg][1] = mfma(a, fc.u[s2], acc[mg][1]);
      }
    }
    if (NG) {
      n0.template decode<GN>(fn.g);
      n1.template decode<GN>(fn.u);
    }
  }
  st.ar[J ^ 1].store(As[J ^ 1], t);
  __syncthreads();
}

template <int WFMT, int NW, int NG>
__device__ __forceinline__ void gemm2_loop_sb(const uint16_t* asrc, const uint8_t* w0,
                                              const uint8_t* w1, int nk, int g0,
                                              uint16_t (*As)[kBM * kAS], f32x16_t (&acc)[4][2]) {
  const int t = threadIdx.x, lane = t & 63, h = lane >> 5;
  const int nsb = nk / 4;
  SBState<WFMT, NW> st;
  st.ar[0].load(asrc, 0, t);
  if (NG) {
    st.r0a.load(w0, 0, h);
    st.r1a.load(w1, 0, h);
  }
  st.ar[0].store(As[0], t);
  if (NG) {
    st.r0a.template decode<0>(st.f0.g);
    st.r1a.template decode<0>(st.f0.u);
  }
  __syncthreads();
  for (int sp = 0; sp < nsb; sp += 2) {
    // even super-block sp (set a); its step 0 requests sp + 1 into set b
    sb_step<WFMT, NW, NG, 0, true>(st, 4 * sp + 0, nk, asrc, g0, As, acc, w0, w1, min(sp + 1, nsb - 1));
    sb_step<WFMT, NW, NG, 1, true>(st, 4 * sp + 1, nk, asrc, g0, As, acc);
    sb_step<WFMT, NW, NG, 2, true>(st, 4 * sp + 2, nk, asrc, g0, As, acc);
    sb_step<WFMT, NW, NG, 3, true>(st, 4 * sp + 3, nk, asrc, g0, As, acc);
    if (sp + 1 < nsb) {
      sb_step<WFMT, NW, NG, 0, false>(st, 4 * sp + 4, nk, asrc, g0, As, acc, w0, w1, min(sp + 2, nsb - 1));
      sb_step<WFMT, NW, NG, 1, false>(st, 4 * sp + 5, nk, asrc, g0, As, acc);
      sb_step<WFMT, NW, NG, 2, false>(st, 4 * sp + 6, nk, asrc, g0, As, acc);
      sb_step<WFMT, NW, NG, 3, false>(st, 4 * sp + 7, nk, asrc, g0, As, acc);
    }
  }
}

template <int WFMT, int NW, int PD>
__device__ __forceinline__ void gemm2_run(int ng, const uint16_t* asrc, const uint8_t* w0,
                                          const uint8_t* w1, int nk, int g0,
                                          uint16_t (*As)[kBM * kAS], f32x16_t (&acc)[4][2]) {
  if (PD == 0) {
    if (NW == 4) {
      if (ng >= 4) gemm2_loop_sb<WFMT, NW, 4>(asrc, w0, w1, nk, g0, As, acc);
      else if (ng == 3) gemm2_loop_sb<WFMT, NW, 3>(asrc, w0, w1, nk, g0, As, acc);
      else if (ng == 2) gemm2_loop_sb<WFMT, NW, 2>(asrc, w0, w1, nk, g0, As, acc);
      else gemm2_loop_sb<WFMT, NW, 1>(asrc, w0, w1, nk, g0, As, acc);
    } else {
      if (ng >= 2) gemm2_loop_sb<WFMT, NW, 2>(asrc, w0, w1, nk, g0, As, acc);
      else if (ng == 1) gemm2_loop_sb<WFMT, NW, 1>(asrc, w0, w1, nk, g0, As, acc);
      else gemm2_loop_sb<WFMT, NW, 0>(asrc, w0, w1, nk, g0, As, acc);
    }
  } else if (NW == 4) {
    if (ng >= 4) gemm2_loop<WFMT, NW, 4, PD>(asrc, w0, w1, nk, g0, As, acc);
    else if (ng == 3) gemm2_loop<WFMT, NW, 3, PD>(asrc, w0, w1, nk, g0, As, acc);
    else if (ng == 2) gemm2_loop<WFMT, NW, 2, PD>(asrc, w0, w1, nk, g0, As, acc);
    else gemm2_loop<WFMT, NW, 1, PD>(asrc, w0, w1, nk, g0, As, acc);
  } else {
    if (ng >= 2) gemm2_loop<WFMT, NW, 2, PD>(asrc, w0, w1, nk, g0, As, acc);
    else if (ng == 1) gemm2_loop<WFMT, NW, 1, PD>(asrc, w0, w1, nk, g0, As, acc);
    else gemm2_loop<WFMT, NW, 0, PD>(asrc, w0, w1, nk, g0, As, acc);
  }
}

#ifndef MOE_GEMM2_NW
#define MOE_GEMM2_NW 4
#endif
#ifndef MOE_GEMM2_PD
#define MOE_GEMM2_PD 0
#endif
constexpr int kNW = MOE_GEMM2_NW;       // waves per block
constexpr int kPD = MOE_GEMM2_PD;       // 0: super-block pipeline; 1..3: prefetch distance in steps
constexpr int kRPW = kBM * 4 / kNW;     // rows per wave

// ----------------------------------------------------------------------------------- gate/up --
template <int WFMT>
__global__ __launch_bounds__(kNW * 64) __attribute__((amdgpu_waves_per_eu(kNW / 4, kNW / 4))) void k_gemm2_gateup(
    const uint16_t* __restrict__ x16, const uint8_t* __restrict__ wg, const uint8_t* __restrict__ wu,
    size_t estride, const int32_t* __restrict__ tiles, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ sorted_pairs, int K, int H, int I, int T,
    uint16_t* __restrict__ S) {
  __shared__ __attribute__((aligned(16))) uint16_t As[2][kBM * kAS];
  int e, m0, mend, col;
  if (!tile_rows(tiles, offsets, T, I / 128, e, m0, mend, col)) return;
  const int t = threadIdx.x, lane = t & 63, h = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);   // wave-uniform (an SGPR)
  const int r0 = kRPW * (wave >> 2);
  const int n = col * 128 + 32 * (wave & 3) + (lane & 31);
  const size_t rowb = row_bytes2(WFMT, H);
  const uint8_t* grow = wg + (size_t)e * estride + (size_t)n * rowb;
  const uint8_t* urow = wu + (size_t)e * estride + (size_t)n * rowb;
  const int m = min(m0 + t / (kNW * 64 / kBM), mend - 1);
  const uint16_t* asrc = x16 + (size_t)(tiles ? sorted_pairs[m] / K : m) * H;
  f32x16_t acc[4][2];
#pragma unroll
  for (int mg = 0; mg < 4; ++mg) { acc[mg][0] = (f32x16_t){}; acc[mg][1] = (f32x16_t){}; }
  const int ng = __builtin_amdgcn_readfirstlane(min(max((mend - m0 - r0 + 31) >> 5, 0), kRPW / 32));
  gemm2_run<WFMT, kNW, kPD>(ng, asrc, grow, urow, H / kBK, r0 / 32, As, acc);
  // s = silu(gate) * up, C layout: reg r -> row 8(r/4) + 4(lane/32) + r%4, col lane%32
#pragma unroll
  for (int mg = 0; mg < kRPW / 32; ++mg) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int mm = m0 + r0 + 32 * mg + 8 * (r >> 2) + 4 * h + (r & 3);
      if (mm < mend) {
        float v = silu_f32(acc[mg][0][r]) * acc[mg][1][r];
        v = fminf(fmaxf(v, -65504.0f), 65504.0f);
        S[(size_t)mm * I + n] = __builtin_bit_cast(uint16_t, (_Float16)v);
      }
    }
  }
}

// -------------------------------------------------------------------------------------- down --
template <int WFMT>
__global__ __launch_bounds__(kNW * 64) __attribute__((amdgpu_waves_per_eu(kNW / 4, kNW / 4))) void k_gemm2_down(
    const uint16_t* __restrict__ S, const uint8_t* __restrict__ wd, size_t estride,
    const int32_t* __restrict__ tiles, const int32_t* __restrict__ offsets, int H, int I, int T,
    float* __restrict__ y) {
  __shared__ __attribute__((aligned(16))) uint16_t As[2][kBM * kAS];
  int e, m0, mend, col;
  if (!tile_rows(tiles, offsets, T, H / 256, e, m0, mend, col)) return;
  const int t = threadIdx.x, lane = t & 63, h = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);   // wave-uniform (an SGPR)
  const int r0 = kRPW * (wave >> 2);
  const int nb = col * 256 + 64 * (wave & 3) + (lane & 31);
  const size_t rowb = row_bytes2(WFMT, I);
  const uint8_t* w0 = wd + (size_t)e * estride + (size_t)nb * rowb;
  const uint8_t* w1 = w0 + 32 * rowb;
  const uint16_t* asrc = S + (size_t)min(m0 + t / (kNW * 64 / kBM), mend - 1) * I;
  f32x16_t acc[4][2];
#pragma unroll
  for (int mg = 0; mg < 4; ++mg) { acc[mg][0] = (f32x16_t){}; acc[mg][1] = (f32x16_t){}; }
  const int ng = __builtin_amdgcn_readfirstlane(min(max((mend - m0 - r0 + 31) >> 5, 0), kRPW / 32));
  gemm2_run<WFMT, kNW, kPD>(ng, asrc, w0, w1, I / kBK, r0 / 32, As, acc);
#pragma unroll
  for (int mg = 0; mg < kRPW / 32; ++mg) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int mm = m0 + r0 + 32 * mg + 8 * (r >> 2) + 4 * h + (r & 3);
      if (mm < mend) {
        y[(size_t)mm * H + nb] = acc[mg][0][r];
        y[(size_t)mm * H + nb + 32] = acc[mg][1][r];
      }
    }
  }
}

// ------------------------------------------------------------------------- f32 / bf16 -> f16 --
template <int XDT>
__global__ __launch_bounds__(256) void k_to_f16(const void* __restrict__ x, size_t n8,
                                                uint16_t* __restrict__ out) {
  for (size_t i = blockIdx.x * 256 + threadIdx.x; i < n8; i += (size_t)gridDim.x * 256) {
    // f16 RNE, saturated to +-65504 (an activation past f16's range would otherwise become inf)
    auto pk = [](float u, float v) {
      u = fminf(fmaxf(u, -65504.0f), 65504.0f);
      v = fminf(fmaxf(v, -65504.0f), 65504.0f);
      return __builtin_bit_cast(uint32_t, (f16x2_t){(_Float16)u, (_Float16)v});
    };
    uint4 o;
    if (XDT == MOE_DT_BF16) {
      const uint4 v = reinterpret_cast<const uint4*>(x)[i];
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
      uint32_t r[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) r[j] = pk(__uint_as_float(w[j] << 16), __uint_as_float(w[j] & 0xFFFF0000u));
      o = make_uint4(r[0], r[1], r[2], r[3]);
    } else {
      const float4 a = reinterpret_cast<const float4*>(x)[2 * i];
      const float4 b = reinterpret_cast<const float4*>(x)[2 * i + 1];
      o = make_uint4(pk(a.x, a.y), pk(a.z, a.w), pk(b.x, b.y), pk(b.z, b.w));
    }
    reinterpret_cast<uint4*>(out)[i] = o;
  }
}

}  // namespace moe

using namespace moe;

bool moe_gemm2_supports(int fmt) { return fmt == MOE_FMT_Q4_K || fmt == MOE_FMT_BF16; }

int moe_launch_to_f16(const void* x, int x_dtype, size_t n, uint16_t* out, hipStream_t st) {
  if (n % 8) return moe_set_error(MOE_E_UNSUPPORTED, "to_f16: n %% 8 != 0");
  const size_t n8 = n / 8;
  const int grid = (int)((n8 + 255) / 256 < 2048 ? (n8 + 255) / 256 : 2048);
  if (x_dtype == MOE_DT_BF16)
    hipLaunchKernelGGL(k_to_f16<MOE_DT_BF16>, dim3(grid), dim3(256), 0, st, x, n8, out);
  else
    hipLaunchKernelGGL(k_to_f16<MOE_DT_F32>, dim3(grid), dim3(256), 0, st, x, n8, out);
  return moe_check_launch("to_f16");
}

int moe_launch_gemm2_gateup(const uint16_t* x16, const void* w_gate, const void* w_up, int fmt,
                            size_t expert_stride, const int32_t* tiles, int max_tiles, int T,
                            const int32_t* offsets, const int32_t* sorted_pairs, int K, int H,
                            int I, uint16_t* S, hipStream_t st) {
  if (H % 256 || I % 128)
    return moe_set_error(MOE_E_UNSUPPORTED, "gemm2 gate_up needs H %% 256 == 0, I %% 128 == 0");
  const uint8_t* g = reinterpret_cast<const uint8_t*>(w_gate);
  const uint8_t* u = reinterpret_cast<const uint8_t*>(w_up);
  const int ntile = tiles ? max_tiles : (T + kBM - 1) / kBM;
  const dim3 grid(kXcd * ((ntile + kXcd - 1) / kXcd) * (I / 128));
  if (fmt == MOE_FMT_Q4_K)
    hipLaunchKernelGGL(k_gemm2_gateup<MOE_FMT_Q4_K>, grid, dim3(kNW * 64), 0, st, x16, g, u, expert_stride, tiles, offsets, sorted_pairs, K, H, I, T, S);
  else if (fmt == MOE_FMT_BF16)
    hipLaunchKernelGGL(k_gemm2_gateup<MOE_FMT_BF16>, grid, dim3(kNW * 64), 0, st, x16, g, u, expert_stride, tiles, offsets, sorted_pairs, K, H, I, T, S);
  else
    return moe_set_error(MOE_E_FORMAT, "gemm2 gate_up: unsupported format %d", fmt);
  return moe_check_launch("gemm2_gateup");
}

int moe_launch_gemm2_down(const uint16_t* S, const void* w_down, int fmt, size_t expert_stride,
                          const int32_t* tiles, int max_tiles, int T, const int32_t* offsets,
                          int H, int I, float* y, hipStream_t st) {
  if (H % 256 || I % 256)
    return moe_set_error(MOE_E_UNSUPPORTED, "gemm2 down needs H %% 256 == 0, I %% 256 == 0");
  const uint8_t* w = reinterpret_cast<const uint8_t*>(w_down);
  const int ntile = tiles ? max_tiles : (T + kBM - 1) / kBM;
  const dim3 grid(kXcd * ((ntile + kXcd - 1) / kXcd) * (H / 256));
  if (fmt == MOE_FMT_Q4_K)
    hipLaunchKernelGGL(k_gemm2_down<MOE_FMT_Q4_K>, grid, dim3(kNW * 64), 0, st, S, w, expert_stride, tiles, offsets, H, I, T, y);
  else if (fmt == MOE_FMT_BF16)
    hipLaunchKernelGGL(k_gemm2_down<MOE_FMT_BF16>, grid, dim3(kNW * 64), 0, st, S, w, expert_stride, tiles, offsets, H, I, T, y);
  else
    return moe_set_error(MOE_E_FORMAT, "gemm2 down: unsupported format %d", fmt);
  return moe_check_launch("gemm2_down");
}
