// Prefill-path grouped GEMM for Q4_K experts with the weight decode in the MFMA waves
// (gfx950, v_mfma_f32_32x32x16_f16, f32 accumulation).
//
// Work item: one tile of up to 160 sorted (token, slot) rows of one expert (k_build_tiles,
// 160-row tiles, largest first) times one 256-row weight slab (gate_up: 128 gate + the matching
// 128 up rows; down: 256 rows). The grid is persistent: two blocks per CU, block b serving XCD
// b % 8 and taking that XCD's items (tiles x, x + 8, ... times the slabs) with stride
// gridDim.x / 8, so the slabs of one tile run side by side on one XCD and share its rows in L2.
//
// Block = 4 waves (one per SIMD) and 80 KB of LDS, so each SIMD runs two independent waves: one
// block's MFMAs cover the other's waits. Operands reach LDS by direct global->LDS loads
// (global_load_lds_dwordx4, no registers): every wave issues its share of the next K step's
// activation chunks, of the raw nibble bytes three steps ahead and of the next super-block's
// 16-byte headers, and waits for its own loads with explicit vmcnt counts before the step's
// barrier. The K steps of consecutive items form one stream: the last super-block of an item
// issues the next item's first loads, so an item's epilogue runs while the next one's operands
// arrive. LDS rings:
//   A[2]:  f16 activations of one 64-wide K step, 160 rows x 128 B, 16-byte chunk c of row m at
//          chunk c ^ swz(m) (swz(m) = (m ^ m >> 1) & 7, so the fragment reads of 8 or 16 lanes
//          hit distinct banks under either a 32- or a 64-bank layout);
//   Q[4]:  the 32 nibble bytes of one K step for 256 weight rows, half h of row n at h ^ bit;
//   Hd[2]: the 16-byte header (d, dmin, 12 scale bytes) of one super-block for 256 rows.
// Each wave owns all 160 rows x (32 gate + 32 up) columns (gate_up) or 64 columns (down), reads
// its rows' raw bytes and headers from LDS, decodes them in registers straight into MFMA B
// fragments (q * f16(d sc) + f16(-dmin m) on the f16 mantissa trick) and runs the MFMAs.
// k order inside a K step: lane half h takes nibble bytes 16h..16h+15 of the step, so substep
// ss covers k = 32 (ss >> 1) + 16 h + 8 (ss & 1) + 0..7 and the activation fragments follow.
// Results leave through raw buffer stores whose descriptor ends at the tile's last row, so rows
// past it are dropped by the hardware (the whole offset is in the VGPR operand: the range check
// does not cover the SGPR offset) and every wave issues the same number of stores.
#include "common.h"
#include "moe_internal.h"
#include "lds_dma.h"
#include "q4k_mfma.h"

namespace moe {

namespace g4 {

using dma::lds_addr;
using dma::opaque;
using dma::tid_fresh;
using dma::wait_vm;

constexpr int kBM = MOE_GEMM3_BM;       // 160 activation rows per tile
constexpr int kMG = kBM / 32;           // MFMA row groups
constexpr int kBN = 256;                // weight rows per item
constexpr int kSBB = 144;               // bytes per Q4_K super-block row (256 K)
constexpr int kQR = 4;                  // raw nibble ring depth (K steps)
constexpr int kXcd = 8;
constexpr int kWaves = 4;
constexpr int kBlocksPerCu = 2;
constexpr int kAI = kBM * 8 / 64 / kWaves;   // A loads per wave per K step (5)
constexpr int kQI = kBN * 2 / 64 / kWaves;   // nibble loads per wave per K step (2)
static_assert(kAI == 5 && kQI == 2 && kBN / 64 == kWaves, "load split assumes 160 x 256 items");

struct Smem {
  uint8_t A[2][kBM * 128];
  uint8_t Q[kQR][kBN * 32];
  uint8_t Hd[2][kBN * 16];
};
static_assert(sizeof(Smem) * kBlocksPerCu <= 160 * 1024, "two blocks per CU");

using q4m::a_swz;
using q4m::q_swz;
using q4m::mfma;
using q4m::q4_frag;
using q4m::q4_scales;

// ------------------------------------------------------------------------------- items --
struct Item {
  int e, m0, mend, col;
};

// Item q of this block's XCD: tile x + 8 (q / ncol), slab q % ncol. False past the list.
__device__ __forceinline__ bool get_item(const int32_t* __restrict__ tiles,
                                         const int32_t* __restrict__ offsets, int q, int ncol,
                                         Item& it) {
  const int x = blockIdx.x % kXcd;
  const int count = tiles[0];
  const int ntx = count > x ? (count - x + kXcd - 1) / kXcd : 0;
  if (q >= ntx * ncol) return false;
  const int t = x + kXcd * (q / ncol);
  it.col = q % ncol;
  it.e = tiles[1 + 2 * t];
  it.m0 = tiles[2 + 2 * t];
  it.mend = min(it.m0 + kBM, offsets[it.e + 1]);
  return true;
}

// Load geometry. Wave w, lane l: its j-th load of a ring slot covers the slot's 16-byte units
// 64 (w + 4 j) + l.
//   A unit u: tile row u >> 3, chunk (u & 7) ^ a_swz(row) of that row's 64 K of the step.
//   Q unit u: weight row u >> 1, logical half (u & 1) ^ q_swz(row) of the step's 32 nibble bytes.
//   Hd unit u: weight row u (one load per wave).
struct Lane {
  uint32_t qoff[kQI];                   // byte offset of Q load j from its base (sb 0, step 0)
  uint32_t hoff;                        // byte offset of the Hd load from its base
  uint32_t la, lq, lh;                  // LDS address of this wave's first unit in slot 0
};
// A load j of wave w, lane l: tile row and the chunk's byte offset within the row (t = thread)
__device__ __forceinline__ int a_row(int t, int j) { return (t + 256 * j) >> 3; }
__device__ __forceinline__ uint32_t a_chunk(int t, int j) {
  const int u = t + 256 * j;
  return 16u * (uint32_t)((u & 7) ^ a_swz(u >> 3));
}

// per-item addresses: uniform bases, per-lane A row offsets
struct Addr {
  const uint8_t* qb[kQI];               // Q load j's base; the Hd load of waves 0, 1 uses qb[0],
  const uint8_t* ab;                    // of waves 2, 3 qb[kQI - 1]
  uint32_t aoff[kAI];
};

__device__ __forceinline__ void ld_a(const Lane& ln, const Addr& ad, int slot, int ks) {
  const uint8_t* b = ad.ab + (size_t)ks * 128;
#pragma unroll
  for (int j = 0; j < kAI; ++j) dma::load16(ad.aoff[j], b, ln.la + slot * (kBM * 128) + j * 4096);
}
__device__ __forceinline__ void ld_q(const Lane& ln, const Addr& ad, int slot, int ks) {
  const int off = (ks >> 2) * kSBB + 32 * (ks & 3);
#pragma unroll
  for (int j = 0; j < kQI; ++j) dma::load16(ln.qoff[j], ad.qb[j] + off, ln.lq + slot * (kBN * 32) + j * 4096);
}
__device__ __forceinline__ void ld_h(const Lane& ln, const Addr& ad, int slot, int sb) {
  const uint8_t* hb = __builtin_amdgcn_readfirstlane(threadIdx.x >> 7) ? ad.qb[kQI - 1] : ad.qb[0];
  dma::load16(ln.hoff, hb + sb * kSBB, ln.lh + slot * (kBN * 16));
}

__device__ __forceinline__ void lane_common(Lane& ln, Smem& sm, int wave, int lane) {
  (void)lane;
  ln.la = lds_addr(sm.A[0]) + 1024 * wave;
  ln.lq = lds_addr(sm.Q[0]) + 1024 * wave;
  ln.lh = lds_addr(sm.Hd[0]) + 1024 * wave;
}

// keeps values computed before this point (and the waits for their loads) ahead of what follows
__device__ __forceinline__ void pin(const uint32_t (&v)[kAI]) {
  asm volatile("" ::"v"(v[0]), "v"(v[1]), "v"(v[2]), "v"(v[3]), "v"(v[4]));
}

// ------------------------------------------------------------------------------- modes --
struct GateUp {
  const uint16_t* x16;
  const uint8_t *wg, *wu;
  size_t estride, rowb;
  const int32_t* sorted_pairs;
  int K, H, I;
  uint16_t* S;
  static constexpr int kStores = kMG * 16;          // per wave per item
  __device__ int nk() const { return H / 64; }
  __device__ int ncol() const { return I / 128; }
  __device__ int n0(int wave) const { return 32 * wave; }
  __device__ int n1(int wave) const { return 128 + 32 * wave; }
  __device__ void lane_init(Lane& ln, int wave, int lane) const {
    // Q load 0 covers gate rows 32 w + l / 2, load 1 the up rows 128 + 32 w + l / 2
#pragma unroll
    for (int j = 0; j < kQI; ++j) {
      const int u = 64 * (wave + kWaves * j) + lane, n = u >> 1;
      ln.qoff[j] = (uint32_t)((n & 127) * rowb) + 16u + 16u * (uint32_t)((u & 1) ^ q_swz(n));
    }
    ln.hoff = (uint32_t)(((64 * wave + lane) & 127) * rowb);
  }
  __device__ void bases(Addr& ad, const Item& it, int wave) const {
    const uint8_t* g = wg + (size_t)it.e * estride + (size_t)it.col * 128 * rowb;
    const uint8_t* u = wu + (size_t)it.e * estride + (size_t)it.col * 128 * rowb;
    ad.qb[0] = g;
    ad.qb[1] = u;
    ad.ab = reinterpret_cast<const uint8_t*>(x16);
  }
  // stage 1: the rows' token ids (raw, held in aoff); stage 2: byte offsets
  __device__ void rows1(Addr& ad, const Item& it, const Lane&) const {
    const int t = tid_fresh();
#pragma unroll
    for (int j = 0; j < kAI; ++j) ad.aoff[j] = (uint32_t)sorted_pairs[min(it.m0 + a_row(t, j), it.mend - 1)];
  }
  __device__ void rows2(Addr& ad, const Lane&) const {
    const int t = tid_fresh();
#pragma unroll
    for (int j = 0; j < kAI; ++j) ad.aoff[j] = (ad.aoff[j] / (uint32_t)K) * (uint32_t)H * 2u + a_chunk(t, j);
  }
  __device__ void epilogue(const Item& it, int wave, int lane, const f32x16_t (&acc)[kMG][2]) const {
    const __amdgpu_buffer_rsrc_t rs = dma::rsrc(S + (size_t)it.m0 * I, (it.mend - it.m0) * I * 2);
    // row 32 mg + 8 (r >> 2) + 4 h + (r & 3), column n: lane part + uniform row part
    const int rs2 = opaque(I * 2);
    const int lane_off = (4 * (lane >> 5) * I + it.col * 128 + 32 * wave + (lane & 31)) * 2;
#pragma unroll
    for (int mg = 0; mg < kMG; ++mg) {
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        const int vo = lane_off + (32 * mg + 8 * rq) * rs2;
#pragma unroll
        for (int r3 = 0; r3 < 4; ++r3) {
          const int r = 4 * rq + r3;
          const float g = acc[mg][0][r];
          float v = g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * acc[mg][1][r];
          v = fminf(fmaxf(v, -65504.0f), 65504.0f);
          __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, (_Float16)v), rs,
                                                vo + r3 * rs2, 0, 0);
        }
      }
    }
  }
};

// Y16: the rows leave as f16 (saturated to +-65504, the combine's operand in the block forward)
// instead of f32.
template <bool Y16>
struct Down {
  const uint16_t* S;
  const uint8_t* wd;
  size_t estride, rowb;
  int H, I;
  void* y;
  static constexpr int kStores = kMG * 32;          // per wave per item (b32 or b16 stores alike)
  __device__ int nk() const { return I / 64; }
  __device__ int ncol() const { return H / kBN; }
  __device__ int n0(int wave) const { return 64 * wave; }
  __device__ int n1(int wave) const { return 64 * wave + 32; }
  __device__ void lane_init(Lane& ln, int wave, int lane) const {
#pragma unroll
    for (int j = 0; j < kQI; ++j) {
      const int u = 64 * (wave + kWaves * j) + lane, n = u >> 1;
      ln.qoff[j] = (uint32_t)(n * rowb) + 16u + 16u * (uint32_t)((u & 1) ^ q_swz(n));
    }
    ln.hoff = (uint32_t)((64 * wave + lane) * rowb);
  }
  __device__ void bases(Addr& ad, const Item& it, int) const {
    const uint8_t* w = wd + (size_t)it.e * estride + (size_t)it.col * kBN * rowb;
    ad.qb[0] = w;
    ad.qb[1] = w;
    ad.ab = reinterpret_cast<const uint8_t*>(S + (size_t)it.m0 * I);
  }
  __device__ void rows1(Addr&, const Item&, const Lane&) const {}
  __device__ void rows2_item(Addr& ad, const Item& it, const Lane&) const {
    const int last = it.mend - it.m0 - 1;
    const int t = tid_fresh();
#pragma unroll
    for (int j = 0; j < kAI; ++j) ad.aoff[j] = (uint32_t)min(a_row(t, j), last) * (uint32_t)I * 2u + a_chunk(t, j);
  }
  __device__ void epilogue(const Item& it, int wave, int lane, const f32x16_t (&acc)[kMG][2]) const {
    constexpr int kB = Y16 ? 2 : 4;                   // bytes per element
    char* yb = reinterpret_cast<char*>(y) + (size_t)it.m0 * H * kB;
    const __amdgpu_buffer_rsrc_t rs = dma::rsrc(yb, (it.mend - it.m0) * H * kB);
    const int rsb = opaque(H * kB);
    const int lane_off = (4 * (lane >> 5) * H + it.col * kBN + 64 * wave + (lane & 31)) * kB;
#pragma unroll
    for (int mg = 0; mg < kMG; ++mg) {
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        const int vo = lane_off + (32 * mg + 8 * rq) * rsb;
#pragma unroll
        for (int r3 = 0; r3 < 4; ++r3) {
          const int r = 4 * rq + r3;
          // the builtins' data operand is an integer: pass the bits, not the value (copied out of
          // the vector first: a bit cast of the vector element itself read element 0 here)
          float v0 = acc[mg][0][r], v1 = acc[mg][1][r];
          if constexpr (Y16) {
            v0 = fminf(fmaxf(v0, -65504.0f), 65504.0f);
            v1 = fminf(fmaxf(v1, -65504.0f), 65504.0f);
            __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, (_Float16)v0), rs,
                                                  vo + r3 * rsb, 0, 0);
            __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, (_Float16)v1), rs,
                                                  vo + r3 * rsb + 64, 0, 0);
          } else {
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v0), rs, vo + r3 * rsb, 0, 0);
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v1), rs, vo + r3 * rsb + 128, 0, 0);
          }
        }
      }
    }
  }
};

__device__ __forceinline__ void rows_all(const GateUp& md, Addr& ad, const Item& it, const Lane& ln) {
  md.rows1(ad, it, ln);
  md.rows2(ad, ln);
}
template <bool Y16>
__device__ __forceinline__ void rows_all(const Down<Y16>& md, Addr& ad, const Item& it, const Lane& ln) {
  md.rows2_item(ad, it, ln);
}
// next item's A row offsets in two stages (loads issued in step 1, consumed in step 2)
__device__ __forceinline__ void rows_stage1(const GateUp& md, Addr& ad, const Item& it, const Lane& ln) {
  md.rows1(ad, it, ln);
}
__device__ __forceinline__ void rows_stage2(const GateUp& md, Addr& ad, const Item&, const Lane& ln) {
  md.rows2(ad, ln);
}
template <bool Y16>
__device__ __forceinline__ void rows_stage1(const Down<Y16>&, Addr&, const Item&, const Lane&) {}
template <bool Y16>
__device__ __forceinline__ void rows_stage2(const Down<Y16>& md, Addr& ad, const Item& it, const Lane& ln) {
  md.rows2_item(ad, it, ln);
}

// ------------------------------------------------------------------------------- one item --
// Step ks (super-block sb = ks / 4, s = ks % 4) of the item reads A[ks & 1], Q[ks % 4] and
// Hd[(hp + sb) & 1]. After the step's barrier the wave issues A of step ks + 1, Q of step ks + 3
// and (s == 0) Hd of super-block sb + 1, each into the slot step ks - 1 (super-block sb - 1)
// used; in the last super-block those are the next item's steps 0..2 and super-block 0 (or, with
// no next item, clamped repeats of this item's last ones, into slots nothing reads again), so
// every step issues the same loads and the vmcnt counts are constants.
// Lane l: weight rows n0 + l % 32 (group 0) and n1 + l % 32 (group 1); half h = l / 32.
template <int NG, class M>
__device__ __forceinline__ void run_item(const M& md, const Lane& ln, const Addr& ca, Addr& na,
                                         const Item& nx, bool has_next, bool first, int hp, int n0,
                                         int n1, Smem& sm, f32x16_t (&acc)[kMG][2]) {
  const int lane = threadIdx.x & 63;
  const int h = lane >> 5, r = lane & 31;
  const int nk = md.nk(), nsb = nk / 4;
  int aoff[4];
#pragma unroll
  for (int ss = 0; ss < 4; ++ss)
    aoff[ss] = 16 * (8 * r + ((4 * (ss >> 1) + 2 * h + (ss & 1)) ^ a_swz(r)));
  const int qo0 = 16 * (2 * (n0 + r) + (h ^ q_swz(r)));
  const int qo1 = 16 * (2 * (n1 + r) + (h ^ q_swz(r)));
  auto step = [&](int sb, int s, bool first_sb, bool last) {
    const int ks = 4 * sb + s;
    // wait for this wave's loads of step ks (A was issued last in step ks - 1, then its Q and,
    // after s == 0, Hd; before an item's first step: the previous item's epilogue stores)
    if (first_sb && s == 0) {
      if (!first) wait_vm<(kQI + M::kStores < 63 ? kQI + M::kStores : 63)>();
    } else if (s == 1) {
      wait_vm<kQI + 1>();
    } else {
      wait_vm<kQI>();
    }
    __syncthreads();
    // the next item's row offsets: loads issued in step 1 (after its loads), consumed here, ahead
    // of this step's loads (with no next item they describe the current one and go unused)
    if (first_sb && s == 2) {
      rows_stage2(md, na, nx, ln);
      pin(na.aoff);
    }
    if (!last) {
      ld_a(ln, ca, (s + 1) & 1, ks + 1);
      ld_q(ln, ca, (s + 3) & 3, min(ks + 3, nk - 1));
      if (s == 0) ld_h(ln, ca, (hp + sb + 1) & 1, sb + 1);
    } else if (has_next) {
      if (s == 3) ld_a(ln, na, 0, 0); else ld_a(ln, ca, (s + 1) & 1, ks + 1);
      if (s == 0) ld_q(ln, ca, 3, nk - 1); else ld_q(ln, na, s - 1, s - 1);
      if (s == 0) ld_h(ln, na, (hp + nsb) & 1, 0);
    } else {
      ld_a(ln, ca, (s + 1) & 1, min(ks + 1, nk - 1));
      ld_q(ln, ca, (s + 3) & 3, nk - 1);
      if (s == 0) ld_h(ln, ca, (hp + nsb) & 1, nsb - 1);
    }
    if (first_sb && s == 1) rows_stage1(md, na, nx, ln);
    const uint8_t* As = sm.A[s & 1];
    const uint8_t* Qs = sm.Q[s];
    // the super-block's headers stay in their slot for its four steps: read them every step
    const uint8_t* Hs = sm.Hd[(hp + sb) & 1];
    const uint4 hdr0 = *reinterpret_cast<const uint4*>(Hs + 16 * (n0 + r));
    const uint4 hdr1 = *reinterpret_cast<const uint4*>(Hs + 16 * (n1 + r));
    const uint4 q0 = *reinterpret_cast<const uint4*>(Qs + qo0);
    const uint4 q1 = *reinterpret_cast<const uint4*>(Qs + qo1);
    f16x2_t ds0l, nd0l, ds0h, nd0h, ds1l, nd1l, ds1h, nd1h;
    q4_scales(hdr0, 2 * s, ds0l, nd0l);
    q4_scales(hdr0, 2 * s + 1, ds0h, nd0h);
    q4_scales(hdr1, 2 * s, ds1l, nd1l);
    q4_scales(hdr1, 2 * s + 1, ds1h, nd1h);
    auto decode = [&](int ss, uint4& bg, uint4& bu) {
      if (ss == 0) { bg = q4_frag<false>(q0.x, q0.y, ds0l, nd0l); bu = q4_frag<false>(q1.x, q1.y, ds1l, nd1l); }
      else if (ss == 1) { bg = q4_frag<false>(q0.z, q0.w, ds0l, nd0l); bu = q4_frag<false>(q1.z, q1.w, ds1l, nd1l); }
      else if (ss == 2) { bg = q4_frag<true>(q0.x, q0.y, ds0h, nd0h); bu = q4_frag<true>(q1.x, q1.y, ds1h, nd1h); }
      else { bg = q4_frag<true>(q0.z, q0.w, ds0h, nd0h); bu = q4_frag<true>(q1.z, q1.w, ds1h, nd1h); }
    };
    auto afrag = [&](int ss, uint4 (&a)[NG]) {
#pragma unroll
      for (int mg = 0; mg < NG; ++mg) a[mg] = *reinterpret_cast<const uint4*>(As + aoff[ss] + 4096 * mg);
    };
    // one set of A and B fragments: substep ss + 1's are read and decoded into the same
    // registers once substep ss's MFMAs have issued (an MFMA holds its operands from issue)
    uint4 ac[NG], bg, bu;
    afrag(0, ac);
    decode(0, bg, bu);
#pragma unroll
    for (int ss = 0; ss < 4; ++ss) {
#pragma unroll
      for (int mg = 0; mg < NG; ++mg) {
        acc[mg][0] = mfma(ac[mg], bg, acc[mg][0]);
        acc[mg][1] = mfma(ac[mg], bu, acc[mg][1]);
      }
      if (ss < 3) {
        afrag(ss + 1, ac);
        decode(ss + 1, bg, bu);
      }
    }
  };

#pragma unroll
  for (int s = 0; s < 4; ++s) step(0, s, true, false);
  for (int sb = 1; sb < nsb - 1; ++sb) {
#pragma unroll
    for (int s = 0; s < 4; ++s) step(sb, s, false, false);
  }
#pragma unroll
  for (int s = 0; s < 4; ++s) step(nsb - 1, s, false, true);
}

template <class M>
__device__ __forceinline__ void run_n(int ng, const M& md, const Lane& ln, const Addr& ca, Addr& na,
                                      const Item& nx, bool has_next, bool first, int hp, int n0,
                                      int n1, Smem& sm, f32x16_t (&acc)[kMG][2]) {
  if (ng >= 5) run_item<5>(md, ln, ca, na, nx, has_next, first, hp, n0, n1, sm, acc);
  else if (ng == 4) run_item<4>(md, ln, ca, na, nx, has_next, first, hp, n0, n1, sm, acc);
  else if (ng == 3) run_item<3>(md, ln, ca, na, nx, has_next, first, hp, n0, n1, sm, acc);
  else if (ng == 2) run_item<2>(md, ln, ca, na, nx, has_next, first, hp, n0, n1, sm, acc);
  else run_item<1>(md, ln, ca, na, nx, has_next, first, hp, n0, n1, sm, acc);
}

// The block's items in order; the first one's operands are loaded up front, every later one's
// by the previous item's last super-block.
template <class M>
__device__ __forceinline__ void persistent(const M& md, const int32_t* __restrict__ tiles,
                                           const int32_t* __restrict__ offsets, Smem& sm) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int stride = gridDim.x / kXcd;
  const int ncol = md.ncol(), nsb = md.nk() / 4;
  int q = blockIdx.x / kXcd;
  Item cur;
  if (!get_item(tiles, offsets, q, ncol, cur)) return;
  Lane ln;
  lane_common(ln, sm, wave, lane);
  md.lane_init(ln, wave, lane);
  Addr ca;
  md.bases(ca, cur, wave);
  rows_all(md, ca, cur, ln);
  // step 0's operands first; steps 1 and 2's nibbles may still be in flight at step 0
  ld_h(ln, ca, 0, 0);
  ld_q(ln, ca, 0, 0);
  ld_a(ln, ca, 0, 0);
#pragma unroll
  for (int j = 1; j < kQR - 1; ++j) ld_q(ln, ca, j, j);
  wait_vm<(kQR - 2) * kQI>();
  int hp = 0;
  bool first = true;
  for (;;) {
    Item nx;
    const bool has_next = get_item(tiles, offsets, q + stride, ncol, nx);
    if (!has_next) nx = cur;
    Addr na;
    md.bases(na, nx, wave);
    f32x16_t acc[kMG][2];
#pragma unroll
    for (int mg = 0; mg < kMG; ++mg) { acc[mg][0] = (f32x16_t){}; acc[mg][1] = (f32x16_t){}; }
    const int ng = __builtin_amdgcn_readfirstlane((cur.mend - cur.m0 + 31) >> 5);
    run_n(ng, md, ln, ca, na, nx, has_next, first, hp, md.n0(wave), md.n1(wave), sm, acc);
    md.epilogue(cur, wave, lane, acc);
    if (!has_next) break;
    cur = nx;
    ca = na;
    hp = (hp + nsb) & 1;
    q += stride;
    first = false;
  }
  // no load may still be writing this block's LDS when its waves exit
  wait_vm<0>();
}

}  // namespace g4

// ----------------------------------------------------------------------------------- kernels --
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_gemm4_gateup(
    const uint16_t* __restrict__ x16, const uint8_t* __restrict__ wg, const uint8_t* __restrict__ wu,
    size_t estride, const int32_t* __restrict__ tiles, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ sorted_pairs, int K, int H, int I, uint16_t* __restrict__ S) {
  using namespace g4;
  __shared__ __attribute__((aligned(16))) Smem sm;
  const GateUp md{x16, wg, wu, estride, (size_t)(H / 256) * kSBB, sorted_pairs, K, H, I, S};
  persistent(md, tiles, offsets, sm);
}

template <bool Y16>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_gemm4_down(
    const uint16_t* __restrict__ S, const uint8_t* __restrict__ wd, size_t estride,
    const int32_t* __restrict__ tiles, const int32_t* __restrict__ offsets, int H, int I,
    void* __restrict__ y) {
  using namespace g4;
  __shared__ __attribute__((aligned(16))) Smem sm;
  const Down<Y16> md{S, wd, estride, (size_t)(I / 256) * kSBB, H, I, y};
  persistent(md, tiles, offsets, sm);
}

}  // namespace moe

using namespace moe;

static int persistent_grid(int max_tiles, int ncol) {
  static int n_cu = 0;
  if (!n_cu) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
      n_cu = n;
    else
      n_cu = 256;
  }
  const int per_xcd_items = (max_tiles + g4::kXcd - 1) / g4::kXcd * ncol;
  const int per_xcd_slots = (n_cu * g4::kBlocksPerCu + g4::kXcd - 1) / g4::kXcd;
  return g4::kXcd * (per_xcd_items < per_xcd_slots ? per_xcd_items : per_xcd_slots);
}

int moe_launch_gemm4_gateup(const uint16_t* x16, const void* w_gate, const void* w_up,
                            size_t expert_stride, const int32_t* tiles, int max_tiles,
                            const int32_t* offsets, const int32_t* sorted_pairs, int K, int H,
                            int I, uint16_t* S, hipStream_t st) {
  if (H % 256 || H < 512 || I % 128)
    return moe_set_error(MOE_E_UNSUPPORTED, "gemm4 gate_up needs H %% 256 == 0, H >= 512, I %% 128 == 0");
  const dim3 grid(persistent_grid(max_tiles, I / 128));
  hipLaunchKernelGGL(k_gemm4_gateup, grid, dim3(256), 0, st, x16, reinterpret_cast<const uint8_t*>(w_gate),
                     reinterpret_cast<const uint8_t*>(w_up), expert_stride, tiles, offsets, sorted_pairs,
                     K, H, I, S);
  return moe_check_launch("gemm4_gateup");
}

int moe_launch_gemm4_down(const uint16_t* S, const void* w_down, size_t expert_stride,
                          const int32_t* tiles, int max_tiles, const int32_t* offsets, int H, int I,
                          void* y, int y16, hipStream_t st) {
  if (H % g4::kBN || I % 256 || I < 512)
    return moe_set_error(MOE_E_UNSUPPORTED, "gemm4 down needs H %% 256 == 0, I %% 256 == 0, I >= 512");
  const dim3 grid(persistent_grid(max_tiles, H / g4::kBN));
  if (y16)
    hipLaunchKernelGGL(k_gemm4_down<true>, grid, dim3(256), 0, st, S, reinterpret_cast<const uint8_t*>(w_down),
                       expert_stride, tiles, offsets, H, I, y);
  else
    hipLaunchKernelGGL(k_gemm4_down<false>, grid, dim3(256), 0, st, S, reinterpret_cast<const uint8_t*>(w_down),
                       expert_stride, tiles, offsets, H, I, y);
  return moe_check_launch("gemm4_down");
}
