// Prefill-path grouped GEMM for few rows per expert (small batches): Q4_K gate_up and down with
// the weight decode in the MFMA waves (gfx950, v_mfma_f32_32x32x16_f16, f32 accumulation).
//
// When T * K / E is small an expert has a few dozen (token, slot) rows. The 160-row persistent
// kernels (gemm4.hip) then run one short item per block and wait, at every K step, for that
// step's activation rows, which they request one step ahead: the step time is an L2 round trip.
// Here a work item is one tile of up to 32 sorted rows of one expert (k_build_tiles with 32-row
// tiles) times one 256-row weight slab (gate_up: 128 gate + the matching 128 up rows; down: 256
// rows), one block per item, and the activation rows go through the same 4-deep ring as the
// nibble bytes: each step requests step ks + 3's activations and nibbles (and, at a super-block's
// first step, the next super-block's headers), so three steps of loads stay in flight.
// Block = 4 waves (one per SIMD), 56 KB of LDS:
//   A[4]:  f16 activations of one 64-wide K step, 32 rows x 128 B, chunk c of row m at c ^ swz(m);
//   Q[4]:  the 32 nibble bytes of one K step for 256 weight rows, half h of row n at h ^ bit;
//   Hd[2]: the 16-byte header (d, dmin, 12 scale bytes) of one super-block for 256 rows.
// Operands reach LDS by direct global->LDS loads (global_load_lds_dwordx4); every wave waits for
// its own loads with an explicit vmcnt count before the step's barrier. Each wave owns the 32 rows
// x (32 gate + 32 up) columns (gate_up) or 64 columns (down) of the item, decodes its weight rows
// from LDS in registers (q4k_mfma.h) and runs the MFMAs. The slabs of one tile run on one XCD
// (block b serves XCD b % 8), where they share the tile's rows in L2. Results leave through raw
// buffer stores whose descriptor ends at the tile's last row.
#include "common.h"
#include "moe_internal.h"
#include "lds_dma.h"
#include "q4k_mfma.h"
#include "shared_small.h"

namespace moe {
namespace g6 {

using dma::lds_addr;
using dma::opaque;
using dma::wait_vm;
using q4m::a_swz;
using q4m::mfma;
using q4m::q4_frag;
using q4m::q4_scales;
using q4m::q_swz;

constexpr int kBM = MOE_GEMM6_BM;       // 32 activation rows per tile
constexpr int kBN = 256;                // weight rows per item
constexpr int kSBB = 144;               // bytes per Q4_K super-block row (256 K)
constexpr int kR = 4;                   // ring depth (K steps) of A and Q
constexpr int kXcd = 8;
constexpr int kWaves = 4;
constexpr int kQI = kBN * 2 / 64 / kWaves;   // nibble loads per wave per K step (2)
constexpr int kAI = kBM * 8 / 64 / kWaves;   // activation loads per wave per K step (1)
// loads a step issues (activations and nibbles of step ks + 3); a super-block's first step also
// issues the next headers
constexpr int kPerStep = kAI + kQI;
static_assert(kAI == 1 && kQI == 2 && kBN / 64 == kWaves, "load split assumes 32 x 256 items");

struct Smem {
  uint8_t A[kR][kBM * 128];
  uint8_t Q[kR][kBN * 32];
  uint8_t Hd[2][kBN * 16];
};
static_assert(sizeof(Smem) * 2 <= 160 * 1024, "two blocks per CU");

struct Item {
  int e, m0, mend, col;
};

// Block b: XCD x = b % 8, q = b / 8 -> slab q % ncol of tile 8 (q / ncol) + x. False past the list.
__device__ __forceinline__ bool get_item(const int32_t* __restrict__ tiles,
                                         const int32_t* __restrict__ offsets, int ncol, Item& it) {
  const int x = blockIdx.x % kXcd, q = blockIdx.x / kXcd;
  const int t = (q / ncol) * kXcd + x;
  if (t >= tiles[0]) return false;
  it.col = q % ncol;
  it.e = tiles[1 + 2 * t];
  it.m0 = tiles[2 + 2 * t];
  it.mend = min(it.m0 + kBM, offsets[it.e + 1]);
  return true;
}

// Per-thread load geometry. Thread t: activation unit t (tile row t >> 3, physical chunk t & 7,
// logical chunk (t & 7) ^ swz(row)); Q load j of wave w, lane l: unit 64 (w + 4 j) + l = weight row
// u >> 1, logical half (u & 1) ^ q_swz(row); header load: weight row 64 w + l.
struct Geo {
  const uint8_t* ab;                    // activation rows' base
  uint32_t aoff;                        // byte offset of this thread's activation chunk (step 0)
  const uint8_t* qb[kQI];               // Q load j's base (the headers of waves 0, 1: qb[0]; 2, 3: qb[1])
  uint32_t qoff[kQI];
  uint32_t hoff;
  uint32_t la, lq, lh;                  // LDS address of this wave's first unit in slot 0
};

__device__ __forceinline__ void ld_step(const Geo& g, int slot, int ks) {
  dma::load16(g.aoff, g.ab + (size_t)ks * 128, g.la + slot * (kBM * 128));
  const int off = (ks >> 2) * kSBB + 32 * (ks & 3);
#pragma unroll
  for (int j = 0; j < kQI; ++j) dma::load16(g.qoff[j], g.qb[j] + off, g.lq + slot * (kBN * 32) + j * 4096);
}
__device__ __forceinline__ void ld_hdr(const Geo& g, int slot, int sb) {
  const uint8_t* hb = __builtin_amdgcn_readfirstlane(threadIdx.x >> 7) ? g.qb[kQI - 1] : g.qb[0];
  dma::load16(g.hoff, hb + sb * kSBB, g.lh + slot * (kBN * 16));
}

// The item's K steps: acc[0] (weight rows n0 + l % 32) and acc[1] (n1 + l % 32) over the tile's
// 32 rows. nk = K / 64 steps (a multiple of 4).
__device__ __forceinline__ void run(const Geo& g, int nk, int n0, int n1, Smem& sm, f32x16_t (&acc)[2]) {
  const int lane = threadIdx.x & 63;
  const int h = lane >> 5, r = lane & 31;
  const int nsb = nk / 4;
  int aoff[4];
#pragma unroll
  for (int ss = 0; ss < 4; ++ss) aoff[ss] = 16 * (8 * r + ((4 * (ss >> 1) + 2 * h + (ss & 1)) ^ a_swz(r)));
  const int qo0 = 16 * (2 * (n0 + r) + (h ^ q_swz(r)));
  const int qo1 = 16 * (2 * (n1 + r) + (h ^ q_swz(r)));
  // prologue: super-block 0's headers, steps 0..2's activations and nibbles
  ld_hdr(g, 0, 0);
#pragma unroll
  for (int j = 0; j < kR - 1; ++j) ld_step(g, j, min(j, nk - 1));
  acc[0] = (f32x16_t){};
  acc[1] = (f32x16_t){};
  for (int sb = 0; sb < nsb; ++sb) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int ks = 4 * sb + s;
      // this wave's loads of step ks were issued three steps ago; after them came the loads of
      // two steps and, unless s == 0, one super-block's headers
      if (s == 0) wait_vm<2 * kPerStep>();
      else wait_vm<2 * kPerStep + 1>();
      __syncthreads();
      // into the slot step ks - 1 used (past the end: clamped repeats into slots nothing reads)
      ld_step(g, (s + 3) & 3, min(ks + 3, nk - 1));
      if (s == 0) ld_hdr(g, (sb + 1) & 1, min(sb + 1, nsb - 1));
      const uint8_t* As = sm.A[s];
      const uint8_t* Qs = sm.Q[s];
      const uint8_t* Hs = sm.Hd[sb & 1];
      const uint4 hdr0 = *reinterpret_cast<const uint4*>(Hs + 16 * (n0 + r));
      const uint4 hdr1 = *reinterpret_cast<const uint4*>(Hs + 16 * (n1 + r));
      const uint4 q0 = *reinterpret_cast<const uint4*>(Qs + qo0);
      const uint4 q1 = *reinterpret_cast<const uint4*>(Qs + qo1);
      f16x2_t ds0l, nd0l, ds0h, nd0h, ds1l, nd1l, ds1h, nd1h;
      q4_scales(hdr0, 2 * s, ds0l, nd0l);
      q4_scales(hdr0, 2 * s + 1, ds0h, nd0h);
      q4_scales(hdr1, 2 * s, ds1l, nd1l);
      q4_scales(hdr1, 2 * s + 1, ds1h, nd1h);
#pragma unroll
      for (int ss = 0; ss < 4; ++ss) {
        const uint4 a = *reinterpret_cast<const uint4*>(As + aoff[ss]);
        uint4 bg, bu;
        if (ss == 0) { bg = q4_frag<false>(q0.x, q0.y, ds0l, nd0l); bu = q4_frag<false>(q1.x, q1.y, ds1l, nd1l); }
        else if (ss == 1) { bg = q4_frag<false>(q0.z, q0.w, ds0l, nd0l); bu = q4_frag<false>(q1.z, q1.w, ds1l, nd1l); }
        else if (ss == 2) { bg = q4_frag<true>(q0.x, q0.y, ds0h, nd0h); bu = q4_frag<true>(q1.x, q1.y, ds1h, nd1h); }
        else { bg = q4_frag<true>(q0.z, q0.w, ds0h, nd0h); bu = q4_frag<true>(q1.z, q1.w, ds1h, nd1h); }
        acc[0] = mfma(a, bg, acc[0]);
        acc[1] = mfma(a, bu, acc[1]);
      }
    }
  }
}

__device__ __forceinline__ void geo_lds(Geo& g, Smem& sm, int wave) {
  g.la = lds_addr(sm.A[0]) + 1024 * wave;
  g.lq = lds_addr(sm.Q[0]) + 1024 * wave;
  g.lh = lds_addr(sm.Hd[0]) + 1024 * wave;
}

}  // namespace g6

// the shared-expert blocks reduce their four waves' partial tiles in the routed blocks' LDS
static_assert(sizeof(g6::Smem) >= shs::red_floats<4>() * sizeof(float), "shared-expert partial tiles fit in LDS");

// S [P, I] f16 (sorted order) = SiLU(x16[token] . gate^T) * (x16[token] . up^T) per tile row
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_gemm6_gateup(
    const uint16_t* __restrict__ x16, const uint8_t* __restrict__ wg, const uint8_t* __restrict__ wu,
    size_t estride, const int32_t* __restrict__ tiles, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ sorted_pairs, int K, int H, int I, uint16_t* __restrict__ S) {
  using namespace g6;
  __shared__ __attribute__((aligned(16))) Smem sm;
  Item it;
  if (!get_item(tiles, offsets, I / 128, it)) return;
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const size_t rowb = (size_t)(H / 256) * kSBB;
  Geo g;
  geo_lds(g, sm, wave);
  {
    const int row = t >> 3;
    const uint32_t tok = (uint32_t)sorted_pairs[min(it.m0 + row, it.mend - 1)] / (uint32_t)K;
    g.ab = reinterpret_cast<const uint8_t*>(x16);
    g.aoff = tok * (uint32_t)H * 2u + 16u * (uint32_t)((t & 7) ^ a_swz(row));
  }
  g.qb[0] = wg + (size_t)it.e * estride + (size_t)it.col * 128 * rowb;
  g.qb[1] = wu + (size_t)it.e * estride + (size_t)it.col * 128 * rowb;
#pragma unroll
  for (int j = 0; j < kQI; ++j) {
    // Q load 0 covers gate rows 32 w + l / 2, load 1 the up rows 128 + 32 w + l / 2
    const int u = 64 * (wave + kWaves * j) + lane, n = u >> 1;
    g.qoff[j] = (uint32_t)((n & 127) * rowb) + 16u + 16u * (uint32_t)((u & 1) ^ q_swz(n));
  }
  g.hoff = (uint32_t)(((64 * wave + lane) & 127) * rowb);
  f32x16_t acc[2];
  run(g, H / 64, 32 * wave, 128 + 32 * wave, sm, acc);
  // row 8 (r >> 2) + 4 h + (r & 3) of the tile, column it.col 128 + 32 w + l % 32
  const __amdgpu_buffer_rsrc_t rs = dma::rsrc(S + (size_t)it.m0 * I, (it.mend - it.m0) * I * 2);
  const int rs2 = opaque(I * 2);
  const int lane_off = (4 * (lane >> 5) * I + it.col * 128 + 32 * wave + (lane & 31)) * 2;
#pragma unroll
  for (int rq = 0; rq < 4; ++rq) {
    const int vo = lane_off + 8 * rq * rs2;
#pragma unroll
    for (int r3 = 0; r3 < 4; ++r3) {
      const int r = 4 * rq + r3;
      const float gv = acc[0][r];
      float v = gv * __builtin_amdgcn_rcpf(1.0f + __expf(-gv)) * acc[1][r];
      v = fminf(fmaxf(v, -65504.0f), 65504.0f);
      __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, (_Float16)v), rs, vo + r3 * rs2, 0, 0);
    }
  }
  // no load (the clamped repeats at the end) may still be writing this block's LDS at exit
  wait_vm<0>();
}

// y [P, H] (sorted order; f32, or f16 saturated when Y16) = S . down^T per tile row
template <bool Y16>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_gemm6_down(
    const uint16_t* __restrict__ S, const uint8_t* __restrict__ wd, size_t estride,
    const int32_t* __restrict__ tiles, const int32_t* __restrict__ offsets, int H, int I,
    void* __restrict__ y, MoeShJob sh) {
  using namespace g6;
  __shared__ __attribute__((aligned(16))) Smem sm;
  const int nr = (int)gridDim.x - sh.n;
  if ((int)blockIdx.x >= nr) {
    // the small-T shared expert's down: y = shared_raw
    const int b = (int)blockIdx.x - nr, nslab = sh.H / 32;
    shs::down_tile<4, 32>(sh.S, sh.w0, sh.T, sh.H, sh.Is, b % nslab, (b / nslab) * 32, sh.y,
                          reinterpret_cast<float*>(&sm));
    return;
  }
  Item it;
  if (!get_item(tiles, offsets, H / kBN, it)) return;
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const size_t rowb = (size_t)(I / 256) * kSBB;
  Geo g;
  geo_lds(g, sm, wave);
  {
    const int row = t >> 3;
    g.ab = reinterpret_cast<const uint8_t*>(S + (size_t)it.m0 * I);
    g.aoff = (uint32_t)min(row, it.mend - it.m0 - 1) * (uint32_t)I * 2u + 16u * (uint32_t)((t & 7) ^ a_swz(row));
  }
  const uint8_t* w = wd + (size_t)it.e * estride + (size_t)it.col * kBN * rowb;
  g.qb[0] = w;
  g.qb[1] = w;
#pragma unroll
  for (int j = 0; j < kQI; ++j) {
    const int u = 64 * (wave + kWaves * j) + lane, n = u >> 1;
    g.qoff[j] = (uint32_t)(n * rowb) + 16u + 16u * (uint32_t)((u & 1) ^ q_swz(n));
  }
  g.hoff = (uint32_t)((64 * wave + lane) * rowb);
  f32x16_t acc[2];
  run(g, I / 64, 64 * wave, 64 * wave + 32, sm, acc);
  constexpr int kB = Y16 ? 2 : 4;   // bytes per element
  char* yb = reinterpret_cast<char*>(y) + (size_t)it.m0 * H * kB;
  const __amdgpu_buffer_rsrc_t rs = dma::rsrc(yb, (it.mend - it.m0) * H * kB);
  const int rsb = opaque(H * kB);
  const int lane_off = (4 * (lane >> 5) * H + it.col * kBN + 64 * wave + (lane & 31)) * kB;
#pragma unroll
  for (int rq = 0; rq < 4; ++rq) {
    const int vo = lane_off + 8 * rq * rsb;
#pragma unroll
    for (int r3 = 0; r3 < 4; ++r3) {
      const int r = 4 * rq + r3;
      // the builtins' data operand is an integer: the bits, copied out of the vector first
      float v0 = acc[0][r], v1 = acc[1][r];
      if constexpr (Y16) {
        v0 = fminf(fmaxf(v0, -65504.0f), 65504.0f);
        v1 = fminf(fmaxf(v1, -65504.0f), 65504.0f);
        __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, (_Float16)v0), rs, vo + r3 * rsb, 0, 0);
        __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, (_Float16)v1), rs, vo + r3 * rsb + 64, 0, 0);
      } else {
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v0), rs, vo + r3 * rsb, 0, 0);
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v1), rs, vo + r3 * rsb + 128, 0, 0);
      }
    }
  }
  wait_vm<0>();
}

}  // namespace moe

using namespace moe;

// one block per (tile, slab): the tile list's capacity rounded up to whole groups of 8 tiles
static dim3 g6_grid(int max_tiles, int ncol) {
  return dim3((unsigned)((max_tiles + g6::kXcd - 1) / g6::kXcd * ncol * g6::kXcd));
}

// the shared-expert down blocks need H % 32 == 0 (32-column slabs) and I_s % 256 == 0 (K split
// over 4 waves in 64-wide chunks)
static int check_shjob(const MoeShJob* sh) {
  if (!sh || sh->n == 0) return MOE_OK;
  if (sh->H % 32 || sh->Is % 256 || !sh->S || !sh->w0 || !sh->y)
    return moe_set_error(MOE_E_UNSUPPORTED, "gemm6: shared-expert blocks need H %% 32 == 0, I_s %% 256 == 0 and every pointer");
  const int want = moe_shjob_down_blocks(sh->T, sh->H);
  if (sh->n != want) return moe_set_error(MOE_E_ARG, "gemm6: %d shared-expert blocks given, %d needed", sh->n, want);
  return MOE_OK;
}

int moe_launch_gemm6_gateup(const uint16_t* x16, const void* w_gate, const void* w_up,
                            size_t expert_stride, const int32_t* tiles, int max_tiles,
                            const int32_t* offsets, const int32_t* sorted_pairs, int K, int H,
                            int I, uint16_t* S, hipStream_t st) {
  if (H % 256 || I % 128)
    return moe_set_error(MOE_E_UNSUPPORTED, "gemm6 gate_up needs H %% 256 == 0, I %% 128 == 0");
  hipLaunchKernelGGL(k_gemm6_gateup, g6_grid(max_tiles, I / 128), dim3(256), 0, st, x16,
                     reinterpret_cast<const uint8_t*>(w_gate), reinterpret_cast<const uint8_t*>(w_up),
                     expert_stride, tiles, offsets, sorted_pairs, K, H, I, S);
  return moe_check_launch("gemm6_gateup");
}

int moe_launch_gemm6_down(const uint16_t* S, const void* w_down, size_t expert_stride,
                          const int32_t* tiles, int max_tiles, const int32_t* offsets, int H, int I,
                          void* y, int y16, hipStream_t st, const MoeShJob* sh) {
  if (I % 256 || H % 256) return moe_set_error(MOE_E_UNSUPPORTED, "gemm6 down needs H %% 256 == 0, I %% 256 == 0");
  { const int rc_ = check_shjob(sh); if (rc_ != MOE_OK) return rc_; }
  const MoeShJob job = sh ? *sh : MoeShJob{};
  dim3 grid = g6_grid(max_tiles, H / 256);
  grid.x += (unsigned)job.n;
  const uint8_t* w = reinterpret_cast<const uint8_t*>(w_down);
  if (y16)
    hipLaunchKernelGGL(k_gemm6_down<true>, grid, dim3(256), 0, st, S, w, expert_stride, tiles, offsets, H, I, y, job);
  else
    hipLaunchKernelGGL(k_gemm6_down<false>, grid, dim3(256), 0, st, S, w, expert_stride, tiles, offsets, H, I, y, job);
  return moe_check_launch("gemm6_down");
}
