// Prefill-path down GEMM for Q6_K experts with the weight decode in the MFMA waves (gfx950,
// v_mfma_f32_32x32x16_f16, f32 accumulation): the 210-byte super-block counterpart of gemm4.hip's
// Q4_K down kernel.
//
// Work item, grid and block as in gemm4.hip: one tile of up to 160 sorted (token, slot) rows of
// one expert times one 256-row slab of the down matrix; a persistent grid of two 4-wave blocks per
// CU, block b serving XCD b % 8 and taking that XCD's items with stride gridDim.x / 8.
//
// Q6_K (ggml dequantize_row_q6_K): element s < 64 of K step (half hf, part gp) of a super-block
// takes nibble gp of ql byte 64 hf + s, bits 4 gp + 2 (s / 32) of qh byte 32 hf + s % 32 and int8
// scale 8 hf + 4 gp + s / 16, times the f16 d. Both K steps of a half read the same 64 ql and 32 qh
// bytes, so the weights move one half (two K steps) at a time. Super-blocks are 210 bytes: piece
// starts fall on any even byte. The slab (256 rows x I / 256 super-blocks) is contiguous and
// 16-byte aligned, so each piece is fetched as the 16-byte units that cover it (super-block g of
// the slab starts 2 g mod 16 bytes into its first unit) and that offset is undone when the piece
// is read out of LDS.
//
// LDS (80 KB, two blocks per CU):
//   A[2]: f16 activations of one 64-wide K step, 160 rows x 128 B, 16-byte chunk c of row m at
//         chunk c ^ a_swz(m) (as gemm4.hip);
//   R:    one half of the slab's 256 rows, 10 units per row: units 0-4 cover the 64 ql bytes, 5-7
//         the 32 qh bytes, 8-9 the super-block's 16 scales and d. Unit i of row n sits at
//         R + 4096 i + 16 slot(n); slot(n) transposes n's low five bits (8 x 4 -> 4 x 8), so the
//         32 lanes that read one dword each from rows n0, n0 + 2, .., n0 + 62 (at offsets that
//         follow n % 4) hit 16 different banks (two lanes per bank).
// A half starts when R and the step's A have landed: every lane copies its pieces out of R into
// registers (lane (r, h) of wave w: weight rows 64 w + 2 r and 64 w + 2 r + 1, so that it ends
// with two adjacent output columns; ql bytes 16 h .. 16 h + 15 and 32 + 16 h .. 32 + 16 h + 15,
// qh bytes 16 h .. 16 h + 15, the half's 8 scales and d), the waves meet at a barrier and request
// the next half into R, which then has two K steps to land. A is requested one step ahead. k order
// inside a K step as gemm4.hip: substep ss covers the 16-byte chunks 4 (ss >> 1) + (ss & 1) (lane
// half 0) and that + 2 (half 1).
// Decode (exact): per register of four elements, the two qh bits go to bits 4-5 of each byte and
// the nibble below them; one perm per pair puts two 6-bit q under the f16 magic 0x6400 (1024 + q),
// one packed subtract of 1056 leaves q - 32 and one packed multiply by f16(d * sc) (d * sc exact
// in f32, rounded to f16 once) rounds once: the same values as gemm3.hip's Q6_K decode.
#include "common.h"
#include "moe_internal.h"
#include "lds_dma.h"
#include "q4k_mfma.h"

namespace moe {
namespace g7 {

using dma::opaque;
using dma::tid_fresh;
using dma::wait_vm;
using q4m::a_swz;
using q4m::and_or_s;
using q4m::mfma;
typedef float float2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

constexpr int kBM = MOE_GEMM3_BM;            // 160 activation rows per tile
constexpr int kMG = kBM / 32;                // MFMA row groups
constexpr int kBN = 256;                     // weight rows per item
constexpr int kXcd = 8;
constexpr int kWaves = 4;
constexpr int kBlocksPerCu = 2;
constexpr int kSBB = 210;                    // bytes per Q6_K super-block (256 K)
constexpr int kRU = 10;                      // 16-byte units per weight row per half
constexpr int kAI = kBM * 8 / 64 / kWaves;   // A loads per wave per K step (5)
constexpr int kStores = kMG * 32;            // epilogue stores per wave per item
constexpr int kStoreWait = kStores < 63 ? kStores : 63;
static_assert(kAI == 5 && kBN / 64 == kWaves, "load split assumes 160 x 256 items");

struct Smem {
  uint8_t A[2][kBM * 128];
  uint8_t R[kRU][kBN * 16];
};
static_assert(sizeof(Smem) * kBlocksPerCu <= 160 * 1024, "two blocks per CU");

__device__ __forceinline__ int slot_of(int n) { return (n & ~31) | ((n & 3) << 3) | ((n >> 2) & 7); }
__device__ __forceinline__ int row_of(int p) { return (p & ~31) | ((p & 7) << 2) | ((p >> 3) & 3); }

// slab byte offset of the 16-byte unit that holds the first byte of super-block g of the slab
__device__ __forceinline__ uint32_t unit_start(int g) { return (uint32_t)(kSBB * g) & ~15u; }

// offset of R unit i of half hf from the super-block's unit_start
__host__ __device__ constexpr int xoff(int i, int hf) {
  return i < 5 ? 64 * hf + 16 * i : i < 8 ? 128 + 32 * hf + 16 * (i - 5) : 192 + 16 * (i - 8);
}

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

// per-item operand addresses (uniform)
struct Addr {
  const uint8_t* wb;                    // the slab's first byte
  const uint8_t* ab;                    // the tile's first activation row
};

__device__ __forceinline__ void item_addr(Addr& ad, const Item& it, const uint16_t* S,
                                          const uint8_t* wd, size_t estride, size_t rowb, int I) {
  ad.wb = wd + (size_t)it.e * estride + (size_t)it.col * kBN * rowb;
  ad.ab = reinterpret_cast<const uint8_t*>(S + (size_t)it.m0 * I);
}

// this wave's LDS addresses (slot 0 of A, unit 0 of R), the weight row its R loads cover and its
// A load offset: load j of thread t covers tile row t / 8 + 32 j, 16-byte chunk t % 8 of the
// step's 128 bytes, stored at chunk position (t % 8) ^ a_swz(row) (a_swz(row + 32 j) = a_swz(row),
// so load j adds 32 j rows to the uniform base). Rows past the tile are read as they are (the next
// expert's rows, or the padding rows past S's last): they only reach output rows past the tile,
// which the epilogue's stores drop.
struct Ld {
  uint32_t la, lr, aoff;
  int nrow;
};

__device__ __forceinline__ void ld_a(const Ld& ld, const Addr& ad, int I, int slot, int ks) {
  const uint8_t* b = ad.ab + (size_t)ks * 128;
#pragma unroll
  for (int j = 0; j < kAI; ++j)
    dma::load16(ld.aoff + (uint32_t)(j * 64 * I), b, ld.la + slot * (kBM * 128) + j * 4096);
}

// half hf of super-block sb: unit i of this lane's row into R unit i
template <int HF>
__device__ __forceinline__ void ld_r(const Ld& ld, const Addr& ad, int nsb, int sb) {
  const uint32_t u = unit_start(ld.nrow * nsb + sb);
#pragma unroll
  for (int i = 0; i < kRU; ++i) dma::load16(u, ad.wb + xoff(i, HF), ld.lr + i * 4096);
}

// ------------------------------------------------------------------------------- decode --
// one weight row's half, in registers: p0 / p1 = ql bytes 16 h .. + 15 / 32 + 16 h .. + 15,
// hh = qh bytes 16 h .. + 15, sc = the half's 8 scales, d
struct Row6 {
  uint32_t p0[4], p1[4], hh[4];
  f16x2_t ds[2];                        // part gp: {f16(d sc[4 gp + h]), f16(d sc[4 gp + 2 + h])}
};

// rows n (= 64 w + 2 r) and n + 1 of half hf of super-block sb out of R (byte offset
// o = 2 g mod 16 of super-block g = n nsb + sb within its first unit)
template <int HF>
__device__ __forceinline__ void stash_row(const uint8_t* R, int n, int nsb, int sb, int h, Row6& w) {
  const int o = (2 * (n * nsb + sb)) & 15, q = o >> 2;
  const uint32_t sh = (uint32_t)(o & 3);
  const int base = 16 * slot_of(n);
  // window dword q + t (t < 5) of the row: unit (q + t) / 4, dword (q + t) % 4 of that unit
  int a[5];
#pragma unroll
  for (int t = 0; t < 5; ++t) a[t] = base + 4096 * ((q + t) >> 2) + 4 * ((q + t) & 3);
  auto rd = [&](int addr) { return *reinterpret_cast<const uint32_t*>(R + addr); };
  auto piece = [&](int off, uint32_t (&dst)[4]) {   // 16 bytes from window dword q + 4 h + off / 4
    uint32_t v[5];
#pragma unroll
    for (int t = 0; t < 5; ++t) v[t] = rd(a[t] + 4096 * h + off);
#pragma unroll
    for (int i = 0; i < 4; ++i) dst[i] = __builtin_amdgcn_alignbyte(v[i + 1], v[i], sh);
  };
  piece(0, w.p0);
  piece(2 * 4096, w.p1);
  piece(5 * 4096, w.hh);
  // scales 8 hf .. 8 hf + 7 (window dwords q + 2 hf ..) and d (window bytes 16, 17)
  uint32_t v[3];
#pragma unroll
  for (int t = 0; t < 3; ++t) v[t] = rd(a[t + 2 * HF] + 8 * 4096);
  const uint32_t sc[2] = {__builtin_amdgcn_alignbyte(v[1], v[0], sh), __builtin_amdgcn_alignbyte(v[2], v[1], sh)};
  const float d = f16_to_f32((rd(a[4] + 8 * 4096) >> (8 * sh)) & 0xFFFFu);
  // f16(d * sc) of scales 4 gp + 2 j + h (d * sc exact in f32, rounded to f16 once)
#pragma unroll
  for (int gp = 0; gp < 2; ++gp)
    w.ds[gp] = (f16x2_t){(_Float16)(d * (float)(int)(int8_t)(sc[gp] >> (8 * h))),
                         (_Float16)(d * (float)(int)(int8_t)(sc[gp] >> (16 + 8 * h)))};
}

// the 8 f16 of substep ss's B fragment (chunk 4 (ss >> 1) + 2 h + (ss & 1) of part gp)
template <int GP, int SS>
__device__ __forceinline__ uint4 q6_frag(const Row6& w, f16x2_t ds) {
  constexpr int hs = 4 * GP + 2 * (SS >> 1);
  const f16x2_t off = {(_Float16)1056.0f, (_Float16)1056.0f};
  uint32_t o[4];
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const uint32_t wv = (SS >> 1) ? w.p1[2 * (SS & 1) + e] : w.p0[2 * (SS & 1) + e];
    const uint32_t hv = w.hh[2 * (SS & 1) + e];
    const uint32_t h30 = (hs >= 4 ? (hv >> (hs - 4)) : (hv << (4 - hs))) & 0x30303030u;
    const uint32_t q6 = and_or_s(GP ? (wv >> 4) : wv, 0x0F0F0F0Fu, h30);
    const f16x2_t a = __builtin_bit_cast(f16x2_t, __builtin_amdgcn_perm(0x64646464u, q6, 0x04010400u)) - off;
    const f16x2_t b = __builtin_bit_cast(f16x2_t, __builtin_amdgcn_perm(0x64646464u, q6, 0x04030402u)) - off;
    o[2 * e] = __builtin_bit_cast(uint32_t, a * ds);
    o[2 * e + 1] = __builtin_bit_cast(uint32_t, b * ds);
  }
  return make_uint4(o[0], o[1], o[2], o[3]);
}

// the MFMAs of one K step (part gp of the stashed half) over NG row groups
template <int NG, int GP>
__device__ __forceinline__ void mma_step(const uint8_t* As, const int (&aoff)[4], const Row6& w0,
                                         const Row6& w1, f32x16_t (&acc)[kMG][2]) {
  const f16x2_t d00 = __builtin_shufflevector(w0.ds[GP], w0.ds[GP], 0, 0);
  const f16x2_t d01 = __builtin_shufflevector(w0.ds[GP], w0.ds[GP], 1, 1);
  const f16x2_t d10 = __builtin_shufflevector(w1.ds[GP], w1.ds[GP], 0, 0);
  const f16x2_t d11 = __builtin_shufflevector(w1.ds[GP], w1.ds[GP], 1, 1);
  auto afrag = [&](int ss, uint4 (&a)[NG]) {
#pragma unroll
    for (int mg = 0; mg < NG; ++mg) a[mg] = *reinterpret_cast<const uint4*>(As + aoff[ss] + 4096 * mg);
  };
  uint4 ac[NG];
  afrag(0, ac);
  uint4 bg = q6_frag<GP, 0>(w0, d00), bu = q6_frag<GP, 0>(w1, d10);
#pragma unroll
  for (int ss = 0; ss < 4; ++ss) {
#pragma unroll
    for (int mg = 0; mg < NG; ++mg) {
      acc[mg][0] = mfma(ac[mg], bg, acc[mg][0]);
      acc[mg][1] = mfma(ac[mg], bu, acc[mg][1]);
    }
    // substep ss + 1's operands into the same registers (an MFMA holds its operands from issue)
    if (ss == 0) { afrag(1, ac); bg = q6_frag<GP, 1>(w0, d00); bu = q6_frag<GP, 1>(w1, d10); }
    if (ss == 1) { afrag(2, ac); bg = q6_frag<GP, 2>(w0, d01); bu = q6_frag<GP, 2>(w1, d11); }
    if (ss == 2) { afrag(3, ac); bg = q6_frag<GP, 3>(w0, d01); bu = q6_frag<GP, 3>(w1, d11); }
  }
}

// ------------------------------------------------------------------------------- epilogue --
// Lane r of wave w holds output columns 64 w + 2 r (acc[.][0]) and 64 w + 2 r + 1 (acc[.][1]) of
// rows 32 mg + 8 (i / 4) + 4 h + i % 4: one 4-byte store per row (Y16: the pair as f16, saturated
// to +-65504) or one 8-byte store (f32). Raw buffer stores whose descriptor ends at the tile's
// last row drop the rows past it (the whole offset is in the VGPR operand).
template <bool Y16, int NG>
__device__ __forceinline__ void epilogue(void* y, int H, const Item& it, int wave, int lane,
                                         const f32x16_t (&acc)[kMG][2]) {
  constexpr int kB = Y16 ? 2 : 4;
  char* yb = reinterpret_cast<char*>(y) + (size_t)it.m0 * H * kB;
  const __amdgpu_buffer_rsrc_t rs = dma::rsrc(yb, (it.mend - it.m0) * H * kB);
  const int rsb = opaque(H * kB);
  const int lane_off = (4 * (lane >> 5) * H + it.col * kBN + 64 * wave + 2 * (lane & 31)) * kB;
#pragma unroll
  for (int mg = 0; mg < NG; ++mg) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int vo = lane_off + (32 * mg + 8 * (i >> 2) + (i & 3)) * rsb;
      const float v0 = acc[mg][0][i], v1 = acc[mg][1][i];
      if constexpr (Y16) {
        const f16x2_t p = {(_Float16)__builtin_amdgcn_fmed3f(v0, -65504.0f, 65504.0f),
                           (_Float16)__builtin_amdgcn_fmed3f(v1, -65504.0f, 65504.0f)};
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, p), rs, vo, 0, 0);
      } else {
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2_t, (float2_t){v0, v1}), rs,
                                              vo, 0, 0);
      }
    }
  }
}

// ------------------------------------------------------------------------------- one item --
// Steps ks = 4 sb + 2 hf + gp read A[gp]. Half (sb, hf) starts with the wait for R and A(ks),
// the barrier, the request of A(ks + 1), the copy out of R and a second barrier after which R
// takes the next half (in the item's last half: the next item's first one, or with no next item a
// repeat of a valid half into R that nothing reads again). Part gp = 1 waits for A(ks) (R's ten
// loads issued after it may stay in flight) and requests A(ks + 1) (in the last step: the next
// item's A(0), or a repeat). Every step thus issues the same loads and the vmcnt counts are
// constants; before an item's first step the previous item's epilogue stores are the newest
// operations.
template <int NG, bool Y16>
__device__ __forceinline__ void run_item(const Ld& ld, const Addr& ca, const Addr& na, bool has_next,
                                         bool first, int nsb, int I, int H, void* y, const Item& it,
                                         int wave, Smem& sm) {
  const int lane = threadIdx.x & 63;
  const int h = lane >> 5, r = lane & 31;
  const int n = 64 * wave + 2 * r;
  int aoff[4];
#pragma unroll
  for (int ss = 0; ss < 4; ++ss)
    aoff[ss] = 16 * (8 * r + ((4 * (ss >> 1) + 2 * h + (ss & 1)) ^ a_swz(r)));
  const uint8_t* R = sm.R[0];
  f32x16_t acc[kMG][2];
#pragma unroll
  for (int mg = 0; mg < kMG; ++mg) { acc[mg][0] = (f32x16_t){}; acc[mg][1] = (f32x16_t){}; }
  Row6 w0, w1;
  for (int sb = 0; sb < nsb; ++sb) {
    const bool last_sb = sb == nsb - 1;
    const int ks = 4 * sb;
    // ---- half 0, part 0
    if (sb == 0 && !first) wait_vm<kStoreWait>(); else wait_vm<0>();
    __syncthreads();
    ld_a(ld, ca, I, 1, ks + 1);
    stash_row<0>(R, n, nsb, sb, h, w0);
    stash_row<0>(R, n + 1, nsb, sb, h, w1);
    __syncthreads();
    ld_r<1>(ld, ca, nsb, sb);
    mma_step<NG, 0>(sm.A[0], aoff, w0, w1, acc);
    // ---- half 0, part 1
    wait_vm<kRU>();
    __syncthreads();
    ld_a(ld, ca, I, 0, ks + 2);
    mma_step<NG, 1>(sm.A[1], aoff, w0, w1, acc);
    // ---- half 1, part 0
    wait_vm<0>();
    __syncthreads();
    ld_a(ld, ca, I, 1, ks + 3);
    stash_row<1>(R, n, nsb, sb, h, w0);
    stash_row<1>(R, n + 1, nsb, sb, h, w1);
    __syncthreads();
    if (!last_sb) ld_r<0>(ld, ca, nsb, sb + 1);
    else if (has_next) ld_r<0>(ld, na, nsb, 0);
    else ld_r<0>(ld, ca, nsb, sb);
    mma_step<NG, 0>(sm.A[0], aoff, w0, w1, acc);
    // ---- half 1, part 1
    wait_vm<kRU>();
    __syncthreads();
    if (!last_sb) ld_a(ld, ca, I, 0, ks + 4);
    else if (has_next) ld_a(ld, na, I, 0, 0);
    else ld_a(ld, ca, I, 0, ks + 3);
    mma_step<NG, 1>(sm.A[1], aoff, w0, w1, acc);
  }
  epilogue<Y16, NG>(y, H, it, wave, lane, acc);
}

template <bool Y16>
__device__ __forceinline__ void run_n(int ng, const Ld& ld, const Addr& ca, const Addr& na,
                                      bool has_next, bool first, int nsb, int I, int H, void* y,
                                      const Item& it, int wave, Smem& sm) {
  if (ng >= 5) run_item<5, Y16>(ld, ca, na, has_next, first, nsb, I, H, y, it, wave, sm);
  else if (ng == 4) run_item<4, Y16>(ld, ca, na, has_next, first, nsb, I, H, y, it, wave, sm);
  else if (ng == 3) run_item<3, Y16>(ld, ca, na, has_next, first, nsb, I, H, y, it, wave, sm);
  else if (ng == 2) run_item<2, Y16>(ld, ca, na, has_next, first, nsb, I, H, y, it, wave, sm);
  else run_item<1, Y16>(ld, ca, na, has_next, first, nsb, I, H, y, it, wave, sm);
}

}  // namespace g7

// ----------------------------------------------------------------------------------- kernel --
template <bool Y16>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_gemm7_down(
    const uint16_t* __restrict__ S, const uint8_t* __restrict__ wd, size_t estride,
    const int32_t* __restrict__ tiles, const int32_t* __restrict__ offsets, int H, int I,
    void* __restrict__ y) {
  using namespace g7;
  __shared__ __attribute__((aligned(16))) Smem sm;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int stride = gridDim.x / kXcd;
  const int ncol = H / kBN, nsb = I / 256;
  const size_t rowb = (size_t)nsb * kSBB;
  int q = blockIdx.x / kXcd;
  Item cur;
  if (!get_item(tiles, offsets, q, ncol, cur)) return;
  Ld ld;
  ld.la = dma::lds_addr(sm.A[0]) + 1024 * wave;
  ld.lr = dma::lds_addr(sm.R[0]) + 1024 * wave;
  ld.nrow = row_of(64 * wave + lane);
  {
    const int t = tid_fresh(), m = t >> 3;
    ld.aoff = (uint32_t)m * (uint32_t)I * 2u + 16u * (uint32_t)((t & 7) ^ a_swz(m));
  }
  Addr ca;
  item_addr(ca, cur, S, wd, estride, rowb, I);
  ld_r<0>(ld, ca, nsb, 0);
  ld_a(ld, ca, I, 0, 0);
  bool first = true;
  for (;;) {
    Item nx;
    const bool has_next = get_item(tiles, offsets, q + stride, ncol, nx);
    if (!has_next) nx = cur;
    Addr na;
    item_addr(na, nx, S, wd, estride, rowb, I);
    const int ng = __builtin_amdgcn_readfirstlane((cur.mend - cur.m0 + 31) >> 5);
    run_n<Y16>(ng, ld, ca, na, has_next, first, nsb, I, H, y, cur, wave, sm);
    if (!has_next) break;
    cur = nx;
    ca = na;
    q += stride;
    first = false;
  }
  // no load may still be writing this block's LDS when its waves exit
  wait_vm<0>();
}

}  // namespace moe

using namespace moe;

static int gemm7_grid(int max_tiles, int ncol) {
  static int n_cu = 0;
  if (!n_cu) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
      n_cu = n;
    else
      n_cu = 256;
  }
  const int per_xcd_items = (max_tiles + g7::kXcd - 1) / g7::kXcd * ncol;
  const int per_xcd_slots = (n_cu * g7::kBlocksPerCu + g7::kXcd - 1) / g7::kXcd;
  return g7::kXcd * (per_xcd_items < per_xcd_slots ? per_xcd_items : per_xcd_slots);
}

bool moe_gemm7_down_supports(const void* w_down, size_t expert_stride, int H, int I) {
  // 16-byte units of a slab start on 16-byte boundaries only if the expert base, the expert
  // stride and the slab stride (256 rows x 210 I / 256 bytes) are multiples of 16; H % 8 == 0
  // makes the tensor's last super-block end its unit (no unit reaches past the tensor)
  return H % g7::kBN == 0 && H % 8 == 0 && I % 256 == 0 && I >= 256 &&
         reinterpret_cast<uintptr_t>(w_down) % 16 == 0 && expert_stride % 16 == 0 &&
         expert_stride == (size_t)H * (I / 256) * g7::kSBB;
}

int moe_launch_gemm7_down(const uint16_t* S, const void* w_down, size_t expert_stride,
                          const int32_t* tiles, int max_tiles, const int32_t* offsets, int H, int I,
                          void* y, int y16, hipStream_t st) {
  if (!moe_gemm7_down_supports(w_down, expert_stride, H, I))
    return moe_set_error(MOE_E_UNSUPPORTED,
                         "gemm7 down needs H %% 256 == 0, I %% 256 == 0, a 16-byte aligned Q6_K tensor");
  const dim3 grid(gemm7_grid(max_tiles, H / g7::kBN));
  if (y16)
    hipLaunchKernelGGL(k_gemm7_down<true>, grid, dim3(256), 0, st, S, reinterpret_cast<const uint8_t*>(w_down),
                       expert_stride, tiles, offsets, H, I, y);
  else
    hipLaunchKernelGGL(k_gemm7_down<false>, grid, dim3(256), 0, st, S, reinterpret_cast<const uint8_t*>(w_down),
                       expert_stride, tiles, offsets, H, I, y);
  return moe_check_launch("gemm7_down");
}
