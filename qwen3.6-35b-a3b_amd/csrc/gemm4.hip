// Prefill-path grouped GEMM for Q4_K experts with the weight decode in the MFMA waves
// (gfx950, v_mfma_f32_32x32x16_f16, f32 accumulation).
//
// Work: one tile of up to 160 sorted (token, slot) rows of one expert (k_build_tiles, 160-row
// tiles) times one 256-row weight slab per block (gate_up: 128 gate + the matching 128 up rows;
// down: 256 rows), tiles dealt to XCDs so the slabs of one tile share its activation rows in L2.
// Block = 8 waves:
//   producers (waves 4..7) only move bytes. Raw Q4_K super-blocks (256 K, 144 B per row) go to an
//     LDS ring of two super-blocks, nine lanes per row so a load instruction covers seven whole
//     rows; f16 activation rows go to an LDS ring of four 64-wide K steps (eight lanes per
//     128-byte row segment, 16-byte chunks XOR-swizzled by row so fragment reads spread over
//     the banks). Both are requested four steps / one super-block ahead in registers.
//   consumers (waves 0..3) read their two 32-row weight groups' raw nibbles and scales from LDS,
//     decode them in registers straight into MFMA B fragments, and run the MFMAs; each owns all
//     160 rows x (32 gate + 32 up) columns (gate_up) or 64 columns (down). The decode is VALU
//     work that issues while the wave's earlier MFMAs execute.
// One barrier per K step hands the rings over. The decode arithmetic and the k order of every
// MFMA equal gemm3.hip's (q * f16(d sc) + f16(-dmin m) on the f16 mantissa trick), so both give
// the same bits.
#include "common.h"
#include "moe_internal.h"

namespace moe {

typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

namespace g4 {

constexpr int kBM = MOE_GEMM3_BM;       // 160 activation rows per tile
constexpr int kMG = kBM / 32;           // MFMA row groups
constexpr int kBN = 256;                // weight rows per block
constexpr int kSBB = 144;               // bytes per Q4_K super-block row (256 K)
constexpr int kAR = 4;                  // activation ring depth (K steps of 64)
constexpr int kXcd = 8;
constexpr int kChunks = kBN * kSBB / 16 / 256;   // 9 raw 16-byte chunks per producer thread

struct Smem {
  uint8_t B[2][kBN * kSBB];             // 2 x 36 KB raw super-blocks
  uint16_t A[kAR][kBM * 64];            // 4 x 20 KB f16, chunk c of row r at c ^ (r & 7)
};

__device__ __forceinline__ f32x16_t mfma(uint4 a, uint4 b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                               __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

__device__ __forceinline__ uint32_t and_or_s(uint32_t p, uint32_t mask, uint32_t magic) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(p), "s"(mask), "v"(magic));
  return r;
}

// 2 nibbles (bytes of w at positions sel) -> f16x2, scale applied: a low nibble under the f16
// 0x6400 (1024) gives 1024 + q, a high nibble left at bits 4-7 under 0x5400 (64, ulp 1/16) gives
// 64 + q; one packed subtract leaves q exactly and one packed FMA gives q * ds + ndm.
template <bool HIGH>
__device__ __forceinline__ uint32_t q4_pair(uint32_t w, uint32_t sel, f16x2_t ds, f16x2_t ndm) {
  const uint32_t p = __builtin_amdgcn_perm(0u, w, sel);
  const uint32_t magic = HIGH ? and_or_s(p, 0x00F000F0u, 0x54005400u)
                              : and_or_s(p, 0x000F000Fu, 0x64006400u);
  const _Float16 off = HIGH ? (_Float16)64.0f : (_Float16)1024.0f;
  const f16x2_t q = __builtin_bit_cast(f16x2_t, magic) - (f16x2_t){off, off};
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(q, ds, ndm));
}

// 8 bytes of nibbles (w0, w1) -> the 8 f16 of one B fragment (low or high nibbles, k order)
template <bool HIGH>
__device__ __forceinline__ uint4 q4_frag(uint32_t w0, uint32_t w1, f16x2_t ds, f16x2_t ndm) {
  return make_uint4(q4_pair<HIGH>(w0, 0x0C010C00u, ds, ndm), q4_pair<HIGH>(w0, 0x0C030C02u, ds, ndm),
                    q4_pair<HIGH>(w1, 0x0C010C00u, ds, ndm), q4_pair<HIGH>(w1, 0x0C030C02u, ds, ndm));
}

// scale and negated min of sub-block j of a super-block header as f16 pairs (get_scale_min_k4,
// tools/gguf_reader.py:165-175; d * sc and dmin * m rounded to f16 once, as the LDS decode does)
__device__ __forceinline__ void q4_scales(uint4 hdr, int j, f16x2_t& ds, f16x2_t& ndm) {
  uint32_t sc, m;
  q4k_scale_min(hdr.y, hdr.z, hdr.w, j, sc, m);
  const _Float16 d = (_Float16)(f16_to_f32(hdr.x & 0xFFFFu) * (float)sc);
  const _Float16 n = (_Float16)(-(f16_to_f32(hdr.x >> 16) * (float)m));
  ds = (f16x2_t){d, d};
  ndm = (f16x2_t){n, n};
}

__device__ __forceinline__ int tile_rows(const int32_t* tiles, const int32_t* offsets, int ncol,
                                         int& e, int& m0, int& mend, int& col) {
  const int count = tiles[0];
  const int per = (count + kXcd - 1) / kXcd;
  const int xcd = blockIdx.x % kXcd, slot = blockIdx.x / kXcd;
  const int tl = slot / ncol;
  col = slot % ncol;
  const int tile = xcd * per + tl;
  if (tl >= per || tile >= count) return 0;
  e = tiles[1 + 2 * tile];
  m0 = tiles[2 + 2 * tile];
  mend = min(m0 + kBM, offsets[e + 1]);
  return 1;
}

// ------------------------------------------------------------------------------- producer --
// Thread p (0..255). Raw chunk q = 256 i + p (i < 9) of a super-block slab is row q / 9, bytes
// 16 (q % 9) .. +16 of that row's super-block; it lands at LDS byte 16 q. Activation chunk
// p & 7 of rows (p >> 3) + 32 i (i < 5) of a K step lands at chunk (p & 7) ^ (row & 7).
struct Producer {
  const uint8_t* wsrc[kChunks];         // each raw chunk's bytes in super-block 0 of its row
  const uint16_t* arow[kMG];            // activation row starts
  uint4 braw[kChunks];                  // one super-block's chunks in flight
  uint4 areg[kAR][kMG];                 // kAR K steps of activation chunks in flight
  int p;

  __device__ __forceinline__ void load_b(int sb, int i0, int i1) {
#pragma unroll
    for (int i = 0; i < kChunks; ++i)
      if (i >= i0 && i < i1) braw[i] = *reinterpret_cast<const uint4*>(wsrc[i] + sb * kSBB);
  }
  __device__ __forceinline__ void store_b(uint8_t* Bs, int i0, int i1) const {
#pragma unroll
    for (int i = 0; i < kChunks; ++i)
      if (i >= i0 && i < i1) *reinterpret_cast<uint4*>(Bs + 16 * (256 * i + p)) = braw[i];
  }
  template <int R>
  __device__ __forceinline__ void load_a(int ks) {
#pragma unroll
    for (int i = 0; i < kMG; ++i)
      areg[R][i] = *reinterpret_cast<const uint4*>(arow[i] + 64 * ks + 8 * (p & 7));
  }
  template <int R>
  __device__ __forceinline__ void store_a(uint16_t* As) const {
#pragma unroll
    for (int i = 0; i < kMG; ++i) {
      const int row = (p >> 3) + 32 * i;
      *reinterpret_cast<uint4*>(As + row * 64 + 8 * ((p & 7) ^ (row & 7))) = areg[R][i];
    }
  }
};

// chunks of the next super-block stored at step s of the current one (9 = 3 + 2 + 2 + 2)
__device__ __forceinline__ int chunk_lo(int s) { return s == 0 ? 0 : 1 + 2 * s; }
__device__ __forceinline__ int chunk_hi(int s) { return 3 + 2 * s; }

// Step ks = 4 sb + s: consumers read A[s] and B[sb & 1]. The producer stores step ks + 3's
// activations into A[(s + 3) % 4] (set (s + 3) % 4, then reloads it with step ks + 7) and part s
// of super-block sb + 1 into B[(sb + 1) & 1] (then reloads those registers from sb + 2).
template <int S>
__device__ __forceinline__ void pstep(Producer& pr, int sb, int nk, int nsb, Smem& sm) {
  const int ks = 4 * sb + S;
  pr.store_a<(S + 3) % 4>(sm.A[(S + 3) % 4]);
  pr.store_b(sm.B[(sb + 1) & 1], chunk_lo(S), chunk_hi(S));
  pr.load_a<(S + 3) % 4>(min(ks + 7, nk - 1));
  pr.load_b(min(sb + 2, nsb - 1), chunk_lo(S), chunk_hi(S));
  __syncthreads();
}

__device__ __forceinline__ void produce(Producer& pr, int nk, Smem& sm) {
  const int nsb = nk / 4;
  // prologue: super-block 0 and steps 0..2 in LDS; super-block 1 and steps 3..6 in registers
  pr.load_b(0, 0, kChunks);
  pr.load_a<0>(0);
  pr.load_a<1>(min(1, nk - 1));
  pr.load_a<2>(min(2, nk - 1));
  pr.store_b(sm.B[0], 0, kChunks);
  pr.store_a<0>(sm.A[0]);
  pr.store_a<1>(sm.A[1]);
  pr.store_a<2>(sm.A[2]);
  pr.load_b(min(1, nsb - 1), 0, kChunks);
  pr.load_a<3>(min(3, nk - 1));
  pr.load_a<0>(min(4, nk - 1));
  pr.load_a<1>(min(5, nk - 1));
  pr.load_a<2>(min(6, nk - 1));
  __syncthreads();
  for (int sb = 0; sb < nsb; ++sb) {
    pstep<0>(pr, sb, nk, nsb, sm);
    pstep<1>(pr, sb, nk, nsb, sm);
    pstep<2>(pr, sb, nk, nsb, sm);
    pstep<3>(pr, sb, nk, nsb, sm);
  }
}

// ------------------------------------------------------------------------------- consumer --
// Consumer lane l: weight rows n0 + l % 32 (group 0) and n1 + l % 32 (group 1) of the slab, half
// h = l / 32 of every 16-wide MFMA k substep. In step s of a super-block the lane needs bytes
// [8h, 8h+8) and [16 + 8h, +8) of the row's 32-byte nibble group s: substep 0 = low nibbles of the
// first, 1 = low of the second, 2 = high of the first, 3 = high of the second (elements
// 16 ss + 8h .. +8, the natural k order).
template <int NG>
__device__ __forceinline__ void consume(int nk, int n0, int n1, Smem& sm, f32x16_t (&acc)[kMG][2]) {
  const int lane = threadIdx.x & 63;
  const int h = lane >> 5, r = lane & 31;
  const int nsb = nk / 4;
  __syncthreads();
  for (int sb = 0; sb < nsb; ++sb) {
    const uint8_t* Bs = sm.B[sb & 1];
    const uint8_t* rg0 = Bs + (n0 + r) * kSBB;
    const uint8_t* rg1 = Bs + (n1 + r) * kSBB;
    const uint4 hdr0 = *reinterpret_cast<const uint4*>(rg0);
    const uint4 hdr1 = *reinterpret_cast<const uint4*>(rg1);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const uint2 a0 = *reinterpret_cast<const uint2*>(rg0 + 16 + 32 * s + 8 * h);
      const uint2 b0 = *reinterpret_cast<const uint2*>(rg0 + 32 + 32 * s + 8 * h);
      const uint2 a1 = *reinterpret_cast<const uint2*>(rg1 + 16 + 32 * s + 8 * h);
      const uint2 b1 = *reinterpret_cast<const uint2*>(rg1 + 32 + 32 * s + 8 * h);
      f16x2_t ds0l, nd0l, ds0h, nd0h, ds1l, nd1l, ds1h, nd1h;
      q4_scales(hdr0, 2 * s, ds0l, nd0l);
      q4_scales(hdr0, 2 * s + 1, ds0h, nd0h);
      q4_scales(hdr1, 2 * s, ds1l, nd1l);
      q4_scales(hdr1, 2 * s + 1, ds1h, nd1h);
      const uint16_t* As = sm.A[s];
      // software pipeline over the 4 substeps: substep ss + 1's A fragments are requested and its
      // B fragments decoded while substep ss's MFMAs run
      auto decode = [&](int ss, uint4& bg, uint4& bu) {
        if (ss == 0) { bg = q4_frag<false>(a0.x, a0.y, ds0l, nd0l); bu = q4_frag<false>(a1.x, a1.y, ds1l, nd1l); }
        else if (ss == 1) { bg = q4_frag<false>(b0.x, b0.y, ds0l, nd0l); bu = q4_frag<false>(b1.x, b1.y, ds1l, nd1l); }
        else if (ss == 2) { bg = q4_frag<true>(a0.x, a0.y, ds0h, nd0h); bu = q4_frag<true>(a1.x, a1.y, ds1h, nd1h); }
        else { bg = q4_frag<true>(b0.x, b0.y, ds0h, nd0h); bu = q4_frag<true>(b1.x, b1.y, ds1h, nd1h); }
      };
      auto afrag = [&](int ss, uint4 (&a)[NG]) {
#pragma unroll
        for (int mg = 0; mg < NG; ++mg) {
          const int row = 32 * mg + r;
          a[mg] = *reinterpret_cast<const uint4*>(As + row * 64 + 8 * ((2 * ss + h) ^ (row & 7)));
        }
      };
      uint4 ac[NG], an[NG], bgc, buc, bgn, bun;
      afrag(0, ac);
      decode(0, bgc, buc);
#pragma unroll
      for (int ss = 0; ss < 4; ++ss) {
        if (ss < 3) {
          afrag(ss + 1, an);
          decode(ss + 1, bgn, bun);
        }
#pragma unroll
        for (int mg = 0; mg < NG; ++mg) {
          acc[mg][0] = mfma(ac[mg], bgc, acc[mg][0]);
          acc[mg][1] = mfma(ac[mg], buc, acc[mg][1]);
        }
        if (ss < 3) {
#pragma unroll
          for (int mg = 0; mg < NG; ++mg) ac[mg] = an[mg];
          bgc = bgn;
          buc = bun;
        }
      }
      __syncthreads();
    }
  }
}

__device__ __forceinline__ void consume_n(int ng, int nk, int n0, int n1, Smem& sm,
                                          f32x16_t (&acc)[kMG][2]) {
  if (ng >= 5) consume<5>(nk, n0, n1, sm, acc);
  else if (ng == 4) consume<4>(nk, n0, n1, sm, acc);
  else if (ng == 3) consume<3>(nk, n0, n1, sm, acc);
  else if (ng == 2) consume<2>(nk, n0, n1, sm, acc);
  else consume<1>(nk, n0, n1, sm, acc);
}

}  // namespace g4

// ----------------------------------------------------------------------------------- gate/up --
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_gemm4_gateup(
    const uint16_t* __restrict__ x16, const uint8_t* __restrict__ wg, const uint8_t* __restrict__ wu,
    size_t estride, const int32_t* __restrict__ tiles, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ sorted_pairs, int K, int H, int I, uint16_t* __restrict__ S) {
  using namespace g4;
  __shared__ __attribute__((aligned(16))) Smem sm;
  int e, m0, mend, col;
  if (!tile_rows(tiles, offsets, I / 128, e, m0, mend, col)) return;
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int nk = H / 64;
  if (wave >= 4) {
    Producer pr;
    pr.p = t - 256;
    const size_t rowb = (size_t)(H / 256) * kSBB;
#pragma unroll
    for (int i = 0; i < kChunks; ++i) {
      const int q = 256 * i + pr.p, row = q / 9;
      pr.wsrc[i] = (row < 128 ? wg : wu) + (size_t)e * estride + (size_t)(col * 128 + (row & 127)) * rowb +
                   16 * (q % 9);
    }
#pragma unroll
    for (int i = 0; i < kMG; ++i) {
      const int m = min(m0 + (pr.p >> 3) + 32 * i, mend - 1);
      pr.arow[i] = x16 + (size_t)(sorted_pairs[m] / K) * H;
    }
    produce(pr, nk, sm);
    return;
  }
  f32x16_t acc[kMG][2];
#pragma unroll
  for (int mg = 0; mg < kMG; ++mg) { acc[mg][0] = (f32x16_t){}; acc[mg][1] = (f32x16_t){}; }
  const int ng = __builtin_amdgcn_readfirstlane((mend - m0 + 31) >> 5);
  consume_n(ng, nk, 32 * wave, 128 + 32 * wave, sm, acc);
  const int n = col * 128 + 32 * wave + (lane & 31), h = lane >> 5;
#pragma unroll
  for (int mg = 0; mg < kMG; ++mg) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int mm = m0 + 32 * mg + 8 * (r >> 2) + 4 * h + (r & 3);
      if (mm < mend) {
        float v = silu_f32(acc[mg][0][r]) * acc[mg][1][r];
        v = fminf(fmaxf(v, -65504.0f), 65504.0f);
        S[(size_t)mm * I + n] = __builtin_bit_cast(uint16_t, (_Float16)v);
      }
    }
  }
}

// -------------------------------------------------------------------------------------- down --
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_gemm4_down(
    const uint16_t* __restrict__ S, const uint8_t* __restrict__ wd, size_t estride,
    const int32_t* __restrict__ tiles, const int32_t* __restrict__ offsets, int H, int I,
    float* __restrict__ y) {
  using namespace g4;
  __shared__ __attribute__((aligned(16))) Smem sm;
  int e, m0, mend, col;
  if (!tile_rows(tiles, offsets, H / kBN, e, m0, mend, col)) return;
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int nk = I / 64;
  if (wave >= 4) {
    Producer pr;
    pr.p = t - 256;
    const size_t rowb = (size_t)(I / 256) * kSBB;
#pragma unroll
    for (int i = 0; i < kChunks; ++i) {
      const int q = 256 * i + pr.p, row = q / 9;
      pr.wsrc[i] = wd + (size_t)e * estride + (size_t)(col * kBN + row) * rowb + 16 * (q % 9);
    }
#pragma unroll
    for (int i = 0; i < kMG; ++i) pr.arow[i] = S + (size_t)min(m0 + (pr.p >> 3) + 32 * i, mend - 1) * I;
    produce(pr, nk, sm);
    return;
  }
  f32x16_t acc[kMG][2];
#pragma unroll
  for (int mg = 0; mg < kMG; ++mg) { acc[mg][0] = (f32x16_t){}; acc[mg][1] = (f32x16_t){}; }
  const int ng = __builtin_amdgcn_readfirstlane((mend - m0 + 31) >> 5);
  consume_n(ng, nk, 64 * wave, 64 * wave + 32, sm, acc);
  const int nb = col * kBN + 64 * wave + (lane & 31), h = lane >> 5;
#pragma unroll
  for (int mg = 0; mg < kMG; ++mg) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int mm = m0 + 32 * mg + 8 * (r >> 2) + 4 * h + (r & 3);
      if (mm < mend) {
        y[(size_t)mm * H + nb] = acc[mg][0][r];
        y[(size_t)mm * H + nb + 32] = acc[mg][1][r];
      }
    }
  }
}

}  // namespace moe

using namespace moe;

int moe_launch_gemm4_gateup(const uint16_t* x16, const void* w_gate, const void* w_up,
                            size_t expert_stride, const int32_t* tiles, int max_tiles,
                            const int32_t* offsets, const int32_t* sorted_pairs, int K, int H,
                            int I, uint16_t* S, hipStream_t st) {
  if (H % 256 || I % 128)
    return moe_set_error(MOE_E_UNSUPPORTED, "gemm4 gate_up needs H %% 256 == 0, I %% 128 == 0");
  const dim3 grid(g4::kXcd * ((max_tiles + g4::kXcd - 1) / g4::kXcd) * (I / 128));
  hipLaunchKernelGGL(k_gemm4_gateup, grid, dim3(512), 0, st, x16, reinterpret_cast<const uint8_t*>(w_gate),
                     reinterpret_cast<const uint8_t*>(w_up), expert_stride, tiles, offsets, sorted_pairs,
                     K, H, I, S);
  return moe_check_launch("gemm4_gateup");
}

int moe_launch_gemm4_down(const uint16_t* S, const void* w_down, size_t expert_stride,
                          const int32_t* tiles, int max_tiles, const int32_t* offsets, int H, int I,
                          float* y, hipStream_t st) {
  if (H % g4::kBN || I % 256)
    return moe_set_error(MOE_E_UNSUPPORTED, "gemm4 down needs H %% 256 == 0, I %% 256 == 0");
  const dim3 grid(g4::kXcd * ((max_tiles + g4::kXcd - 1) / g4::kXcd) * (H / g4::kBN));
  hipLaunchKernelGGL(k_gemm4_down, grid, dim3(512), 0, st, S, reinterpret_cast<const uint8_t*>(w_down),
                     expert_stride, tiles, offsets, H, I, y);
  return moe_check_launch("gemm4_down");
}
