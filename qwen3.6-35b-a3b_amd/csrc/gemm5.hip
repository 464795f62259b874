// Prefill-path shared expert: dense GEMMs over all T token rows with bf16 weights (gfx950, f32
// accumulation): gate/up with SiLU(gate) * up fused into the epilogue (f16 rows, the down GEMM's
// operand), then down (f32 rows).
//
// Work: one block per (128-row token tile, 256-row weight slab) item (gate_up: 128 gate + the
// matching 128 up rows; down: 256 rows); the slabs of a tile are adjacent block indices so they
// run side by side and share the tile's rows in L2. Block = 8 waves (two per SIMD) and 144 KB of
// LDS. Per 64-wide K step every wave issues 2 activation and 4 weight direct global->LDS loads
// (16 bytes per lane) two steps ahead into 3-deep rings, and waits for its own loads with an
// explicit vmcnt count before the step's barrier:
//   A[3]: activations, 128 rows x 128 B, 16-byte chunk c of row m at chunk c ^ swz(m);
//   B[3]: bf16 weights, 256 rows x 128 B, the same swizzle by weight row;
// swz(m) = (m ^ (m >> 1)) & 7, so the fragment reads of 8 or 16 lanes hit distinct banks under
// either a 32- or a 64-bank layout. Wave w owns token rows 64 (w / 4) .. + 63 (two MFMA row
// groups) x (32 gate + 32 up) columns 32 (w % 4) .. of the slab (gate_up) or 64 columns 64 (w % 4)
// .. (down).
// Operands: gate/up on bf16 activations runs v_mfma_f32_32x32x16_bf16 on the rows and weights as
// they are (every product exact, f32 sums). Otherwise (f16 activations: converted f32 rows, or
// the f16 SiLU rows of down) v_mfma_f32_32x32x16_f16 with the weight fragments converted bf16 ->
// f16 in registers: exact for |w| >= 2^-17 (and up to 65504); below, the f16 subnormal rounding
// moves a weight by at most 2^-25. Results leave through raw buffer stores clipped at row T.
#include "common.h"
#include "moe_internal.h"
#include "lds_dma.h"
#include "shared_small.h"

namespace moe {

typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

namespace g5 {

using dma::lds_addr;
using dma::opaque;
using dma::wait_vm;

constexpr int kBM = 128;                // token rows per item
constexpr int kBN = 256;                // weight rows per item
constexpr int kBK = 64;                 // K per step
constexpr int kR = 3;                   // ring depth (steps)
constexpr int kWaves = 8;
constexpr int kAI = kBM * 8 / 64 / kWaves;   // A loads per wave per step (2)
constexpr int kBI = kBN * 8 / 64 / kWaves;   // B loads per wave per step (4)
static_assert(kAI == 2 && kBI == 4, "load split assumes 128 x 256 items");

struct Smem {
  uint8_t A[kR][kBM * 128];
  uint8_t B[kR][kBN * 128];
};
static_assert(sizeof(Smem) <= 160 * 1024, "one block per CU");

__device__ __forceinline__ int swz(int m) { return (m ^ (m >> 1)) & 7; }

using shs::bf16x8_to_f16;
using shs::mfma;

// One item: rows [m0, m0 + rows) of A (row length K elements, 2 bytes each) against the 256
// weight rows n (n < 128: base g, else base u, each + (n & 127) * K * 2). Lane l of wave w: token
// rows 64 (w / 4) + 32 mg + ..., weight rows n0 + l % 32 (group 0) and n1 + l % 32 (group 1), half
// h = l / 32 of every 16-wide MFMA k substep. BF: bf16 A on the bf16 MFMA; else f16 A with the
// weights converted.
template <bool BF, class Epi>
__device__ __forceinline__ void item(const uint8_t* abase, int rows, int K, const uint8_t* g,
                                     const uint8_t* u, int n0, int n1, Smem& sm, const Epi& epi) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int h = lane >> 5, r = lane & 31;
  const int rh = wave >> 2;
  const int nk = K / kBK;
  // load geometry: load j of wave w covers the slot's 16-byte units 64 (w + 8 j) + l, unit u =
  // row u >> 3, physical chunk u & 7 (logical chunk (u & 7) ^ swz(row))
  uint32_t aoff[kAI], boff[kBI];
  const uint8_t* bb[kBI];
#pragma unroll
  for (int j = 0; j < kAI; ++j) {
    const int uu = 64 * (wave + kWaves * j) + lane, m = uu >> 3;
    aoff[j] = (uint32_t)min(m, rows - 1) * (uint32_t)K * 2u + 16u * (uint32_t)((uu & 7) ^ swz(m));
  }
#pragma unroll
  for (int j = 0; j < kBI; ++j) {
    const int uu = 64 * (wave + kWaves * j) + lane, n = uu >> 3;
    boff[j] = (uint32_t)(n & 127) * (uint32_t)K * 2u + 16u * (uint32_t)((uu & 7) ^ swz(n));
    bb[j] = j < 2 ? g : u;   // rows 0..127 from g, 128..255 from u
  }
  const uint32_t la = lds_addr(sm.A[0]) + 1024 * wave, lb = lds_addr(sm.B[0]) + 1024 * wave;
  auto issue = [&](int slot, int ks) {
#pragma unroll
    for (int j = 0; j < kAI; ++j)
      dma::load16(aoff[j], abase + (size_t)ks * 128, la + slot * (kBM * 128) + j * 8192);
#pragma unroll
    for (int j = 0; j < kBI; ++j)
      dma::load16(boff[j], bb[j] + (size_t)ks * 128, lb + slot * (kBN * 128) + j * 8192);
  };
  f32x16_t acc[2][2];
#pragma unroll
  for (int mg = 0; mg < 2; ++mg) { acc[mg][0] = (f32x16_t){}; acc[mg][1] = (f32x16_t){}; }
  // per-lane LDS byte offsets of substep ss's fragments (rows 64 rh + 32 mg + r, n0 + r, n1 + r:
  // the swizzle of each is swz(r), the row bases being multiples of 32)
  int ao[4], bo0[4], bo1[4];
#pragma unroll
  for (int ss = 0; ss < 4; ++ss) {
    const int c = 16 * ((2 * ss + h) ^ swz(r));
    ao[ss] = 128 * (64 * rh + r) + c;
    bo0[ss] = 128 * (n0 + r) + c;
    bo1[ss] = 128 * (n1 + r) + c;
  }
  issue(0, 0);
  issue(1, min(1, nk - 1));
  wait_vm<kAI + kBI>();
  int slot = 0;
  for (int ks = 0; ks < nk; ++ks) {
    // this wave's loads of step ks were issued two steps ago; one step's loads came after them
    if (ks > 0) wait_vm<kAI + kBI>();
    __syncthreads();
    // into the slot step ks - 1 used (clamped repeats past the end land in slots nothing reads)
    issue(slot == 0 ? 2 : slot - 1, min(ks + 2, nk - 1));
    const uint8_t* As = sm.A[slot];
    const uint8_t* Bs = sm.B[slot];
#pragma unroll
    for (int ss = 0; ss < 4; ++ss) {
      const uint4 a0 = *reinterpret_cast<const uint4*>(As + ao[ss]);
      const uint4 a1 = *reinterpret_cast<const uint4*>(As + ao[ss] + 128 * 32);
      uint4 bg = *reinterpret_cast<const uint4*>(Bs + bo0[ss]);
      uint4 bu = *reinterpret_cast<const uint4*>(Bs + bo1[ss]);
      if constexpr (!BF) {
        bg = bf16x8_to_f16(bg);
        bu = bf16x8_to_f16(bu);
      }
      acc[0][0] = mfma<BF>(a0, bg, acc[0][0]);
      acc[0][1] = mfma<BF>(a0, bu, acc[0][1]);
      acc[1][0] = mfma<BF>(a1, bg, acc[1][0]);
      acc[1][1] = mfma<BF>(a1, bu, acc[1][1]);
    }
    slot = slot == 2 ? 0 : slot + 1;
  }
  // no load may still be writing this block's LDS when its waves exit
  wait_vm<0>();
  epi(acc, rh, lane);
}

// gate/up: A [T, H] (bf16 rows when BF, else f16), w_gate / w_up [I_s, H] bf16 -> S [T, I_s] f16
// = SiLU(gate) * up
template <bool BF>
__device__ __forceinline__ void gateup(const uint16_t* __restrict__ a, const uint16_t* __restrict__ wg,
                                       const uint16_t* __restrict__ wu, int T, int H, int Is,
                                       uint16_t* __restrict__ S, Smem& sm) {
  const int ncol = Is / 128;
  const int m0 = (blockIdx.x / ncol) * kBM, col = blockIdx.x % ncol;
  if (m0 >= T) return;
  const int rows = min(kBM, T - m0);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int cq = wave & 3;
  const uint8_t* g = reinterpret_cast<const uint8_t*>(wg + (size_t)col * 128 * H);
  const uint8_t* u = reinterpret_cast<const uint8_t*>(wu + (size_t)col * 128 * H);
  auto epi = [&](const f32x16_t (&acc)[2][2], int rh, int lane) {
    const __amdgpu_buffer_rsrc_t rs = dma::rsrc(S + (size_t)m0 * Is, rows * Is * 2);
    const int rs2 = opaque(Is * 2);
    const int lane_off = ((64 * rh + 4 * (lane >> 5)) * Is + col * 128 + 32 * cq + (lane & 31)) * 2;
#pragma unroll
    for (int mg = 0; mg < 2; ++mg) {
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        const int vo = lane_off + (32 * mg + 8 * rq) * rs2;
#pragma unroll
        for (int r3 = 0; r3 < 4; ++r3) {
          const float gv = acc[mg][0][4 * rq + r3], uv = acc[mg][1][4 * rq + r3];
          float v = gv * __builtin_amdgcn_rcpf(1.0f + __expf(-gv)) * uv;
          v = fminf(fmaxf(v, -65504.0f), 65504.0f);
          __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, (_Float16)v), rs,
                                                vo + r3 * rs2, 0, 0);
        }
      }
    }
  };
  item<BF>(reinterpret_cast<const uint8_t*>(a + (size_t)m0 * H), rows, H, g, u, 32 * cq,
           128 + 32 * cq, sm, epi);
}

}  // namespace g5

template <bool BF>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_gemm5_gateup(
    const uint16_t* __restrict__ a, const uint16_t* __restrict__ wg, const uint16_t* __restrict__ wu,
    int T, int H, int Is, uint16_t* __restrict__ S) {
  __shared__ __attribute__((aligned(16))) g5::Smem sm;
  g5::gateup<BF>(a, wg, wu, T, H, Is, S, sm);
}

// down: S [T, I_s] f16, w_down [H, I_s] bf16 -> y [T, H] f32
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_gemm5_down(
    const uint16_t* __restrict__ S, const uint16_t* __restrict__ wd, int T, int H, int Is,
    float* __restrict__ y) {
  using namespace g5;
  __shared__ __attribute__((aligned(16))) Smem sm;
  const int ncol = H / kBN;
  const int m0 = (blockIdx.x / ncol) * kBM, col = blockIdx.x % ncol;
  if (m0 >= T) return;
  const int rows = min(kBM, T - m0);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int cq = wave & 3;
  const uint8_t* w0 = reinterpret_cast<const uint8_t*>(wd + (size_t)col * kBN * Is);
  const uint8_t* w1 = reinterpret_cast<const uint8_t*>(wd + ((size_t)col * kBN + 128) * Is);
  auto epi = [&](const f32x16_t (&acc)[2][2], int rh, int lane) {
    const __amdgpu_buffer_rsrc_t rs = dma::rsrc(y + (size_t)m0 * H, rows * H * 4);
    const int rs4 = opaque(H * 4);
    const int lane_off = ((64 * rh + 4 * (lane >> 5)) * H + col * kBN + 64 * cq + (lane & 31)) * 4;
#pragma unroll
    for (int mg = 0; mg < 2; ++mg) {
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        const int vo = lane_off + (32 * mg + 8 * rq) * rs4;
#pragma unroll
        for (int r3 = 0; r3 < 4; ++r3) {
          // copied out of the vector first: a bit cast of the vector element itself read element
          // 0 here; the builtin's data operand is an integer (the bits, not the value)
          const float v0 = acc[mg][0][4 * rq + r3], v1 = acc[mg][1][4 * rq + r3];
          __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v0), rs, vo + r3 * rs4, 0, 0);
          __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v1), rs, vo + r3 * rs4 + 128, 0, 0);
        }
      }
    }
  };
  item<false>(reinterpret_cast<const uint8_t*>(S + (size_t)m0 * Is), rows, Is, w0, w1, 64 * cq,
              64 * cq + 32, sm, epi);
}

// ------------------------------------------------------------ small-T shared expert --
// Below a few hundred tokens the 128 x 256 items above leave most CUs idle (T = 64: 4 blocks of
// gate/up, each streaming 1 MB of weights on its own). These launches run shared_small.h's narrow
// slab blocks with 8 waves each. The gate/up launch also computes the scalar gate (one wave per
// token, k_shared_gate's arithmetic) and, when asked, the routed GEMMs' f16 copy of x (k_to_f16's
// conversion), so the small-T shared expert is two launches.

// grid (Is / 16, ceil(T / 64)): S [T, Is] f16 = SiLU(x wg^T) * (x wu^T) from x (f32 or bf16);
// gate_prob [T] = sigmoid(x . wsg) (NULL: skipped); x16 [T, H] = f16(x) (NULL: skipped)
template <int XDT>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_gemm5s_gateup(
    const void* __restrict__ x, const uint16_t* __restrict__ wg, const uint16_t* __restrict__ wu,
    const void* __restrict__ wsg, int gdt, int T, int H, int Is, uint16_t* __restrict__ S,
    float* __restrict__ gate_prob, uint16_t* __restrict__ x16) {
  __shared__ float red[shs::red_floats<8>()];
  const int nblk = gridDim.x * gridDim.y;
  const int bid = blockIdx.y * gridDim.x + blockIdx.x;
  if (x16) {
    // k_to_f16's conversion, 8 elements per unit, spread over the whole grid
    const size_t n8 = (size_t)T * H / 8;
    for (size_t i = (size_t)bid * 512 + threadIdx.x; i < n8; i += (size_t)nblk * 512) {
      uint4 o;
      if constexpr (XDT == MOE_DT_BF16) {
        const uint4 v = reinterpret_cast<const uint4*>(x)[i];
        o = make_uint4(shs::f16x2_sat(bf16_to_f32(v.x & 0xFFFFu), bf16_to_f32(v.x >> 16)),
                       shs::f16x2_sat(bf16_to_f32(v.y & 0xFFFFu), bf16_to_f32(v.y >> 16)),
                       shs::f16x2_sat(bf16_to_f32(v.z & 0xFFFFu), bf16_to_f32(v.z >> 16)),
                       shs::f16x2_sat(bf16_to_f32(v.w & 0xFFFFu), bf16_to_f32(v.w >> 16)));
      } else {
        const float4 a = reinterpret_cast<const float4*>(x)[2 * i];
        const float4 b = reinterpret_cast<const float4*>(x)[2 * i + 1];
        o = make_uint4(shs::f16x2_sat(a.x, a.y), shs::f16x2_sat(a.z, a.w), shs::f16x2_sat(b.x, b.y),
                       shs::f16x2_sat(b.z, b.w));
      }
      reinterpret_cast<uint4*>(x16)[i] = o;
    }
  }
  shs::gateup_tile<XDT, 8>(x, wg, wu, T, H, Is, blockIdx.x, blockIdx.y * shs::kBM, S, red);
  if (gate_prob) shs::gate_rows<XDT>(x, wsg, gdt, T, H, gate_prob, bid * 8 + (int)(threadIdx.x >> 6), nblk * 8);
}

// grid (H / 32, ceil(T / 64)): y [T, H] f32 = S [T, Is] f16 . w_down^T (w_down [H, Is] bf16)
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_gemm5s_down(
    const uint16_t* __restrict__ S, const uint16_t* __restrict__ wd, int T, int H, int Is,
    float* __restrict__ y) {
  __shared__ float red[shs::red_floats<8>()];
  shs::down_tile<8>(S, wd, T, H, Is, blockIdx.x, blockIdx.y * shs::kBM, y, red);
}

}  // namespace moe

using namespace moe;

bool moe_gemm5s_supports(int H, int Is) {
  // K per wave a whole number of 64-wide chunks; the scalar gate's 512-wide passes
  return H % 512 == 0 && Is % 512 == 0;
}

int moe_launch_gemm5s_gateup(const void* x, int x_dtype, const void* w_gate, const void* w_up,
                             const void* wsg, int gate_dtype, int T, int H, int Is, uint16_t* S,
                             float* gate_prob, uint16_t* x16, hipStream_t st) {
  if (!moe_gemm5s_supports(H, Is))
    return moe_set_error(MOE_E_UNSUPPORTED, "small-T shared gate_up needs H %% 512 == 0, I_s %% 512 == 0");
  const dim3 grid(Is / 16, (T + shs::kBM - 1) / shs::kBM);
  const uint16_t* g = reinterpret_cast<const uint16_t*>(w_gate);
  const uint16_t* u = reinterpret_cast<const uint16_t*>(w_up);
  if (x_dtype == MOE_DT_BF16)
    hipLaunchKernelGGL(k_gemm5s_gateup<MOE_DT_BF16>, grid, dim3(512), 0, st, x, g, u, wsg, gate_dtype, T, H,
                       Is, S, gate_prob, x16);
  else
    hipLaunchKernelGGL(k_gemm5s_gateup<MOE_DT_F32>, grid, dim3(512), 0, st, x, g, u, wsg, gate_dtype, T, H,
                       Is, S, gate_prob, x16);
  return moe_check_launch("gemm5s_gateup");
}

int moe_launch_gemm5s_down(const uint16_t* S, const void* w_down, int T, int H, int Is, float* y,
                           hipStream_t st) {
  if (!moe_gemm5s_supports(H, Is))
    return moe_set_error(MOE_E_UNSUPPORTED, "small-T shared down needs H %% 512 == 0, I_s %% 512 == 0");
  const dim3 grid(H / 32, (T + shs::kBM - 1) / shs::kBM);
  hipLaunchKernelGGL(k_gemm5s_down, grid, dim3(512), 0, st, S, reinterpret_cast<const uint16_t*>(w_down), T,
                     H, Is, y);
  return moe_check_launch("gemm5s_down");
}

bool moe_gemm5_supports(int H, int Is) {
  return H % 256 == 0 && Is % 128 == 0 && Is % g5::kBK == 0 && Is >= 64;
}

int moe_launch_gemm5_gateup(const void* a, int a_bf16, const void* w_gate, const void* w_up, int T,
                            int H, int Is, uint16_t* S, hipStream_t st) {
  if (!moe_gemm5_supports(H, Is))
    return moe_set_error(MOE_E_UNSUPPORTED, "gemm5 gate_up needs H %% 256 == 0, I_s %% 128 == 0");
  if ((size_t)g5::kBM * Is * 4 > 0x7FFFFFFFu || (size_t)g5::kBM * H * 4 > 0x7FFFFFFFu)
    return moe_set_error(MOE_E_UNSUPPORTED, "gemm5: a tile's rows exceed 31-bit buffer offsets");
  const dim3 grid(((T + g5::kBM - 1) / g5::kBM) * (Is / 128));
  const uint16_t* ap = reinterpret_cast<const uint16_t*>(a);
  const uint16_t* g = reinterpret_cast<const uint16_t*>(w_gate);
  const uint16_t* u = reinterpret_cast<const uint16_t*>(w_up);
  if (a_bf16)
    hipLaunchKernelGGL(k_gemm5_gateup<true>, grid, dim3(512), 0, st, ap, g, u, T, H, Is, S);
  else
    hipLaunchKernelGGL(k_gemm5_gateup<false>, grid, dim3(512), 0, st, ap, g, u, T, H, Is, S);
  return moe_check_launch("gemm5_gateup");
}

int moe_launch_gemm5_down(const uint16_t* S, const void* w_down, int T, int H, int Is, float* y,
                          hipStream_t st) {
  if (!moe_gemm5_supports(H, Is))
    return moe_set_error(MOE_E_UNSUPPORTED, "gemm5 down needs H %% 256 == 0, I_s %% 128 == 0");
  const dim3 grid(((T + g5::kBM - 1) / g5::kBM) * (H / g5::kBN));
  hipLaunchKernelGGL(k_gemm5_down, grid, dim3(512), 0, st, S, reinterpret_cast<const uint16_t*>(w_down),
                     T, H, Is, y);
  return moe_check_launch("gemm5_down");
}
