// Prefill-path grouped GEMM on MFMA (gfx950 v_mfma_f32_32x32x16_{f16,bf16}): weight tiles are
// decoded from Q4_K / Q6_K super-blocks (or converted from bf16) into LDS as 16-bit MFMA operands
// and contracted against 16-bit activation tiles with f32 accumulation (speccheck/moe_ref.py:
// 367-451 semantics; the decode arithmetic is the exact f32 one of dequant.hip, rounded once to
// the operand type).
//
// Operand type. f16 (the default, MOE_PATH_MFMA) and bf16 (MOE_PATH_MFMA_BF16) run at the same
// dense MFMA rate on gfx950. f16 keeps 11 significant bits against bf16's 8, so rounding the
// decoded weights and the SwiGLU intermediate s costs 8x less; with bf16 operands the block output
// lands at ~3e-3 max-abs from the f32 oracle, with f16 well inside the 2e-3 bar. f16 covers
// |v| <= 65504; s is saturated to that range rather than overflowing.
//
// Work list: one 64-row tile of sorted pairs of one expert per blockIdx.y (built on the device by
// k_build_tiles, so no routing value reaches the host); blockIdx.x walks 64-column output tiles.
// gate_up: B = 64 gate rows + the matching 64 up rows (gate first, spec §11.4); the epilogue
// writes s = silu(gate) * up as a 16-bit operand. down: B = 64 down rows; the epilogue writes y
// in f32. Block = 4 waves in a 2x2 arrangement, each wave one 32x32 output tile per matrix.
#include "common.h"
#include "moe_internal.h"

namespace moe {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kBK = 64;
constexpr int kLdsPad = 72;   // row stride in 16-bit elements (144 B, keeps 16-B alignment)
constexpr int OP_F16 = 0, OP_BF16 = 1;

__device__ __forceinline__ uint32_t f32_to_f16_sat(float v) {
  v = fminf(fmaxf(v, -65504.0f), 65504.0f);
  return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v);   // RNE
}
template <int OP>
__device__ __forceinline__ uint32_t to_op(float v) {
  return OP == OP_F16 ? f32_to_f16_sat(v) : f32_to_bf16(v);
}
template <int OP>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  return to_op<OP>(a) | (to_op<OP>(b) << 16);
}
// two bf16 in a dword -> two operand values
template <int OP>
__device__ __forceinline__ uint32_t bf16x2_to_op(uint32_t w) {
  if (OP == OP_BF16) return w;
  return pack2<OP_F16>(bf16_to_f32(w & 0xFFFFu), bf16_to_f32(w >> 16));
}

__device__ __forceinline__ size_t fmt_row_bytes(int fmt, int cols) {
  return fmt == MOE_FMT_Q4_K ? (size_t)(cols / 256) * 144
       : fmt == MOE_FMT_Q6_K ? (size_t)(cols / 256) * 210
                             : (size_t)cols * 2;
}

// Decode k-local elements [16p, 16p+16) of the 64-wide K step starting at column k0 of one weight
// row into the operand type (RNE of the exact f32 value).
template <int WFMT, int OP>
__device__ __forceinline__ void decode16(const uint8_t* row, int k0, int p, uint16_t* dst) {
  if (WFMT == MOE_FMT_BF16) {
    const uint4* s = reinterpret_cast<const uint4*>(row + (size_t)(k0 + 16 * p) * 2);
    uint4 a = s[0], b = s[1];
    if (OP == OP_F16) {
      a = make_uint4(bf16x2_to_op<OP>(a.x), bf16x2_to_op<OP>(a.y), bf16x2_to_op<OP>(a.z), bf16x2_to_op<OP>(a.w));
      b = make_uint4(bf16x2_to_op<OP>(b.x), bf16x2_to_op<OP>(b.y), bf16x2_to_op<OP>(b.z), bf16x2_to_op<OP>(b.w));
    }
    reinterpret_cast<uint4*>(dst)[0] = a;
    reinterpret_cast<uint4*>(dst)[1] = b;
  } else if (WFMT == MOE_FMT_Q4_K) {
    const uint8_t* b = row + (size_t)(k0 >> 8) * 144;
    const int g = (k0 >> 6) & 3;
    const uint4 hdr = *reinterpret_cast<const uint4*>(b);
    const uint4 qs = *reinterpret_cast<const uint4*>(b + 16 + 32 * g + 16 * (p & 1));
    const int hi = p >> 1;
    uint32_t sc, m;
    q4k_scale_min(hdr.y, hdr.z, hdr.w, 2 * g + hi, sc, m);
    const float ds = f16_to_f32(hdr.x & 0xFFFFu) * (float)sc;
    const float dm = f16_to_f32(hdr.x >> 16) * (float)m;
    const uint32_t w[4] = {qs.x, qs.y, qs.z, qs.w};
    uint32_t packed[8];
#pragma unroll
    for (int i = 0; i < 16; i += 2) {
      const uint32_t b0 = (w[i >> 2] >> (8 * (i & 3))) & 0xFFu;
      const uint32_t b1 = (w[(i + 1) >> 2] >> (8 * ((i + 1) & 3))) & 0xFFu;
      const float v0 = fmaf(ds, (float)(hi ? (b0 >> 4) : (b0 & 15u)), -dm);
      const float v1 = fmaf(ds, (float)(hi ? (b1 >> 4) : (b1 & 15u)), -dm);
      packed[i >> 1] = pack2<OP>(v0, v1);
    }
    uint4* d4 = reinterpret_cast<uint4*>(dst);
    d4[0] = make_uint4(packed[0], packed[1], packed[2], packed[3]);
    d4[1] = make_uint4(packed[4], packed[5], packed[6], packed[7]);
  } else {  // Q6_K: 210-byte blocks, 2-byte aligned -> 16-bit reads
    const uint16_t* b = reinterpret_cast<const uint16_t*>(row + (size_t)(k0 >> 8) * 210);
    const int h4 = (k0 >> 6) & 3, g = h4 >> 1, nib = h4 & 1;
    const int j = p >> 1, lh = p & 1;
    const int kk = 2 * nib + j;
    const uint16_t* ql = b + (64 * g + 32 * j + 16 * lh) / 2;
    const uint16_t* qh = b + (128 + 32 * g + 16 * lh) / 2;
    const int scb = 192 + 8 * g + 2 * kk + lh;
    const uint32_t scw = b[scb >> 1];
    const int8_t sc = (int8_t)((scb & 1) ? (scw >> 8) : (scw & 0xFFu));
    const float ds = f16_to_f32(b[104]) * (float)sc;
    const int sl = 4 * nib, sh = 2 * kk;
    uint32_t packed[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t lw = ql[i], hw = qh[i];
      const int q0 = (int)(((lw >> sl) & 15u) | (((hw >> sh) & 3u) << 4)) - 32;
      const int q1 = (int)((((lw >> 8) >> sl) & 15u) | ((((hw >> 8) >> sh) & 3u) << 4)) - 32;
      packed[i] = pack2<OP>(ds * (float)q0, ds * (float)q1);
    }
    uint4* d4 = reinterpret_cast<uint4*>(dst);
    d4[0] = make_uint4(packed[0], packed[1], packed[2], packed[3]);
    d4[1] = make_uint4(packed[4], packed[5], packed[6], packed[7]);
  }
}

// 16 activations [k, k+16) of one row as operands. XDT: source dtype (f32, bf16, or OPND = the
// operand type itself, i.e. a copy).
constexpr int XDT_OPND = 7;
template <int XDT, int OP>
__device__ __forceinline__ void load_a16(const void* src, size_t off, uint16_t* dst) {
  uint4* d4 = reinterpret_cast<uint4*>(dst);
  if (XDT == XDT_OPND || (XDT == MOE_DT_BF16 && OP == OP_BF16)) {
    const uint4* s = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(src) + off);
    d4[0] = s[0];
    d4[1] = s[1];
  } else if (XDT == MOE_DT_BF16) {
    const uint4* s = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(src) + off);
    const uint4 a = s[0], b = s[1];
    d4[0] = make_uint4(bf16x2_to_op<OP>(a.x), bf16x2_to_op<OP>(a.y), bf16x2_to_op<OP>(a.z), bf16x2_to_op<OP>(a.w));
    d4[1] = make_uint4(bf16x2_to_op<OP>(b.x), bf16x2_to_op<OP>(b.y), bf16x2_to_op<OP>(b.z), bf16x2_to_op<OP>(b.w));
  } else {
    const float4* s = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(src) + off);
    uint32_t pk[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 v = s[i];
      pk[2 * i] = pack2<OP>(v.x, v.y);
      pk[2 * i + 1] = pack2<OP>(v.z, v.w);
    }
    d4[0] = make_uint4(pk[0], pk[1], pk[2], pk[3]);
    d4[1] = make_uint4(pk[4], pk[5], pk[6], pk[7]);
  }
}

template <int OP>
__device__ __forceinline__ f32x16_t mfma32(const uint16_t* pa, const uint16_t* pb, f32x16_t c) {
  const uint4 a = *reinterpret_cast<const uint4*>(pa);
  const uint4 b = *reinterpret_cast<const uint4*>(pb);
  if (OP == OP_F16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                 __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// AMODE 0: A rows gathered from x through sorted_pairs / K, tiles from the work list.
// AMODE 1: A rows are x rows 0..T-1 (shared expert), no work list.
template <int WFMT, int XDT, int AMODE, int OP>
__global__ __launch_bounds__(256) void k_gemm_gateup(
    const void* __restrict__ x, const uint8_t* __restrict__ wg, const uint8_t* __restrict__ wu,
    size_t estride, const int32_t* __restrict__ tiles, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ sorted_pairs, int K, int H, int I, int T,
    uint16_t* __restrict__ S) {
  __shared__ __attribute__((aligned(16))) uint16_t As[64 * kLdsPad];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[128 * kLdsPad];
  int e = 0, m0, mend;
  if (AMODE == 0) {
    if ((int)blockIdx.y >= tiles[0]) return;
    e = tiles[1 + 2 * blockIdx.y];
    m0 = tiles[2 + 2 * blockIdx.y];
    mend = min(m0 + 64, offsets[e + 1]);
  } else {
    m0 = blockIdx.y * 64;
    if (m0 >= T) return;
    mend = min(m0 + 64, T);
  }
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int n0 = blockIdx.x * 64;
  const size_t rowb = fmt_row_bytes(WFMT, H);
  // A loader: row ar, quarter aq (16 columns)
  const int ar = tid >> 2, aq = tid & 3;
  int asrc = -1;
  if (m0 + ar < mend) asrc = (AMODE == 0) ? sorted_pairs[m0 + ar] / K : m0 + ar;
  // B loader: row br (0..63 gate, 64..127 up), half bc (32 columns)
  const int br = tid >> 1, bc = tid & 1;
  const uint8_t* brow = (br < 64) ? wg + e * estride + (size_t)(n0 + br) * rowb
                                  : wu + e * estride + (size_t)(n0 + br - 64) * rowb;
  f32x16_t accg = {}, accu = {};
  for (int k0 = 0; k0 < H; k0 += kBK) {
    if (asrc >= 0) {
      load_a16<XDT, OP>(x, (size_t)asrc * H + k0 + 16 * aq, &As[ar * kLdsPad + 16 * aq]);
    } else {
      uint4* d4 = reinterpret_cast<uint4*>(&As[ar * kLdsPad + 16 * aq]);
      d4[0] = make_uint4(0, 0, 0, 0);
      d4[1] = make_uint4(0, 0, 0, 0);
    }
    decode16<WFMT, OP>(brow, k0, 2 * bc, &Bs[br * kLdsPad + 32 * bc]);
    decode16<WFMT, OP>(brow, k0, 2 * bc + 1, &Bs[br * kLdsPad + 32 * bc + 16]);
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < kBK; ks += 16) {
      const int kk = ks + 8 * (lane >> 5);
      const uint16_t* pa = &As[(wm * 32 + (lane & 31)) * kLdsPad + kk];
      accg = mfma32<OP>(pa, &Bs[(wn * 32 + (lane & 31)) * kLdsPad + kk], accg);
      accu = mfma32<OP>(pa, &Bs[(64 + wn * 32 + (lane & 31)) * kLdsPad + kk], accu);
    }
    __syncthreads();
  }
  const int n = n0 + wn * 32 + (lane & 31);
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int m = m0 + wm * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
    if (m < mend) S[(size_t)m * I + n] = (uint16_t)to_op<OP>(silu_f32(accg[r]) * accu[r]);
  }
}

// A = S (operand type, sorted rows or token rows); B = 64 down rows; out f32 rows.
template <int WFMT, int AMODE, int OP>
__global__ __launch_bounds__(256) void k_gemm_down(
    const uint16_t* __restrict__ S, const uint8_t* __restrict__ wd, size_t estride,
    const int32_t* __restrict__ tiles, const int32_t* __restrict__ offsets, int H, int I, int T,
    float* __restrict__ y) {
  __shared__ __attribute__((aligned(16))) uint16_t As[64 * kLdsPad];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[64 * kLdsPad];
  int e = 0, m0, mend;
  if (AMODE == 0) {
    if ((int)blockIdx.y >= tiles[0]) return;
    e = tiles[1 + 2 * blockIdx.y];
    m0 = tiles[2 + 2 * blockIdx.y];
    mend = min(m0 + 64, offsets[e + 1]);
  } else {
    m0 = blockIdx.y * 64;
    if (m0 >= T) return;
    mend = min(m0 + 64, T);
  }
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int n0 = blockIdx.x * 64;
  const size_t rowb = fmt_row_bytes(WFMT, I);
  const int ar = tid >> 2, aq = tid & 3;
  const bool avalid = m0 + ar < mend;
  const int br = tid >> 2, bq = tid & 3;
  const uint8_t* brow = wd + e * estride + (size_t)(n0 + br) * rowb;
  f32x16_t acc = {};
  for (int k0 = 0; k0 < I; k0 += kBK) {
    if (avalid) {
      load_a16<XDT_OPND, OP>(S, (size_t)(m0 + ar) * I + k0 + 16 * aq, &As[ar * kLdsPad + 16 * aq]);
    } else {
      uint4* d4 = reinterpret_cast<uint4*>(&As[ar * kLdsPad + 16 * aq]);
      d4[0] = make_uint4(0, 0, 0, 0);
      d4[1] = make_uint4(0, 0, 0, 0);
    }
    decode16<WFMT, OP>(brow, k0, bq, &Bs[br * kLdsPad + 16 * bq]);
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < kBK; ks += 16) {
      const int kk = ks + 8 * (lane >> 5);
      acc = mfma32<OP>(&As[(wm * 32 + (lane & 31)) * kLdsPad + kk],
                       &Bs[(wn * 32 + (lane & 31)) * kLdsPad + kk], acc);
    }
    __syncthreads();
  }
  const int n = n0 + wn * 32 + (lane & 31);
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int m = m0 + wm * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
    if (m < mend) y[(size_t)m * H + n] = acc[r];
  }
}

}  // namespace moe

using namespace moe;

template <int WFMT, int OP>
static void launch_gu(const void* x, int x_dtype, const uint8_t* wg, const uint8_t* wu,
                      size_t estride, const int32_t* tiles, int max_tiles, const int32_t* offsets,
                      const int32_t* sorted_pairs, int K, int H, int I, int T, uint16_t* S,
                      hipStream_t st) {
  const bool ident = (tiles == nullptr);
  dim3 grid(I / 64, ident ? (T + 63) / 64 : max_tiles);
  if (x_dtype == MOE_DT_F32) {
    if (ident) hipLaunchKernelGGL((k_gemm_gateup<WFMT, MOE_DT_F32, 1, OP>), grid, dim3(256), 0, st, x, wg, wu, estride, tiles, offsets, sorted_pairs, K, H, I, T, S);
    else hipLaunchKernelGGL((k_gemm_gateup<WFMT, MOE_DT_F32, 0, OP>), grid, dim3(256), 0, st, x, wg, wu, estride, tiles, offsets, sorted_pairs, K, H, I, T, S);
  } else {
    if (ident) hipLaunchKernelGGL((k_gemm_gateup<WFMT, MOE_DT_BF16, 1, OP>), grid, dim3(256), 0, st, x, wg, wu, estride, tiles, offsets, sorted_pairs, K, H, I, T, S);
    else hipLaunchKernelGGL((k_gemm_gateup<WFMT, MOE_DT_BF16, 0, OP>), grid, dim3(256), 0, st, x, wg, wu, estride, tiles, offsets, sorted_pairs, K, H, I, T, S);
  }
}

template <int OP>
static int gu_fmt(const void* x, int x_dtype, const uint8_t* g, const uint8_t* u, int fmt,
                  size_t es, const int32_t* tiles, int mt, int T, const int32_t* off,
                  const int32_t* sp, int K, int H, int I, uint16_t* S, hipStream_t st) {
  if (fmt == MOE_FMT_Q4_K) launch_gu<MOE_FMT_Q4_K, OP>(x, x_dtype, g, u, es, tiles, mt, off, sp, K, H, I, T, S, st);
  else if (fmt == MOE_FMT_Q6_K) launch_gu<MOE_FMT_Q6_K, OP>(x, x_dtype, g, u, es, tiles, mt, off, sp, K, H, I, T, S, st);
  else if (fmt == MOE_FMT_BF16) launch_gu<MOE_FMT_BF16, OP>(x, x_dtype, g, u, es, tiles, mt, off, sp, K, H, I, T, S, st);
  else return moe_set_error(MOE_E_FORMAT, "MFMA gate_up: unsupported format %d", fmt);
  return MOE_OK;
}

int moe_launch_gemm_gateup(const void* x, int x_dtype, const void* w_gate, const void* w_up,
                           int fmt, size_t expert_stride, const int32_t* tiles, int max_tiles,
                           int T, const int32_t* offsets, const int32_t* sorted_pairs, int K,
                           int H, int I, int op_bf16, uint16_t* S, hipStream_t st) {
  if (H % 256 || I % 64)
    return moe_set_error(MOE_E_UNSUPPORTED, "MFMA gate_up needs H %% 256 == 0, I %% 64 == 0");
  const uint8_t* g = reinterpret_cast<const uint8_t*>(w_gate);
  const uint8_t* u = reinterpret_cast<const uint8_t*>(w_up);
  const int rc = op_bf16 ? gu_fmt<OP_BF16>(x, x_dtype, g, u, fmt, expert_stride, tiles, max_tiles, T, offsets, sorted_pairs, K, H, I, S, st)
                         : gu_fmt<OP_F16>(x, x_dtype, g, u, fmt, expert_stride, tiles, max_tiles, T, offsets, sorted_pairs, K, H, I, S, st);
  if (rc != MOE_OK) return rc;
  return moe_check_launch("gemm_gateup");
}

template <int OP>
static int dn_fmt(const uint16_t* S, const uint8_t* w, int fmt, size_t es, const int32_t* tiles,
                  int mt, int T, const int32_t* off, int H, int I, float* y, hipStream_t st) {
  const bool ident = (tiles == nullptr);
  dim3 grid(H / 64, ident ? (T + 63) / 64 : mt);
#define MOE_DN(F)                                                                                   \
  do {                                                                                              \
    if (ident) hipLaunchKernelGGL((k_gemm_down<F, 1, OP>), grid, dim3(256), 0, st, S, w, es, tiles, off, H, I, T, y); \
    else hipLaunchKernelGGL((k_gemm_down<F, 0, OP>), grid, dim3(256), 0, st, S, w, es, tiles, off, H, I, T, y);      \
  } while (0)
  if (fmt == MOE_FMT_Q4_K) MOE_DN(MOE_FMT_Q4_K);
  else if (fmt == MOE_FMT_Q6_K) MOE_DN(MOE_FMT_Q6_K);
  else if (fmt == MOE_FMT_BF16) MOE_DN(MOE_FMT_BF16);
  else return moe_set_error(MOE_E_FORMAT, "MFMA down: unsupported format %d", fmt);
#undef MOE_DN
  return MOE_OK;
}

int moe_launch_gemm_down(const uint16_t* S, const void* w_down, int fmt, size_t expert_stride,
                         const int32_t* tiles, int max_tiles, int T, const int32_t* offsets,
                         int H, int I, int op_bf16, float* y, hipStream_t st) {
  if (H % 64 || I % 256)
    return moe_set_error(MOE_E_UNSUPPORTED, "MFMA down needs H %% 64 == 0, I %% 256 == 0");
  const uint8_t* w = reinterpret_cast<const uint8_t*>(w_down);
  const int rc = op_bf16 ? dn_fmt<OP_BF16>(S, w, fmt, expert_stride, tiles, max_tiles, T, offsets, H, I, y, st)
                         : dn_fmt<OP_F16>(S, w, fmt, expert_stride, tiles, max_tiles, T, offsets, H, I, y, st);
  if (rc != MOE_OK) return rc;
  return moe_check_launch("gemm_down");
}
