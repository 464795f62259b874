// Untied lm_head GEMV (gfx950): logits[b][j] = sum_k h[b][k] * W[row_j][k], f32, for a table W of
// V rows of H = 2048 in Q6_K (the shipped artifact's output.weight), Q8_0 or bf16, over all rows
// (dense) or a list of row ids (gather). This is prototype/lm_head/lm_head_kernels.h:474-512
// (lmh_dot_batch: one row's dot for up to LMH_MAX_BATCH = 8 hidden vectors) on the path
// lm_head.hip:51 launches, with the Q6_K width the prototype defers (prototype/lm_head/results.md:341-343).
//
// HBM-bound: every table byte is read once per pass (one pass per 4 tokens), 1680 B per row in
// Q6_K (417 MB at V = 248320), 2176 B in Q8_0, 4096 B in bf16. Layout of the work:
//   * one row per wave; each lane owns a fixed set of 32 element positions of every row, so its
//     slice of the hidden vectors (32 floats per token) stays in registers for the whole sweep;
//   * Q6_K / Q8_0 rows (2-byte-aligned blocks of 210 / 34 B) are staged into LDS by the block with
//     coalesced 16-byte loads, 8 or 16 rows per iteration, double buffered (the next iteration's loads
//     are in flight while the current rows are decoded); lanes then read their bytes from LDS as
//     aligned dwords and realign them with v_alignbyte;
//   * bf16 rows are read straight from HBM, 64 lanes x 16 B contiguous per load, two rows in
//     flight per wave.
// Arithmetic: the block's integer quants are accumulated against h (the quant as an exact small
// float), and the block scale multiplies the partial sum: sum_i h_i (s q_i) = s sum_i h_i q_i, a
// re-association of the reference's f32 dot, which the reference's own band covers
// (prototype/lm_head/gate.py:214-240: gamma_{2K-1} sum |h_k w_k| when products are inexact).
#include "common.h"
#include "moe_internal.h"

namespace moe {
namespace lmh {

constexpr int kH = 2048;                 // the lane mapping covers 64 lanes x 32 positions
constexpr int kThreads = 256;            // 4 waves
constexpr int kPad = 16;                 // LDS slack after the last row (the Q8_0 window overreads 6 B)
// Rows per wave per block iteration of the staged formats: with one token the decode is light
// and registers are few, so smaller iterations (less LDS) let four blocks share a CU; with more
// tokens the FMAs dominate, registers allow two blocks, and longer iterations amortise the sync.
template <int NB> struct Iter {
  static constexpr int kRowsPerWave = NB == 1 ? 2 : 4;
  static constexpr int kRows = 4 * kRowsPerWave;
  static constexpr int kBlocksPerCu = NB == 1 ? 4 : 2;
};

template <int FMT> struct Staged;
template <> struct Staged<MOE_FMT_Q6_K> {
  static constexpr int kRowB = kH / 256 * 210;                      // 1680
};
template <> struct Staged<MOE_FMT_Q8_0> {
  static constexpr int kRowB = kH / 32 * 34;                        // 2176
};

template <int XDT>
__device__ __forceinline__ float load_h(const void* h, size_t i) {
  if (XDT == MOE_DT_F32) return reinterpret_cast<const float*>(h)[i];
  return bf16_to_f32(reinterpret_cast<const uint16_t*>(h)[i]);
}

// byte b of v as a float (one v_cvt_f32_ubyteN)
__device__ __forceinline__ float cvt_b(uint32_t v, int b) { return (float)((v >> (8 * b)) & 0xFFu); }

// the table row of output j: j itself, or ids[j] (-1 when that id is outside [0, V))
template <int GATHER>
__device__ __forceinline__ long long row_of(const int32_t* ids, long long j, long long V) {
  if (!GATHER) return j;
  const int id = ids[j];
  return (id >= 0 && (long long)id < V) ? (long long)id : -1;
}

// Lane L's 32 positions: Q6_K: super-block sb = L >> 3, half g, 16-element run j and nibble
// parity k2 (element 128g + 32k + l of the super-block, k in {k2, k2 + 2}, l in [16j, 16j + 16):
// tools/gguf_reader.py:299-322 addresses it as ql[64g + 32(k & 1) + l] nibble k >> 1,
// qh[32g + l] bits 2k, sc[8g + 2k + (l >> 4)]); Q8_0: block L (elements 32L .. 32L + 31).
template <int FMT>
__device__ __forceinline__ int pos_of(int lane, int i) {
  if (FMT == MOE_FMT_Q6_K) {
    const int sb = lane >> 3, g = (lane >> 2) & 1, j = (lane >> 1) & 1, k2 = lane & 1;
    return 256 * sb + 128 * g + 32 * k2 + 16 * j + (i & 15) + ((i >> 4) << 6);
  }
  return 32 * lane + i;
}

template <int FMT, int NB, int XDT, int GATHER>
__global__ __launch_bounds__(kThreads) void k_lm_head_staged(const void* __restrict__ h,
                                                             const uint8_t* __restrict__ w,
                                                             long long V,
                                                             const int32_t* __restrict__ ids,
                                                             long long n_rows,
                                                             float* __restrict__ out) {
  constexpr int kRowB = Staged<FMT>::kRowB;
  constexpr int kRowsPerWave = Iter<NB>::kRowsPerWave, kRows = Iter<NB>::kRows;
  constexpr int kChunks = kRowB / 16;                               // 105 / 136 per row
  constexpr int kBuf = kRows * kRowB + kPad;
  constexpr int kLoads = (kRows * kChunks + kThreads - 1) / kThreads;
  __shared__ __attribute__((aligned(16))) uint8_t smem[2][kBuf];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;

  // this lane's slice of the hidden vectors, and its sums (the quant offsets below)
  float hv[NB][32], hs[NB][2];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    hs[b][0] = 0.0f;
    hs[b][1] = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      hv[b][i] = load_h<XDT>(h, (size_t)b * kH + pos_of<FMT>(lane, i));
      hs[b][(FMT == MOE_FMT_Q6_K) ? (i >> 4) : 0] += hv[b][i];
    }
  }

  const long long n_it = (n_rows + kRows - 1) / kRows;
  uint4 reg[kLoads];
  long long it = blockIdx.x;
  auto load = [&](long long it_) {
    const long long r0 = it_ * kRows;
#pragma unroll
    for (int q = 0; q < kLoads; ++q) {
      const int c = t + kThreads * q;
      const int r = c / kChunks;
      reg[q] = make_uint4(0u, 0u, 0u, 0u);
      if (c < kRows * kChunks && r0 + r < n_rows) {
        const long long row = row_of<GATHER>(ids, r0 + r, V);
        if (row >= 0)
          reg[q] = *reinterpret_cast<const uint4*>(w + (size_t)row * kRowB + 16 * (c - r * kChunks));
      }
    }
  };
  auto stage = [&](uint8_t* buf) {
#pragma unroll
    for (int q = 0; q < kLoads; ++q) {
      const int c = t + kThreads * q;
      if (c < kRows * kChunks) *reinterpret_cast<uint4*>(buf + 16 * c) = reg[q];
    }
  };
  if (it < n_it) load(it);
  int cur = 0;
  for (; it < n_it; it += gridDim.x) {
    stage(smem[cur]);
    __syncthreads();
    if (it + gridDim.x < n_it) load(it + gridDim.x);
    const uint32_t* L32 = reinterpret_cast<const uint32_t*>(smem[cur]);
#pragma unroll 1
    for (int rr = 0; rr < kRowsPerWave; ++rr) {
      const int r = kRowsPerWave * wave + rr;
      const long long j = it * kRows + r;
      if (j >= n_rows) break;
      float part[NB];
      if (FMT == MOE_FMT_Q6_K) {
        const int sb = lane >> 3, g = (lane >> 2) & 1, jj = (lane >> 1) & 1, k2 = lane & 1;
        const int sbb = r * kRowB + 210 * sb;                       // 2-byte aligned
        const int s = (sbb & 3) * 8;                                // bit shift 0 or 16
        const int oql = (sbb + 64 * g + 32 * k2 + 16 * jj) >> 2;    // dword index, same offset
        const int oqh = (sbb + 128 + 32 * g + 16 * jj) >> 2;
        uint32_t ql[5], qh[5];
#pragma unroll
        for (int i = 0; i < 5; ++i) { ql[i] = L32[oql + i]; qh[i] = L32[oqh + i]; }
        const int osc = sbb + 192 + 8 * g + 2 * k2 + jj;
        const uint32_t sw0 = L32[osc >> 2], sw1 = L32[(osc >> 2) + 1];
        const int ssh = (osc & 3) * 8;
        const float sc_lo = (float)(int8_t)(sw0 >> ssh), sc_hi = (float)(int8_t)(sw1 >> ssh);
        const int od = sbb + 208;
        const float d = f16_to_f32((L32[od >> 2] >> ((od & 3) * 8)) & 0xFFFFu);
        float alo[NB], ahi[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) { alo[b] = 0.0f; ahi[b] = 0.0f; }
        const uint32_t shl = 4u - 2u * (uint32_t)k2, shr = 2u * (uint32_t)k2;
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          const uint32_t wq = __builtin_amdgcn_alignbyte(ql[m + 1], ql[m], s >> 3);
          const uint32_t wh = __builtin_amdgcn_alignbyte(qh[m + 1], qh[m], s >> 3);
          const uint32_t lo = (wq & 0x0F0F0F0Fu) | ((wh << shl) & 0x30303030u);
          const uint32_t hi = ((wq >> 4) & 0x0F0F0F0Fu) | ((wh >> shr) & 0x30303030u);
#pragma unroll
          for (int bb = 0; bb < 4; ++bb) {
            const float ql_ = cvt_b(lo, bb), qh_ = cvt_b(hi, bb);
#pragma unroll
            for (int b = 0; b < NB; ++b) {
              alo[b] = fmaf(hv[b][4 * m + bb], ql_, alo[b]);
              ahi[b] = fmaf(hv[b][16 + 4 * m + bb], qh_, ahi[b]);
            }
          }
        }
        const float dlo = d * sc_lo, dhi = d * sc_hi;               // exact (<= 19 bits)
#pragma unroll
        for (int b = 0; b < NB; ++b)
          part[b] = dlo * fmaf(-32.0f, hs[b][0], alo[b]) + dhi * fmaf(-32.0f, hs[b][1], ahi[b]);
      } else {
        const int off = r * kRowB + 34 * lane;                      // 2-byte aligned
        const int ow = off >> 2, s = off & 3;                       // s = 0 or 2
        uint32_t q[10];
#pragma unroll
        for (int i = 0; i < 10; ++i) q[i] = L32[ow + i];
        const float d = f16_to_f32((q[0] >> (8 * s)) & 0xFFFFu);
        const int qb = (s + 2) >> 2, qs = (s + 2) & 3;              // quants start at byte s + 2
        float a[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) a[b] = 0.0f;
#pragma unroll
        for (int m = 0; m < 8; ++m) {
          const uint32_t lo_w = qb ? q[m + 1] : q[m], hi_w = qb ? q[m + 2] : q[m + 1];
          // int8 q + 128 as an unsigned byte: the sign bit flipped
          const uint32_t x = __builtin_amdgcn_alignbyte(hi_w, lo_w, qs) ^ 0x80808080u;
#pragma unroll
          for (int bb = 0; bb < 4; ++bb) {
            const float qf = cvt_b(x, bb);
#pragma unroll
            for (int b = 0; b < NB; ++b) a[b] = fmaf(hv[b][4 * m + bb], qf, a[b]);
          }
        }
#pragma unroll
        for (int b = 0; b < NB; ++b) part[b] = d * fmaf(-128.0f, hs[b][0], a[b]);
      }
      const bool valid = row_of<GATHER>(ids, j, V) >= 0;
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const float v = wave_sum_f32(part[b]);
        if (lane == b) out[(size_t)b * n_rows + j] = valid ? v : __builtin_nanf("");
      }
    }
    cur ^= 1;
  }
}

template <int NB, int XDT, int GATHER>
__global__ __launch_bounds__(kThreads) void k_lm_head_bf16(const void* __restrict__ h,
                                                           const uint16_t* __restrict__ w,
                                                           long long V,
                                                           const int32_t* __restrict__ ids,
                                                           long long n_rows,
                                                           float* __restrict__ out) {
  const int t = threadIdx.x, lane = t & 63;
  // lane L: elements 512c + 8L .. +8 (c = 0..3): every load is 64 lanes x 16 B contiguous
  float hv[NB][32];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int i = 0; i < 32; ++i) hv[b][i] = load_h<XDT>(h, (size_t)b * kH + 512 * (i >> 3) + 8 * lane + (i & 7));
  const long long gw = (long long)blockIdx.x * (kThreads / 64) + (t >> 6);
  const long long nw = (long long)gridDim.x * (kThreads / 64);
  for (long long j0 = gw; j0 < n_rows; j0 += 2 * nw) {
    uint4 v[2][4];
    long long rows[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const long long j = j0 + u * nw;
      rows[u] = j < n_rows ? row_of<GATHER>(ids, j, V) : -1;
#pragma unroll
      for (int c = 0; c < 4; ++c)
        v[u][c] = rows[u] >= 0 ? *reinterpret_cast<const uint4*>(w + (size_t)rows[u] * kH + 512 * c + 8 * lane)
                               : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const long long j = j0 + u * nw;
      if (j >= n_rows) break;
      float a[NB];
#pragma unroll
      for (int b = 0; b < NB; ++b) a[b] = 0.0f;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint32_t ww[4] = {v[u][c].x, v[u][c].y, v[u][c].z, v[u][c].w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float wf = bf16_to_f32((e & 1) ? (ww[e >> 1] >> 16) : (ww[e >> 1] & 0xFFFFu));
#pragma unroll
          for (int b = 0; b < NB; ++b) a[b] = fmaf(hv[b][8 * c + e], wf, a[b]);
        }
      }
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const float s = wave_sum_f32(a[b]);
        if (lane == b) out[(size_t)b * n_rows + j] = rows[u] >= 0 ? s : __builtin_nanf("");
      }
    }
  }
}

}  // namespace lmh
}  // namespace moe

using namespace moe;

namespace {

int cu_count() {
  static int ncu = -1;
  if (ncu < 0) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      ncu = 256;
  }
  return ncu;
}

template <int FMT, int NB, int XDT, int GATHER>
void launch_staged(const void* h, const uint8_t* w, long long V, const int32_t* ids, long long n,
                   float* out, hipStream_t st) {
  constexpr int kRows = lmh::Iter<NB>::kRows;
  const long long n_it = (n + kRows - 1) / kRows;
  const long long cap = (long long)lmh::Iter<NB>::kBlocksPerCu * cu_count();
  const long long grid = n_it < cap ? n_it : cap;
  hipLaunchKernelGGL((lmh::k_lm_head_staged<FMT, NB, XDT, GATHER>), dim3((unsigned)grid),
                     dim3(lmh::kThreads), 0, st, h, w, V, ids, n, out);
}

template <int NB, int XDT, int GATHER>
void launch_bf16(const void* h, const uint8_t* w, long long V, const int32_t* ids, long long n,
                 float* out, hipStream_t st) {
  const long long waves = (n + 1) / 2;
  const long long want = (waves + 3) / 4, cap = 8LL * cu_count();
  hipLaunchKernelGGL((lmh::k_lm_head_bf16<NB, XDT, GATHER>), dim3((unsigned)(want < cap ? want : cap)),
                     dim3(lmh::kThreads), 0, st, h, reinterpret_cast<const uint16_t*>(w), V, ids, n, out);
}

template <int NB, int XDT, int GATHER>
void launch_fmt(int fmt, const void* h, const uint8_t* w, long long V, const int32_t* ids,
                long long n, float* out, hipStream_t st) {
  if (fmt == MOE_FMT_Q6_K) launch_staged<MOE_FMT_Q6_K, NB, XDT, GATHER>(h, w, V, ids, n, out, st);
  else if (fmt == MOE_FMT_Q8_0) launch_staged<MOE_FMT_Q8_0, NB, XDT, GATHER>(h, w, V, ids, n, out, st);
  else launch_bf16<NB, XDT, GATHER>(h, w, V, ids, n, out, st);
}

template <int XDT, int GATHER>
void launch_nb(int nb, int fmt, const void* h, const uint8_t* w, long long V, const int32_t* ids,
               long long n, float* out, hipStream_t st) {
  switch (nb) {
    case 1: launch_fmt<1, XDT, GATHER>(fmt, h, w, V, ids, n, out, st); break;
    case 2: launch_fmt<2, XDT, GATHER>(fmt, h, w, V, ids, n, out, st); break;
    case 3: launch_fmt<3, XDT, GATHER>(fmt, h, w, V, ids, n, out, st); break;
    default: launch_fmt<4, XDT, GATHER>(fmt, h, w, V, ids, n, out, st); break;
  }
}

}  // namespace

bool moe_lm_head_supported(int H, int fmt) {
  return H == lmh::kH && (fmt == MOE_FMT_Q6_K || fmt == MOE_FMT_Q8_0 || fmt == MOE_FMT_BF16);
}

int moe_launch_lm_head(const void* h, int h_dtype, int B, const void* w, int fmt, long long V,
                       const int32_t* row_ids, long long n_rows, float* logits, hipStream_t st) {
  const uint8_t* wb = reinterpret_cast<const uint8_t*>(w);
  const size_t hstride = (size_t)lmh::kH * (h_dtype == MOE_DT_F32 ? 4 : 2);
  // tokens in passes of up to four (each pass reads the table once)
  for (int b0 = 0; b0 < B; b0 += 4) {
    const int nb = B - b0 < 4 ? B - b0 : 4;
    const void* hp = reinterpret_cast<const uint8_t*>(h) + (size_t)b0 * hstride;
    float* op = logits + (size_t)b0 * n_rows;
    if (h_dtype == MOE_DT_F32) {
      if (row_ids) launch_nb<MOE_DT_F32, 1>(nb, fmt, hp, wb, V, row_ids, n_rows, op, st);
      else launch_nb<MOE_DT_F32, 0>(nb, fmt, hp, wb, V, nullptr, n_rows, op, st);
    } else {
      if (row_ids) launch_nb<MOE_DT_BF16, 1>(nb, fmt, hp, wb, V, row_ids, n_rows, op, st);
      else launch_nb<MOE_DT_BF16, 0>(nb, fmt, hp, wb, V, nullptr, n_rows, op, st);
    }
    const int rc = moe_check_launch("lm_head");
    if (rc != MOE_OK) return rc;
  }
  return MOE_OK;
}
