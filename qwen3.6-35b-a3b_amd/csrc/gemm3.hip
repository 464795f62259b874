// Prefill-path grouped GEMM, warp-specialized form (gfx950, v_mfma_f32_32x32x16_f16, f32 acc).
//
// Work: one tile of up to 160 sorted (token, slot) rows of one expert (k_build_tiles, 160-row
// tiles: at 4096 tokens an expert averages 128 rows, so almost every expert is one tile and its
// weights are loaded and decoded once) times one output slab per block. Tiles are dealt to XCDs
// so the slabs of one tile run on one XCD and share its activation rows in L2. Block = 8 waves,
// one producer and one consumer per SIMD:
//   producers (waves 4..7): per 64-wide K step, load the activation rows (f16; eight lanes per
//     128-byte row segment, so a load instruction touches eight cache lines) and the raw Q4_K /
//     bf16 bytes of the slab's weight rows, decode the weights to f16 once, and store both tiles
//     into LDS (double buffered), the loads running four steps ahead in registers;
//   consumers (waves 0..3): read A and B fragments from LDS and issue the MFMAs; each owns all 160
//     rows x (32 gate + 32 up) columns (gate_up) or 64 down columns (down).
// A producer's VALU decode and a consumer's MFMAs on the same SIMD run concurrently, and every
// weight element is decoded exactly once per block. One barrier per step hands the buffers over.
//
// Decode arithmetic (mantissa trick): low nibble q under the f16 0x6400 (1024)
// gives 1024 + q, a high nibble left at bits 4-7 under 0x5400 (64, ulp 1/16) gives 64 + q; one
// packed subtract leaves q exactly and one packed FMA gives q * f16(d * sc) - f16(dmin * m).
#include "common.h"
#include "moe_internal.h"

namespace moe {

typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

namespace g3 {

constexpr int kBM = MOE_GEMM3_BM;       // 160 rows per tile (5 MFMA row groups)
constexpr int kMG = kBM / 32;
constexpr int kBK = 64;                 // K per step
constexpr int kS = 72;                  // LDS row stride in f16 (144 B)
constexpr int kXcd = 8;
constexpr int kBN = 256;                // weight rows per block (gate_up: 128 gate + 128 up)

__device__ __forceinline__ f32x16_t mfma(uint4 a, uint4 b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                               __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

__device__ __forceinline__ uint32_t and_or_s(uint32_t p, uint32_t mask, uint32_t magic) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(p), "s"(mask), "v"(magic));
  return r;
}

// 4 nibbles (bytes of w at positions sel) -> f16x2 pairs, scale applied
template <bool HIGH>
__device__ __forceinline__ uint32_t q4_pair(uint32_t w, uint32_t sel, f16x2_t ds, f16x2_t ndm) {
  const uint32_t p = __builtin_amdgcn_perm(0u, w, sel);
  const uint32_t magic = HIGH ? and_or_s(p, 0x00F000F0u, 0x54005400u)
                              : and_or_s(p, 0x000F000Fu, 0x64006400u);
  const _Float16 off = HIGH ? (_Float16)64.0f : (_Float16)1024.0f;
  const f16x2_t q = __builtin_bit_cast(f16x2_t, magic) - (f16x2_t){off, off};
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(q, ds, ndm));
}

// 16 bytes of nibbles -> 16 f16 (low or high nibbles), as two uint4 in k order
template <bool HIGH>
__device__ __forceinline__ void q4_16(uint4 w, f16x2_t ds, f16x2_t ndm, uint4& o0, uint4& o1) {
  o0.x = q4_pair<HIGH>(w.x, 0x0C010C00u, ds, ndm);
  o0.y = q4_pair<HIGH>(w.x, 0x0C030C02u, ds, ndm);
  o0.z = q4_pair<HIGH>(w.y, 0x0C010C00u, ds, ndm);
  o0.w = q4_pair<HIGH>(w.y, 0x0C030C02u, ds, ndm);
  o1.x = q4_pair<HIGH>(w.z, 0x0C010C00u, ds, ndm);
  o1.y = q4_pair<HIGH>(w.z, 0x0C030C02u, ds, ndm);
  o1.z = q4_pair<HIGH>(w.w, 0x0C010C00u, ds, ndm);
  o1.w = q4_pair<HIGH>(w.w, 0x0C030C02u, ds, ndm);
}

// Q5_K: the same with the 5th bits (bytes of qh at the same positions; hs = the bit of each byte:
// 2g for the low nibbles, 2g + 1 for the high): under 0x6400 the bit goes to mantissa bit 4
// (1024 + q, q <= 31), under 0x5400 to mantissa bit 8 (64 + q). Shifting the permuted qh pair
// right by hs <= 7 puts each lane's bit at the lane's bit 0 and moves the upper byte's other
// bits to lane bit 9 or above, so the 1-bit masks read each lane's own byte.
template <bool HIGH>
__device__ __forceinline__ uint32_t q5_pair(uint32_t w, uint32_t h, uint32_t sel, uint32_t hs,
                                            f16x2_t ds, f16x2_t ndm) {
  const uint32_t p = __builtin_amdgcn_perm(0u, w, sel);
  const uint32_t hp = __builtin_amdgcn_perm(0u, h, sel) >> hs;
  const uint32_t magic = HIGH ? and_or_s(p, 0x00F000F0u, 0x54005400u) | ((hp << 8) & 0x01000100u)
                              : and_or_s(p, 0x000F000Fu, 0x64006400u) | ((hp << 4) & 0x00100010u);
  const _Float16 off = HIGH ? (_Float16)64.0f : (_Float16)1024.0f;
  const f16x2_t q = __builtin_bit_cast(f16x2_t, magic) - (f16x2_t){off, off};
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(q, ds, ndm));
}

template <bool HIGH>
__device__ __forceinline__ void q5_16(uint4 w, uint4 h, uint32_t hs, f16x2_t ds, f16x2_t ndm,
                                      uint4& o0, uint4& o1) {
  o0.x = q5_pair<HIGH>(w.x, h.x, 0x0C010C00u, hs, ds, ndm);
  o0.y = q5_pair<HIGH>(w.x, h.x, 0x0C030C02u, hs, ds, ndm);
  o0.z = q5_pair<HIGH>(w.y, h.y, 0x0C010C00u, hs, ds, ndm);
  o0.w = q5_pair<HIGH>(w.y, h.y, 0x0C030C02u, hs, ds, ndm);
  o1.x = q5_pair<HIGH>(w.z, h.z, 0x0C010C00u, hs, ds, ndm);
  o1.y = q5_pair<HIGH>(w.z, h.z, 0x0C030C02u, hs, ds, ndm);
  o1.z = q5_pair<HIGH>(w.w, h.w, 0x0C010C00u, hs, ds, ndm);
  o1.w = q5_pair<HIGH>(w.w, h.w, 0x0C030C02u, hs, ds, ndm);
}

__device__ __forceinline__ void q4_scales(uint4 hdr, int j, f16x2_t& ds, f16x2_t& ndm) {
  uint32_t sc, m;
  q4k_scale_min(hdr.y, hdr.z, hdr.w, j, sc, m);
  const _Float16 d = (_Float16)(f16_to_f32(hdr.x & 0xFFFFu) * (float)sc);
  const _Float16 n = (_Float16)(-(f16_to_f32(hdr.x >> 16) * (float)m));
  ds = (f16x2_t){d, d};
  ndm = (f16x2_t){n, n};
}

__device__ __forceinline__ uint32_t bf2_to_f16x2(uint32_t w) {
  const f16x2_t v = {(_Float16)__uint_as_float(w << 16), (_Float16)__uint_as_float(w & 0xFFFF0000u)};
  return __builtin_bit_cast(uint32_t, v);
}

// One producer thread's share of a step: weight row `row` (a 64-wide K step = 64 elements) and
// activation row `arow` (64 elements = 128 B, as 2 threads x 64 B... see Producer).
template <int WFMT>
struct WRaw;
template <>
struct WRaw<MOE_FMT_Q4_K> {
  uint4 hdr, lo, hi;                    // header, nibble bytes [0,16) and [16,32) of the step's group
  __device__ __forceinline__ void load(const uint8_t* row, int k0) {
    const uint8_t* b = row + (size_t)(k0 >> 8) * 144;
    const int g = (k0 >> 6) & 3;
    hdr = *reinterpret_cast<const uint4*>(b);
    lo = *reinterpret_cast<const uint4*>(b + 16 + 32 * g);
    hi = *reinterpret_cast<const uint4*>(b + 16 + 32 * g + 16);
  }
  // 64 f16 in k order into dst (LDS row, 128 B)
  __device__ __forceinline__ void decode(int k0, uint16_t* dst) const {
    const int g = (k0 >> 6) & 3;
    f16x2_t ds0, nd0, ds1, nd1;
    q4_scales(hdr, 2 * g, ds0, nd0);
    q4_scales(hdr, 2 * g + 1, ds1, nd1);
    uint4 a, b;
    uint4* d = reinterpret_cast<uint4*>(dst);
    q4_16<false>(lo, ds0, nd0, a, b);     // elements 0..15
    d[0] = a; d[1] = b;
    q4_16<false>(hi, ds0, nd0, a, b);     // 16..31
    d[2] = a; d[3] = b;
    q4_16<true>(lo, ds1, nd1, a, b);      // 32..47
    d[4] = a; d[5] = b;
    q4_16<true>(hi, ds1, nd1, a, b);      // 48..63
    d[6] = a; d[7] = b;
  }
};
template <>
struct WRaw<MOE_FMT_Q5_K> {
  uint4 hdr, lo, hi, h0, h1;            // header, the step group's 32 nibble bytes, qh[0..31]
  __device__ __forceinline__ void load(const uint8_t* row, int k0) {
    const uint8_t* b = row + (size_t)(k0 >> 8) * 176;
    const int g = (k0 >> 6) & 3;
    hdr = *reinterpret_cast<const uint4*>(b);
    h0 = *reinterpret_cast<const uint4*>(b + 16);
    h1 = *reinterpret_cast<const uint4*>(b + 32);
    lo = *reinterpret_cast<const uint4*>(b + 48 + 32 * g);
    hi = *reinterpret_cast<const uint4*>(b + 48 + 32 * g + 16);
  }
  // 64 f16 in k order: sub-block 2g (low nibbles, qh bit 2g) then 2g + 1 (high, bit 2g + 1)
  __device__ __forceinline__ void decode(int k0, uint16_t* dst) const {
    const int g = (k0 >> 6) & 3;
    const uint32_t hs = 2u * (uint32_t)g;
    f16x2_t ds0, nd0, ds1, nd1;
    q4_scales(hdr, 2 * g, ds0, nd0);
    q4_scales(hdr, 2 * g + 1, ds1, nd1);
    uint4 a, b;
    uint4* d = reinterpret_cast<uint4*>(dst);
    q5_16<false>(lo, h0, hs, ds0, nd0, a, b);     // elements 0..15
    d[0] = a; d[1] = b;
    q5_16<false>(hi, h1, hs, ds0, nd0, a, b);     // 16..31
    d[2] = a; d[3] = b;
    q5_16<true>(lo, h0, hs + 1, ds1, nd1, a, b);  // 32..47
    d[4] = a; d[5] = b;
    q5_16<true>(hi, h1, hs + 1, ds1, nd1, a, b);  // 48..63
    d[6] = a; d[7] = b;
  }
};
template <>
struct WRaw<MOE_FMT_BF16> {
  uint4 q[8];
  __device__ __forceinline__ void load(const uint8_t* row, int k0) {
    const uint4* r = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(row) + k0);
#pragma unroll
    for (int i = 0; i < 8; ++i) q[i] = r[i];
  }
  __device__ __forceinline__ void decode(int, uint16_t* dst) const {
    uint4* d = reinterpret_cast<uint4*>(dst);
#pragma unroll
    for (int i = 0; i < 8; ++i)
      d[i] = make_uint4(bf2_to_f16x2(q[i].x), bf2_to_f16x2(q[i].y), bf2_to_f16x2(q[i].z), bf2_to_f16x2(q[i].w));
  }
};

// Q6_K (210-byte super-blocks: ql[128] low nibbles, qh[64] 2-bit highs, 16 int8 scales, f16 d).
// Element l + 32 g of half hf (l < 32, g < 4) is d * sc[8 hf + l / 16 + 2 g] * (q - 32), q =
// nibble g / 2 of ql[64 hf + l + 32 (g % 2)] | (bits 2 g, 2 g + 1 of qh[32 hf + l]) << 4. A 64-wide
// K step is g = 2 gp, 2 gp + 1 of one half: its element s takes nibble gp of ql byte 64 hf + s,
// qh byte 32 hf + s % 32 (bits 4 gp + 2 (s / 32)) and scale 8 hf + 4 gp + s / 16. Super-blocks
// start on even bytes only, so each piece is read as the aligned dwords that cover it (never past
// its last byte) and shifted into place by 0 or 2 bytes (alignbyte) at decode.
template <>
struct WRaw<MOE_FMT_Q6_K> {
  uint32_t ql[17], qh[9], sc[2], d, sh;
  __device__ __forceinline__ void load(const uint8_t* row, int k0) {
    const uint8_t* b = row + (size_t)(k0 >> 8) * 210;
    const int q = (k0 >> 6) & 3, hf = q >> 1, gp = q & 1;
    sh = (uint32_t)(reinterpret_cast<uintptr_t>(b) & 3u);        // 0 or 2
    const uint32_t* a = reinterpret_cast<const uint32_t*>(b - sh);
    const int x = sh ? 1 : 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) ql[i] = a[16 * hf + i];
    ql[16] = a[16 * hf + 15 + x];
#pragma unroll
    for (int i = 0; i < 8; ++i) qh[i] = a[32 + 8 * hf + i];
    qh[8] = a[32 + 8 * hf + 7 + x];
    sc[0] = a[48 + 2 * hf + gp];
    sc[1] = a[48 + 2 * hf + gp + x];
    d = *reinterpret_cast<const uint16_t*>(b + 208);
  }
  // 64 f16 in k order into dst (LDS row, 128 B). Four elements at a time: the dword of ql bytes
  // 4i..4i+3 (nibble gp) and the dword of their qh bytes (two bits at 4 gp + 2 (i / 8)) give the
  // four 6-bit q in the bytes of one register (one shift of each, one mask, one and-or); one perm
  // per pair puts two of them under the f16 magic 0x6400 (1024 + q, exact for q <= 63), one packed
  // subtract of 1056 leaves q - 32 exactly and one packed multiply by f16(d * sc) rounds once.
  __device__ __forceinline__ void decode(int k0, uint16_t* dst) const {
    const int gp = (k0 >> 6) & 1;
    const uint32_t scw = __builtin_amdgcn_alignbyte(sc[1], sc[0], sh);
    const float df = f16_to_f32(d);
    const f16x2_t off = {(_Float16)1056.0f, (_Float16)1056.0f};
    uint32_t o[32];
#pragma unroll
    for (int j = 0; j < 4; ++j) {                  // 16 elements of scale j
      const _Float16 dsj = (_Float16)(df * (float)(int8_t)(scw >> (8 * j)));
      const f16x2_t ds = {dsj, dsj};
#pragma unroll
      for (int m = 0; m < 4; ++m) {                // dword i = 4 j + m: elements 4 i .. 4 i + 3
        const int i = 4 * j + m;
        const uint32_t wv = __builtin_amdgcn_alignbyte(ql[i + 1], ql[i], sh);
        const uint32_t hv = __builtin_amdgcn_alignbyte(qh[(i & 7) + 1], qh[i & 7], sh);
        const uint32_t hs = 4u * (uint32_t)gp + 2u * (uint32_t)(i >> 3);
        // the two high bits of each byte to bits 4-5, then the nibble below them
        const uint32_t h30 = (hs >= 4u ? (hv >> (hs - 4u)) : (hv << (4u - hs))) & 0x30303030u;
        const uint32_t q6 = and_or_s(gp ? (wv >> 4) : wv, 0x0F0F0F0Fu, h30);
        const f16x2_t a = __builtin_bit_cast(f16x2_t, __builtin_amdgcn_perm(0x64646464u, q6, 0x04010400u)) - off;
        const f16x2_t b = __builtin_bit_cast(f16x2_t, __builtin_amdgcn_perm(0x64646464u, q6, 0x04030402u)) - off;
        o[2 * i] = __builtin_bit_cast(uint32_t, a * ds);
        o[2 * i + 1] = __builtin_bit_cast(uint32_t, b * ds);
      }
    }
    uint4* dd = reinterpret_cast<uint4*>(dst);
#pragma unroll
    for (int i = 0; i < 8; ++i) dd[i] = make_uint4(o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]);
  }
};

// Q8_0 (the shipped artifact's shared expert, ffn_*_shexp): a 64-wide K step is one pair of
// blocks (f16 d + 32 x int8 each, 68 B, 4-byte aligned in a row of an even block count). Each
// quant becomes an exact f16 through the mantissa trick on its sign-flipped byte (1024 + q + 128
// under 0x6400, minus 1152), and one packed multiply rounds d * q to f16 once.
template <>
struct WRaw<MOE_FMT_Q8_0> {
  uint32_t w[17];
  __device__ __forceinline__ void load(const uint8_t* row, int k0) {
    const uint32_t* p = reinterpret_cast<const uint32_t*>(row + (size_t)(k0 >> 6) * 68);
#pragma unroll
    for (int i = 0; i < 17; ++i) w[i] = p[i];
  }
  __device__ __forceinline__ static void q4(uint32_t q, f16x2_t d, uint32_t& o0, uint32_t& o1) {
    const uint32_t x = q ^ 0x80808080u;
    const f16x2_t off = {(_Float16)1152.0f, (_Float16)1152.0f};
    const f16x2_t a = __builtin_bit_cast(f16x2_t, __builtin_amdgcn_perm(0x64646464u, x, 0x04010400u)) - off;
    const f16x2_t b = __builtin_bit_cast(f16x2_t, __builtin_amdgcn_perm(0x64646464u, x, 0x04030402u)) - off;
    o0 = __builtin_bit_cast(uint32_t, a * d);
    o1 = __builtin_bit_cast(uint32_t, b * d);
  }
  __device__ __forceinline__ void decode(int, uint16_t* dst) const {
    const _Float16 d0 = __builtin_bit_cast(_Float16, (uint16_t)(w[0] & 0xFFFFu));
    const _Float16 d1 = __builtin_bit_cast(_Float16, (uint16_t)(w[8] >> 16));
    uint32_t o[32];
#pragma unroll
    for (int m = 0; m < 8; ++m) q4(__builtin_amdgcn_alignbyte(w[m + 1], w[m], 2), (f16x2_t){d0, d0}, o[2 * m], o[2 * m + 1]);
#pragma unroll
    for (int m = 0; m < 8; ++m) q4(w[9 + m], (f16x2_t){d1, d1}, o[16 + 2 * m], o[17 + 2 * m]);
    uint4* d = reinterpret_cast<uint4*>(dst);
#pragma unroll
    for (int i = 0; i < 8; ++i) d[i] = make_uint4(o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]);
  }
};

__device__ __forceinline__ size_t row_bytes(int fmt, int cols) {
  return fmt == MOE_FMT_Q4_K ? (size_t)(cols / 256) * 144
       : fmt == MOE_FMT_Q5_K ? (size_t)(cols / 256) * 176
       : fmt == MOE_FMT_Q6_K ? (size_t)(cols / 256) * 210
       : fmt == MOE_FMT_Q8_0 ? (size_t)(cols / 32) * 34 : (size_t)cols * 2;
}

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

struct Smem {
  uint16_t A[2][kBM * kS];              // 2 x 22.5 KB
  uint16_t B[2][kBN * kS];              // 2 x 36 KB
};

// Activation rows of one producer thread p (0..255): 16-byte chunk p & 7 of rows (p >> 3) + 32 i,
// i < kMG (pointers to the row starts; rows past the tile repeat its last row, never stored).
struct ARows {
  const uint16_t* r[kMG];
};

// Producer thread p: weight row p of the slab (one 64-wide K step = 64 elements) and the
// activation chunks of ARows. kD sets of raw registers form a ring indexed at compile time.
template <int WFMT>
struct PSet {
  WRaw<WFMT> w;
  uint4 a[kMG];
  __device__ __forceinline__ void load(const uint8_t* wrow, const ARows& ar, int k0, int p) {
    w.load(wrow, k0);
#pragma unroll
    for (int i = 0; i < kMG; ++i) a[i] = *reinterpret_cast<const uint4*>(ar.r[i] + k0 + 8 * (p & 7));
  }
  __device__ __forceinline__ void store(int k0, int p, uint16_t* As, uint16_t* Bs) const {
    w.decode(k0, Bs + p * kS);
#pragma unroll
    for (int i = 0; i < kMG; ++i)
      *reinterpret_cast<uint4*>(As + ((p >> 3) + 32 * i) * kS + 8 * (p & 7)) = a[i];
  }
};

// Producer ring of kD register sets: at step ks the consumers read LDS buffer ks & 1, the producer
// stores step ks + 1 (set (ks + 1) % kD) into the other buffer and requests step ks + kD into the
// set it just freed, so each request has kD - 1 steps to land. kD is even and divides the step
// count (H / 64 = 32 for gate_up, I / 64 = 8 for down), so set and buffer indices are compile-time.
// Q4_K sets are 28 registers and Q5_K 40 (4 deep); bf16 sets 48 and Q6_K 50 (2 deep, within the
// 256-register budget).
template <int WFMT>
__device__ __forceinline__ void produce(int nk, const ARows& asrc, const uint8_t* wrow, int p,
                                        Smem& sm) {
  constexpr int kD = (WFMT == MOE_FMT_BF16 || WFMT == MOE_FMT_Q8_0 || WFMT == MOE_FMT_Q6_K) ? 2 : 4;
  PSet<WFMT> s[kD];
#pragma unroll
  for (int i = 0; i < kD; ++i) s[i].load(wrow, asrc, min(i, nk - 1) * kBK, p);
  s[0].store(0, p, sm.A[0], sm.B[0]);
  __syncthreads();
  for (int k0 = 0; k0 < nk; k0 += kD) {
#pragma unroll
    for (int j = 0; j < kD; ++j) {
      const int ks = k0 + j;
      s[(j + 1) % kD].store(min(ks + 1, nk - 1) * kBK, p, sm.A[(j + 1) & 1], sm.B[(j + 1) & 1]);
      s[j].load(wrow, asrc, min(ks + kD, nk - 1) * kBK, p);
      __syncthreads();
    }
  }
}

__device__ __forceinline__ uint4 frag(const uint16_t* S, int row, int s, int lane) {
  return *reinterpret_cast<const uint4*>(S + row * kS + 16 * s + 8 * (lane >> 5));
}

// Consumer wave c (0..3): all 128 rows (NG active 32-row groups) x B rows {b0 + lane%32} and
// {b1 + lane%32} of the slab.
template <int NG>
__device__ __forceinline__ void consume(int nk, int b0, int b1, Smem& sm, f32x16_t (&acc)[kMG][2]) {
  const int lane = threadIdx.x & 63;
  __syncthreads();
  for (int k2 = 0; k2 < nk; k2 += 2) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint16_t* As = sm.A[j];
      const uint16_t* Bs = sm.B[j];
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const uint4 bg = frag(Bs, b0 + (lane & 31), s, lane);
        const uint4 bu = frag(Bs, b1 + (lane & 31), s, lane);
#pragma unroll
        for (int mg = 0; mg < NG; ++mg) {
          const uint4 a = frag(As, 32 * mg + (lane & 31), s, lane);
          acc[mg][0] = mfma(a, bg, acc[mg][0]);
          acc[mg][1] = mfma(a, bu, acc[mg][1]);
        }
      }
      __syncthreads();
    }
  }
}

template <int NG>
__device__ __forceinline__ void consume_n(int ng, int nk, int b0, int b1, Smem& sm,
                                          f32x16_t (&acc)[kMG][2]) {
  (void)NG;
  if (ng >= 5) consume<5>(nk, b0, b1, sm, acc);
  else if (ng == 4) consume<4>(nk, b0, b1, sm, acc);
  else if (ng == 3) consume<3>(nk, b0, b1, sm, acc);
  else if (ng == 2) consume<2>(nk, b0, b1, sm, acc);
  else consume<1>(nk, b0, b1, sm, acc);
}

}  // namespace g3

// ----------------------------------------------------------------------------------- gate/up --
template <int WFMT>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_gemm3_gateup(
    const uint16_t* __restrict__ x16, const uint8_t* __restrict__ wg, const uint8_t* __restrict__ wu,
    size_t estride, const int32_t* __restrict__ tiles, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ sorted_pairs, int K, int H, int I, int T,
    uint16_t* __restrict__ S) {
  using namespace g3;
  __shared__ __attribute__((aligned(16))) Smem sm;
  int e, m0, mend, col;
  if (!tile_rows(tiles, offsets, T, I / 128, e, m0, mend, col)) return;
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int nk = H / kBK;
  if (wave >= 4) {
    const int p = t - 256;
    ARows ar;
#pragma unroll
    for (int i = 0; i < kMG; ++i) {
      const int m = min(m0 + (p >> 3) + 32 * i, mend - 1);
      ar.r[i] = x16 + (size_t)(tiles ? sorted_pairs[m] / K : m) * H;
    }
    const int r = p & 127;
    const uint8_t* wrow = (p < 128 ? wg : wu) + (size_t)e * estride +
                          (size_t)(col * 128 + r) * row_bytes(WFMT, H);
    produce<WFMT>(nk, ar, wrow, p, sm);
    return;
  }
  f32x16_t acc[kMG][2];
#pragma unroll
  for (int mg = 0; mg < kMG; ++mg) { acc[mg][0] = (f32x16_t){}; acc[mg][1] = (f32x16_t){}; }
  const int ng = __builtin_amdgcn_readfirstlane((mend - m0 + 31) >> 5);
  consume_n<0>(ng, nk, 32 * wave, 128 + 32 * wave, sm, acc);
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
// Y16: rows out as f16 (saturated to +-65504) instead of f32
template <int WFMT, bool Y16>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_gemm3_down(
    const uint16_t* __restrict__ S, const uint8_t* __restrict__ wd, size_t estride,
    const int32_t* __restrict__ tiles, const int32_t* __restrict__ offsets, int H, int I, int T,
    void* __restrict__ y) {
  using namespace g3;
  __shared__ __attribute__((aligned(16))) Smem sm;
  int e, m0, mend, col;
  if (!tile_rows(tiles, offsets, T, H / kBN, e, m0, mend, col)) return;
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int nk = I / kBK;
  if (wave >= 4) {
    const int p = t - 256;
    ARows ar;
#pragma unroll
    for (int i = 0; i < kMG; ++i) ar.r[i] = S + (size_t)min(m0 + (p >> 3) + 32 * i, mend - 1) * I;
    const uint8_t* wrow = wd + (size_t)e * estride + (size_t)(col * kBN + p) * row_bytes(WFMT, I);
    produce<WFMT>(nk, ar, wrow, p, sm);
    return;
  }
  f32x16_t acc[kMG][2];
#pragma unroll
  for (int mg = 0; mg < kMG; ++mg) { acc[mg][0] = (f32x16_t){}; acc[mg][1] = (f32x16_t){}; }
  const int ng = __builtin_amdgcn_readfirstlane((mend - m0 + 31) >> 5);
  consume_n<0>(ng, nk, 64 * wave, 64 * wave + 32, sm, acc);
  const int nb = col * kBN + 64 * wave + (lane & 31), h = lane >> 5;
#pragma unroll
  for (int mg = 0; mg < kMG; ++mg) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int mm = m0 + 32 * mg + 8 * (r >> 2) + 4 * h + (r & 3);
      if (mm < mend) {
        const float v0 = acc[mg][0][r], v1 = acc[mg][1][r];
        if constexpr (Y16) {
          uint16_t* yh = reinterpret_cast<uint16_t*>(y) + (size_t)mm * H + nb;
          yh[0] = __builtin_bit_cast(uint16_t, (_Float16)fminf(fmaxf(v0, -65504.0f), 65504.0f));
          yh[32] = __builtin_bit_cast(uint16_t, (_Float16)fminf(fmaxf(v1, -65504.0f), 65504.0f));
        } else {
          float* yf = reinterpret_cast<float*>(y) + (size_t)mm * H + nb;
          yf[0] = v0;
          yf[32] = v1;
        }
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

bool moe_gemm3_supports(int fmt) { return fmt == MOE_FMT_Q4_K || fmt == MOE_FMT_BF16; }
bool moe_gemm3_down_supports(int fmt) {
  return fmt == MOE_FMT_Q4_K || fmt == MOE_FMT_Q5_K || fmt == MOE_FMT_Q6_K || fmt == MOE_FMT_BF16;
}

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


int moe_launch_gemm3_gateup(const uint16_t* x16, const void* w_gate, const void* w_up, int fmt,
                            size_t expert_stride, const int32_t* tiles, int max_tiles, int T,
                            const int32_t* offsets, const int32_t* sorted_pairs, int K, int H,
                            int I, uint16_t* S, hipStream_t st) {
  if (H % 256 || I % 128)
    return moe_set_error(MOE_E_UNSUPPORTED, "gemm3 gate_up needs H %% 256 == 0, I %% 128 == 0");
  const uint8_t* g = reinterpret_cast<const uint8_t*>(w_gate);
  const uint8_t* u = reinterpret_cast<const uint8_t*>(w_up);
  const int ntile = tiles ? max_tiles : (T + g3::kBM - 1) / g3::kBM;
  const dim3 grid(g3::kXcd * ((ntile + g3::kXcd - 1) / g3::kXcd) * (I / 128));
  if (fmt == MOE_FMT_Q4_K)
    hipLaunchKernelGGL(k_gemm3_gateup<MOE_FMT_Q4_K>, grid, dim3(512), 0, st, x16, g, u, expert_stride, tiles, offsets, sorted_pairs, K, H, I, T, S);
  else if (fmt == MOE_FMT_BF16)
    hipLaunchKernelGGL(k_gemm3_gateup<MOE_FMT_BF16>, grid, dim3(512), 0, st, x16, g, u, expert_stride, tiles, offsets, sorted_pairs, K, H, I, T, S);
  else if (fmt == MOE_FMT_Q8_0)
    hipLaunchKernelGGL(k_gemm3_gateup<MOE_FMT_Q8_0>, grid, dim3(512), 0, st, x16, g, u, expert_stride, tiles, offsets, sorted_pairs, K, H, I, T, S);
  else
    return moe_set_error(MOE_E_FORMAT, "gemm3 gate_up: unsupported format %d", fmt);
  return moe_check_launch("gemm3_gateup");
}

int moe_launch_gemm3_down(const uint16_t* S, const void* w_down, int fmt, size_t expert_stride,
                          const int32_t* tiles, int max_tiles, int T, const int32_t* offsets,
                          int H, int I, void* y, int y16, hipStream_t st) {
  if (H % g3::kBN || I % 256)
    return moe_set_error(MOE_E_UNSUPPORTED, "gemm3 down needs H %% 256 == 0, I %% 256 == 0");
  const uint8_t* w = reinterpret_cast<const uint8_t*>(w_down);
  const int ntile = tiles ? max_tiles : (T + g3::kBM - 1) / g3::kBM;
  const dim3 grid(g3::kXcd * ((ntile + g3::kXcd - 1) / g3::kXcd) * (H / g3::kBN));
#define MOE_G3D(F)                                                                                 \
  do {                                                                                             \
    if (y16) hipLaunchKernelGGL((k_gemm3_down<F, true>), grid, dim3(512), 0, st, S, w, expert_stride, tiles, offsets, H, I, T, y); \
    else hipLaunchKernelGGL((k_gemm3_down<F, false>), grid, dim3(512), 0, st, S, w, expert_stride, tiles, offsets, H, I, T, y);    \
  } while (0)
  if (fmt == MOE_FMT_Q4_K) MOE_G3D(MOE_FMT_Q4_K);
  else if (fmt == MOE_FMT_Q5_K) MOE_G3D(MOE_FMT_Q5_K);
  else if (fmt == MOE_FMT_Q6_K) MOE_G3D(MOE_FMT_Q6_K);
  else if (fmt == MOE_FMT_BF16) MOE_G3D(MOE_FMT_BF16);
  else if (fmt == MOE_FMT_Q8_0) MOE_G3D(MOE_FMT_Q8_0);
  else return moe_set_error(MOE_E_FORMAT, "gemm3 down: unsupported format %d", fmt);
#undef MOE_G3D
  return moe_check_launch("gemm3_down");
}
