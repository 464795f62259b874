// Single-token decode of one MoE block in ONE launch, laid out over the 8 XCDs of an MI355X.
//
// A persistent grid of 256 workgroups of 8 waves (one per CU; the LDS footprint keeps it at one,
// so every XCD holds exactly 32) runs the block's dependent phases and hands data between them
// through self-validating exchange words. A workgroup's role is (x, r) = (blockIdx mod 8,
// blockIdx / 8): the dispatcher hands a launch's workgroups to the 8 XCDs round robin, workgroup
// b to XCD (b + c) mod 8 with one offset c per launch (c is 0 or 7 depending on the hardware
// queue; measured over 4000 launches, eager, graph-replayed and alternating between streams, with
// other kernels of odd grids in between), so the 32 workgroups of role group x share one XCD and
// the role costs no memory round trip: the weights it selects are requested at entry. ("XCD x"
// below is the XCD that role group x runs on.) Were the placement ever different, the XCD-local
// exchanges below would time out and record the spin error bit rather than hang.
// XCD x owns routed slot k = x and the 64-wide slice [64x, 64x+64) of the shared expert's
// intermediate axis, so two of the three exchanges stay among the 32 workgroups of one XCD:
//
//   start    stage x in LDS, RMS-normalized when a post-attention norm weight is given (Form A,
//            engine/m3_forward.py:303-307; f64 sum of squares, one rounding)
//   phase 1  wg (x, r): router logits e in [8r, 8r+8) (one wave each; f64, certified bf16), so
//            each XCD computes all 256 logits itself | shared gate/up rows i = 64x + 2r (+1) |
//            the scalar shared gate p (every workgroup, for its own combine rows)
//   phase 2  wait for the XCD's 256 logits; the top-8 set from the logits alone (same answer
//            everywhere; slots in ascending expert id), with the exact selection where the 8th and
//            9th logits are (nearly) equal; routed gate/up rows of slot x, i in [16r, 16r+16), its
//            down rows requested ahead of use; R2-R5 weights by wave 3 while its rows are in flight;
//            shared-down partial over the XCD's 64 i-values for rows h in [64r, 64r+64)
//   phase 3  wait for slot x's 512 activations (XCD-local); down rows h in [64r, 64r+64) (Q4_K, Q5_K
//            rows on the activations' int8 digit planes)
//   phase 4  wg (x, r) combines rows [8j, 8j+8), j = 32x + r: the 8 slots' outputs in ascending
//            expert id, the 8 shared-down partials in ascending x, gate, residual
//   (hint)   with the next layer's weights named, waves 4-7 read the router rows and the norm
//            weight that role (x, r) will need first into XCD x's L2 while phase 4 waits
//
// Exchange words are 32-bit: a value is stored as the complement of its bit pattern (NaNs made
// canonical first), so 0 never encodes a value and means "not written yet". Each word is written
// once per launch by one dword store and polled 16 bytes at a time; a reader re-polls all of its
// missing words in parallel until every word it needs is non-zero. Words that cross XCDs (expert
// outputs, shared-down partials) go past the XCDs' non-coherent L2s (agent-scope relaxed atomic
// stores and loads, sc1); words read only inside one XCD (logits, shared and routed activations)
// use non-temporal stores and loads, which meet in that XCD's L2 and take half the round trip.
// Exchange latency grows with the number of workgroups reading the same lines, which is why no
// region here has more than 32 readers. Two buffers alternate by the launch's epoch parity, and each launch zeroes the buffer
// the next launch will use, so a zeroed workspace is a valid starting state and graph replays
// work. The launch count (epoch) is kept per role: the one workgroup of role (x, r) reads its word
// at entry (the read overlaps the x and weight loads; the parity is first used at the logit
// store) and writes it back incremented at the end, so no launch starts or ends on a contended
// atomic. Every spin is bounded: on a timeout the workgroup records an error bit and carries on
// (no hang).
#include <atomic>
#include <mutex>

#include "common.h"
#include "moe_internal.h"
#include "router_dev.h"
#include "gemv_dev.h"

namespace moe {

constexpr int kXcd = 8;                 // XCDs on MI355X
constexpr int kPer = 32;                // workgroups (CUs) per XCD
constexpr int kG = kXcd * kPer;         // 256 workgroups
constexpr int kThreads = 512;           // 8 waves
constexpr int kSpinLimit = 1 << 20;     // polls (each a memory round trip) before giving up
constexpr int kOccPad = 5120;           // uint4s of LDS that keep the grid at one workgroup per CU
// sync words (int32 index into the workspace's first kSyncBytes)
constexpr int kErrWord = MOE_STATUS_WORD;   // status bits (moe_workspace_status)
constexpr int kHookWord = MOE_TEST_HOOK_WORD; // test hook: non-zero = every wait reports a timeout
constexpr int kRoleEpoch = 114688;      // [xcd][kPer]: launches run by role (x, r), past the exchange

// status bits (sync word kErrWord)
constexpr int kErrSpin = MOE_STATUS_SPIN_TIMEOUT;   // a bounded wait timed out

// What a bounded wait does when it gives up: the status bit for the caller, and this workgroup's
// LDS flag, which poisons the output rows the workgroup writes (NaN) at the end. With the test
// hook set, every wait completes as usual and then reports a timeout, so the reporting path runs
// on valid data and every workgroup still exits normally.
struct Spin {
  int* err;       // the workspace's status word
  int* bad;       // this workgroup's flag (LDS)
  int force;      // the test hook's value
  __device__ __forceinline__ void give_up() const {
    atomicOr(err, kErrSpin);
    *bad = 1;
  }
  // called after each wait: report a forced timeout
  __device__ __forceinline__ void done() const {
    if (force) give_up();
  }
};

struct LayerArgs {
  const void* x;
  const float* residual;
  const void* w_router;                 // bf16 or f32 rows (the kernel's RDT)
  const float* bias;
  const uint8_t* gu;                    // gate rows of expert e at gu + e * gu_estride
  const uint8_t* gu_up;                 // up rows likewise (a fused record: gu + I rows)
  size_t gu_estride;
  const uint8_t* dn;
  const uint16_t* sg;
  const uint16_t* su;
  const uint16_t* sd;
  const uint16_t* ssg;                  // the scalar gate row: bf16, or f32 when ssg_f32
  int ssg_f32;
  int* sync;                            // sync words (kErrWord, kRoleEpoch)
  uint32_t* xch;                        // two exchange buffers of XW_BUF words
  uint16_t* logits_out;
  int32_t* ids_out;
  float* w_f32_out;
  uint16_t* w_bf16_out;
  float* gate_prob_out;
  float* out;
  float* routed_sum;
  float* shared_out;
  float* expert_raw;
  int exact_order;                      // stage outputs requested: keep torch's slot order
  const float* norm_w;                  // post-attention RMSNorm weight [H] f32, or NULL
  float norm_eps;
  // the next layer's router weight and norm weight (L2 warm-up hint), or NULL
  const uint16_t* nx_router;
  int nx_router_f32;                    // the next layer's router rows are f32 (twice the bytes)
  const float* nx_norm;
};

// exchange buffer layout (uint32 words; every region starts 16-byte aligned)
constexpr int XW_LOG = 0;                       // [xcd][256] router logits (bf16 bits)
constexpr int XW_SSH = XW_LOG + kXcd * 256;     // [xcd][64] shared activations of the xcd's slice
constexpr int XW_SR = XW_SSH + kXcd * 64;       // [slot][512] routed activations
constexpr int XW_Y = XW_SR + kXcd * 512;        // [slot][2048] routed expert outputs
constexpr int XW_SHP = XW_Y + kXcd * 2048;      // [xcd][2048] shared-down partial sums
constexpr int XW_BUF = XW_SHP + kXcd * 2048;    // words per buffer
constexpr int kClearPerWg = (XW_BUF + kG - 1) / kG;

__device__ const float kZeroBias = 0.0f;  // the logit bias of a router without one

__device__ __forceinline__ int aload(const int* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void astore(int* p, int v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint32_t xenc(float v) {
  const uint32_t b = (v != v) ? 0x7FC00000u : __float_as_uint(v);
  return ~b;
}
__device__ __forceinline__ float xdec(uint32_t w) { return __uint_as_float(~w); }

__device__ __forceinline__ void xstore(uint32_t* p, uint32_t w) {
  __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t xload(uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// 16 bytes at byte offset `off` of the buffer, read past the non-coherent L2 (sc1)
__device__ __forceinline__ uint4 xload4(__amdgpu_buffer_rsrc_t r, int off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 16);
  return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ bool xfull(uint4 v) { return v.x && v.y && v.z && v.w; }

// ----------------------------------------------------- activation digit planes (down rows) --
// The Q4_K and Q5_K down rows' dot products (phase 3, right after the slot activations arrive)
// run on v_dot4_i32_i8: 1.1 VALU operations per weight instead of 2.25 (a byte convert and an f32
// FMA per nibble), which took 0.4 us off the launch. The activations of each 16-element group
// become three balanced base-256 digit planes: with e the group's exponent (every |v| < 2^e; 0 for
// an all-zero group), N = rint(v 2^(22-e)) is an integer with |N| <= 2^22, and
// N = 65536 D0 + 256 D1 + D2 with D1, D2 in [-128, 127] and |D0| <= 64. For the 16 quants q of a
// sub-block, sum q v = 2^(e-22) (65536 S0 + 256 S1 + S2) + err, where S_p = sum q D_p is exact in
// int32 (the combination stays below 2^31) and |err| <= 8 qmax 2^(e-22) (half a unit of N per
// element; qmax = 15 for Q4_K, 31 for Q5_K), the order of an f32 multiply-add chain over the
// group. The min term uses the group's float sum, so a NaN or infinite activation still reaches
// the output.
// digits of 4 consecutive values: byte i of dword p holds D_p of value i
__device__ __forceinline__ void digits4(const float (&v)[4], int e, uint32_t (&w)[3]) {
  w[0] = w[1] = w[2] = 0u;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int n = (int)rintf(ldexpf(v[i], 22 - e));
    const int d2 = (int)(int8_t)(n & 0xFF);
    const int n1 = (n - d2) / 256;
    const int d1 = (int)(int8_t)(n1 & 0xFF);
    const int d0 = (n1 - d1) / 256;
    w[0] |= (uint32_t)(d0 & 0xFF) << (8 * i);
    w[1] |= (uint32_t)(d1 & 0xFF) << (8 * i);
    w[2] |= (uint32_t)(d2 & 0xFF) << (8 * i);
  }
}
// exponent e of a group whose largest magnitude is m: m < 2^e (frexp's exponent; 0 for m = 0)
__device__ __forceinline__ int group_exp(float m) {
  int e;
  (void)frexpf(m, &e);
  return e;
}
// The K-quant chunk dot on digit planes: the lane's 16-byte chunk covers sub-blocks 2g (its low
// nibbles) and 2g+1 (high nibbles); lo[i] / hi[i] hold the q values of elements 4i .. 4i+3 of the
// two sub-blocks as bytes (Q4_K: the nibbles; Q5_K: with the 5th bit at bit 4, q <= 31, so the
// combination 65536 S0 + 256 S1 + S2 stays below 2^31). zl / zh are the planes of the two
// activation groups (exponents el / eh, float sums sl / sh for the min terms); the 6-bit scales
// as in q4k_chunk_dot (gemv_dev.h).
__device__ __forceinline__ float kquant_chunk_dot_dig(uint4 hdr, const uint32_t (&lo)[4],
                                                      const uint32_t (&hi)[4], int g,
                                                      const uint4 (&zl)[3], const uint4 (&zh)[3],
                                                      int el, int eh, float sl, float sh) {
  const float d = f16_to_f32(hdr.x & 0xFFFFu), dmin = f16_to_f32(hdr.x >> 16);
  const uint32_t sh0 = 16u * (uint32_t)(g & 1), sh1 = sh0 + 8u;
  const uint32_t low = 0u - (uint32_t)(g < 2);
  const uint32_t y0 = hdr.y >> sh0, z0 = hdr.z >> sh0, w0 = hdr.w >> sh0;
  const uint32_t y1 = hdr.y >> sh1, z1 = hdr.z >> sh1, w1 = hdr.w >> sh1;
  const uint32_t sc0 = ((y0 & 63u) & low) | (((w0 & 15u) | ((y0 >> 2) & 48u)) & ~low);
  const uint32_t m0 = ((z0 & 63u) & low) | ((((w0 >> 4) & 15u) | ((z0 >> 2) & 48u)) & ~low);
  const uint32_t sc1 = ((y1 & 63u) & low) | (((w1 & 15u) | ((y1 >> 2) & 48u)) & ~low);
  const uint32_t m1 = ((z1 & 63u) & low) | ((((w1 >> 4) & 15u) | ((z1 >> 2) & 48u)) & ~low);
  int s[2][3] = {{0, 0, 0}, {0, 0, 0}};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int p = 0; p < 3; ++p) {
      const uint32_t al[4] = {zl[p].x, zl[p].y, zl[p].z, zl[p].w};
      const uint32_t ah[4] = {zh[p].x, zh[p].y, zh[p].z, zh[p].w};
      s[0][p] = __builtin_amdgcn_sdot4((int)lo[i], (int)al[i], s[0][p], false);
      s[1][p] = __builtin_amdgcn_sdot4((int)hi[i], (int)ah[i], s[1][p], false);
    }
  }
  const float fl = ldexpf((float)(s[0][0] * 65536 + s[0][1] * 256 + s[0][2]), el - 22);
  const float fh = ldexpf((float)(s[1][0] * 65536 + s[1][1] * 256 + s[1][2]), eh - 22);
  return d * ((float)sc0 * fl + (float)sc1 * fh) - dmin * ((float)m0 * sl + (float)m1 * sh);
}
// the q bytes of a Q4_K chunk (qs) and of a Q5_K chunk (qs and the qh bytes of its element
// positions, the 5th bits placed as in q5k_chunk_dot)
__device__ __forceinline__ void q4k_bytes(uint4 qs, uint32_t (&lo)[4], uint32_t (&hi)[4]) {
  const uint32_t w[4] = {qs.x, qs.y, qs.z, qs.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    lo[i] = and_opaque(w[i], 0x0F0F0F0Fu);
    hi[i] = and_opaque(w[i] >> 4, 0x0F0F0F0Fu);
  }
}
__device__ __forceinline__ void q5k_bytes(uint4 qs, uint4 qh, int g, uint32_t (&lo)[4], uint32_t (&hi)[4]) {
  const uint32_t w[4] = {qs.x, qs.y, qs.z, qs.w};
  const uint32_t h[4] = {qh.x, qh.y, qh.z, qh.w};
  const uint32_t hs = 2u * (uint32_t)g;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t hb = h[i] >> hs;
    lo[i] = and_opaque(w[i], 0x0F0F0F0Fu) | ((hb << 4) & 0x10101010u);
    hi[i] = and_opaque(w[i] >> 4, 0x0F0F0F0Fu) | ((hb << 3) & 0x10101010u);
  }
}

// one 16-byte group at byte offset `off` of the buffer, same protocol
__device__ __forceinline__ uint4 xwait4(__amdgpu_buffer_rsrc_t r, int off, const Spin& sp) {
  uint4 v = xload4(r, off);
  for (int spins = 0; !xfull(v); ++spins) {
    if (spins >= kSpinLimit) { sp.give_up(); break; }
    __builtin_amdgcn_s_sleep(1);
    v = xload4(r, off);
  }
  sp.done();
  return v;
}

// R1 for one router row held by a wave: w[c] = W[e, 512c + 8 lane .. +8), xd[c] = the matching x
// in f64. The correctly rounded bf16 of sum + bias: f64 sum (every product x_j w_j is exact in
// f64) with the certified error bound 4(H+3) 2^-53 (|x|_2 |w|_2 + |b|), which by Cauchy-Schwarz
// bounds sum |x_j w_j| + |b| times the summation's error factor; a double-double recompute
// settles what that does not. xl2 >= |x|_2 is the workgroup's bound on the input's 2-norm; |w|_2
// comes from an f32 sum of squares (one FMA per weight, where a running maximum of |w| took two
// operations; its rounding stays below 40 * 2^-24 of the sum) raised by 2^-15 before an f32 square
// root, whose result is raised by 2^-20 (more than its error) and taken to f64.
// Weight i (0..7) of chunk c of the row a lane holds: bf16 rows take one uint4 per chunk, f32
// rows two (w[2c], w[2c + 1]); either way x_j w_j is exact in f64.
template <int RDT>
__device__ __forceinline__ float router_w(const uint4* w, int c, int i) {
  if (RDT == MOE_DT_F32) {
    const uint4 v = w[2 * c + (i >> 2)];
    const uint32_t u[4] = {v.x, v.y, v.z, v.w};
    return __uint_as_float(u[i & 3]);
  }
  const uint32_t u[4] = {w[c].x, w[c].y, w[c].z, w[c].w};
  return bf16_to_f32((i & 1) ? (u[i >> 1] >> 16) : (u[i >> 1] & 0xFFFFu));
}

template <int RDT>
__device__ __forceinline__ uint32_t router_row_bits(const uint4* w, const double (*xd)[8],
                                                   double bval, double xl2) {
  constexpr int H = 2048;
  double acc = 0.0;
  float wsq = 0.0f;                      // sum of w^2 (f32)
#pragma unroll
  for (int c = 0; c < 4; ++c) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float wv = router_w<RDT>(w, c, i);
      acc = fma(xd[c][i], (double)wv, acc);
      wsq = fmaf(wv, wv, wsq);
    }
  }
  acc = wave_sum_f64_v(acc);
  wsq = wave_sum_f32_v(wsq);
  const double nrm = xl2 * (double)__builtin_sqrtf(wsq * (1.0f + 0x1p-15f)) * (1.0 + 0x1p-20) + fabs(bval);
  uint32_t bits;
  if (!round_bf16_certified(acc + bval, 4.0 * (double)(H + 3) * 0x1p-53 * nrm, &bits)) {
    DD d = {0.0, 0.0};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
#pragma unroll
      for (int i = 0; i < 8; ++i) d = dd_add(d, DD{xd[c][i] * (double)router_w<RDT>(w, c, i), 0.0});
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      DD other = {__shfl_xor(d.hi, o, 64), __shfl_xor(d.lo, o, 64)};
      d = dd_add(d, other);
    }
    d = dd_add(d, DD{bval, 0.0});
    bits = round_bf16_dd(d, (double)(H + 64) * 0x1p-104 * 16.0 * nrm);
  }
  return bits;
}

__device__ __forceinline__ uint32_t xor4(uint4 v) { return v.x ^ v.y ^ v.z ^ v.w; }

// XCD-local exchange words: written and read only by the workgroups of one XCD, through that
// XCD's L2 (non-temporal stores and loads: the L2 is coherent among its CUs, and the CU's own L1
// is not consulted), which halves the round trip of the agent-scope (MALL) words.
__device__ __forceinline__ void lstore(__amdgpu_buffer_rsrc_t r, int off, uint32_t w) {
  __builtin_amdgcn_raw_buffer_store_b32(w, r, off, 0, 2);
}
__device__ __forceinline__ uint32_t lload(__amdgpu_buffer_rsrc_t r, int off) {
  asm volatile("" ::: "memory");
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 2);
}
__device__ __forceinline__ uint4 lload4(__amdgpu_buffer_rsrc_t r, int off) {
  asm volatile("" ::: "memory");
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2);
  return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ uint4 lwait4(__amdgpu_buffer_rsrc_t r, int off, const Spin& sp) {
  uint4 v = lload4(r, off);
  for (int spins = 0; !xfull(v); ++spins) {
    if (spins >= kSpinLimit) { sp.give_up(); break; }
    __builtin_amdgcn_s_sleep(1);
    v = lload4(r, off);
  }
  sp.done();
  return v;
}

// maximum over the wave, in every lane (DPP maxima inside each 16-lane row, then the four rows)
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, dpp_u32<0xB1>(v));
  v = max(v, dpp_u32<0x4E>(v));
  v = max(v, dpp_u32<0x141>(v));
  v = max(v, dpp_u32<0x140>(v));
  return max(max((uint32_t)__builtin_amdgcn_readlane((int)v, 15), (uint32_t)__builtin_amdgcn_readlane((int)v, 31)),
             max((uint32_t)__builtin_amdgcn_readlane((int)v, 47), (uint32_t)__builtin_amdgcn_readlane((int)v, 63)));
}
// bf16 bits <-> a 16-bit key with the same order as the values (no NaNs on this path)
__device__ __forceinline__ uint32_t bf16_key(uint32_t b) { return (b & 0x8000u) ? (~b & 0xFFFFu) : (b | 0x8000u); }
__device__ __forceinline__ uint32_t bf16_unkey(uint32_t k) { return (k & 0x8000u) ? (k & 0x7FFFu) : (~k & 0xFFFFu); }

// R2-R5 for one token, by one wave holding the 256 logits' bf16 bits lb[q] of experts lane + 64q.
// The 9 largest logits are found on 24-bit keys (value key << 8 | 255 - id: distinct, and the
// logit order is the probability order, since p = exp(l - max) / sum is monotone); their
// probabilities p_r = f32(exp(l_r - max)) * (1 / sum) are the softmax's own values (R2: the full
// sum of 256 exps, as route_softmax). Without two equal probabilities among the first 9 the
// selection is torch's; with equal ones only inside the first 8 it is torch's up to slot order
// (same experts, same weights), accepted when exact_order is false. Otherwise returns false and
// leaves the full probabilities in p for the exact replay. On success lanes < K write ids, w_f32
// (p_r / sum of the 8 in rank order) and w_bf16.
template <int K>
__device__ __forceinline__ bool wave_route_keys(const uint32_t* lb, int lane, bool exact_order,
                                                float* p, int* ids, float* wf, uint16_t* wb) {
  uint32_t k0 = (bf16_key(lb[0]) << 8) | (uint32_t)(255 - lane);
  uint32_t k1 = (bf16_key(lb[1]) << 8) | (uint32_t)(191 - lane);
  uint32_t k2 = (bf16_key(lb[2]) << 8) | (uint32_t)(127 - lane);
  uint32_t k3 = (bf16_key(lb[3]) << 8) | (uint32_t)(63 - lane);
  {
    // each lane's four keys, descending
    uint32_t a = max(k0, k1), b = min(k0, k1), c = max(k2, k3), d = min(k2, k3);
    k0 = max(a, c); const uint32_t t1 = min(a, c);
    k3 = min(b, d); const uint32_t t2 = max(b, d);
    k1 = max(t1, t2); k2 = min(t1, t2);
  }
  uint32_t top[K + 1];
  top[0] = wave_max_u32(k0);
  if (k0 == top[0]) { k0 = k1; k1 = k2; k2 = k3; k3 = 0u; }
  const float m = bf16_to_f32(bf16_unkey(top[0] >> 8));
  float sum = 0.0f;
#pragma unroll
  for (int q = 0; q < 4; ++q) { p[q] = r2_exp(bf16_to_f32(lb[q]) - m); sum += p[q]; }
#pragma unroll
  for (int r = 1; r <= K; ++r) {
    top[r] = wave_max_u32(k0);
    if (k0 == top[r]) { k0 = k1; k1 = k2; k2 = k3; k3 = 0u; }
  }
  sum = wave_sum_f32(sum);
  const float rs = 1.0f / sum;
#pragma unroll
  for (int q = 0; q < 4; ++q) p[q] *= rs;
  uint32_t mine = top[0];
#pragma unroll
  for (int r = 1; r <= K; ++r) mine = lane == r ? top[r] : mine;
  const float ps = r2_exp(bf16_to_f32(bf16_unkey(mine >> 8)) - m) * rs;
  const float nxt = __uint_as_float((uint32_t)__builtin_amdgcn_update_dpp(0, (int)__float_as_uint(ps), 0x101, 0xF, 0xF, false));
  const uint64_t ties = __ballot(lane < K && ps == nxt);       // p_r == p_{r+1}, r < K
  if (((ties >> (K - 1)) & 1ull) || (ties && exact_order)) return false;
  float tot = 0.0f;
#pragma unroll
  for (int r = 0; r < K; ++r) tot += readlane_f32(ps, r);
  if (lane < K) {
    const float wv = ps / tot;
    ids[lane] = 255 - (int)(mine & 255u);
    wf[lane] = wv;
    wb[lane] = (uint16_t)f32_to_bf16(wv);
  }
  return true;
}

// The top-K set of one token's 256 logits (bf16 bits lb[q] of expert lane + 64q; no NaNs), for
// the expert loads, without the probabilities: K + 1 rounds pop the wave maximum of distinct
// 24-bit keys (value key << 8 | 255 - id, wave_route_keys' order). The first K are the set when
// a8 - a9 >= 2^-20, a = f32(l - max) being the softmax's argument (l8, l9 the K-th and (K+1)-th
// logits), and a9 >= -64: then r2_exp(a8) / r2_exp(a9) > 1 + 2^-21 (each is exp rounded once to
// f32, both normal), so after the multiply by 1/sum the K-th probability is strictly above the
// (K+1)-th and the probability-based selection (wave_route_keys, torch's topk) takes the same set.
// Writes s_ids[0..K) in ascending id and returns true; false (equal or nearly equal logits at the
// K-th place) leaves the decision to the exact path.
template <int K>
__device__ __forceinline__ bool wave_topk_set(const uint32_t* lb, int lane, int* s_ids) {
  uint32_t k0 = (bf16_key(lb[0]) << 8) | (uint32_t)(255 - lane);
  uint32_t k1 = (bf16_key(lb[1]) << 8) | (uint32_t)(191 - lane);
  uint32_t k2 = (bf16_key(lb[2]) << 8) | (uint32_t)(127 - lane);
  uint32_t k3 = (bf16_key(lb[3]) << 8) | (uint32_t)(63 - lane);
  {
    const uint32_t a = max(k0, k1), b = min(k0, k1), c = max(k2, k3), d = min(k2, k3);
    k0 = max(a, c); const uint32_t t1 = min(a, c);
    k3 = min(b, d); const uint32_t t2 = max(b, d);
    k1 = max(t1, t2); k2 = min(t1, t2);
  }
  uint32_t top[K + 1];
#pragma unroll
  for (int r = 0; r <= K; ++r) {
    top[r] = wave_max_u32_v(k0);
    if (k0 == top[r]) { k0 = k1; k1 = k2; k2 = k3; k3 = 0u; }
  }
  const float m = bf16_to_f32(bf16_unkey(top[0] >> 8));
  const float a8 = bf16_to_f32(bf16_unkey(top[K - 1] >> 8)) - m;
  const float a9 = bf16_to_f32(bf16_unkey(top[K] >> 8)) - m;
  if (!(a8 - a9 >= 0x1p-20f) || !(a9 >= -64.0f)) return false;
  uint32_t mine = top[0];
#pragma unroll
  for (int r = 1; r < K; ++r) mine = lane == r ? top[r] : mine;
  const uint32_t id = 255u - (mine & 255u);
  int pos = 0;
#pragma unroll
  for (int r = 0; r < K; ++r) pos += (255u - (top[r] & 255u)) < id ? 1 : 0;
  if (lane < K) s_ids[pos] = (int)id;
  return true;
}

// Stage outputs of a token's routing (the workgroup that writes them), in torch's slot order.
struct RouteOut {
  int32_t* ids;
  float* w_f32;
  uint16_t* w_bf16;
};

// The weights of the set wave_topk_set chose (s_ids ascending, s_lb the 256 logits' bits), with
// wave_route_keys' arithmetic: the same softmax, rank order = descending (logit, -id) key, and
// w = p / (sum of the K in rank order) cast to bf16. Writes s_w[slot] (the bf16 weight as f32) and
// s_tslot[slot] (the slot's rank) and, given o.ids, the stage outputs by rank. With exact_order and
// equal probabilities inside the set, the slot order is torch's, from the exact replay (same set).
template <int K>
__device__ __forceinline__ void wave_route_weights(const uint32_t* s_lb, const int* s_ids, int lane,
                                                   bool exact_order, TopkLds& tk, int* s_rid,
                                                   float* s_wf, uint16_t* s_wb, float* s_w,
                                                   int* s_tslot, uint32_t* s_key, RouteOut o) {
  uint32_t lb[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) lb[q] = s_lb[lane + 64 * q];
  const int sid = s_ids[lane < K ? lane : 0];
  const uint32_t sb = s_lb[sid];
  const uint32_t key = lane < K ? (bf16_key(sb) << 8) | (uint32_t)(255 - sid) : 0u;
  if (lane < K) s_key[lane] = key;
  const float m = bf16_to_f32(bf16_unkey(wave_max_u32_v(key) >> 8));
  float p[4], sum = 0.0f;
#pragma unroll
  for (int q = 0; q < 4; ++q) { p[q] = r2_exp(bf16_to_f32(lb[q]) - m); sum += p[q]; }
  sum = wave_sum_f32(sum);
  const float rs = 1.0f / sum;
  const float ps = r2_exp(bf16_to_f32(sb) - m) * rs;
  int rank = 0;
#pragma unroll
  for (int k = 0; k < K; ++k) rank += s_key[k] > key ? 1 : 0;
  if (lane < K) s_wf[rank] = ps;
  wave_sync();
  const uint64_t ties = __ballot(lane < K - 1 && s_wf[lane] == s_wf[lane + 1]);
  if (ties && exact_order) {
#pragma unroll
    for (int q = 0; q < 4; ++q) p[q] *= rs;
    route_replay_and_write(tk, p, 256, K, lane, s_rid, s_wf, s_wb, nullptr);
    if (lane < K) {
      const int id = s_rid[lane];
      int pos = 0;
#pragma unroll
      for (int q = 0; q < K; ++q) pos += s_ids[q] < id ? 1 : 0;
      s_w[pos] = bf16_to_f32(s_wb[lane]);
      s_tslot[pos] = lane;
      if (o.ids) o.ids[lane] = id;
      if (o.w_f32) o.w_f32[lane] = s_wf[lane];
      if (o.w_bf16) o.w_bf16[lane] = s_wb[lane];
    }
    return;
  }
  float tot = 0.0f;
#pragma unroll
  for (int r = 0; r < K; ++r) tot += s_wf[r];
  if (lane < K) {
    const float wv = ps / tot;
    const uint16_t wb = (uint16_t)f32_to_bf16(wv);
    s_w[lane] = bf16_to_f32(wb);
    s_tslot[lane] = rank;
    if (o.ids) o.ids[rank] = sid;
    if (o.w_f32) o.w_f32[rank] = wv;
    if (o.w_bf16) o.w_bf16[rank] = wb;
  }
}

// 32-bit word at a 2-byte-aligned byte offset of an LDS region (4-byte-aligned base): the two
// dwords around it, realigned
__device__ __forceinline__ uint32_t lds_u32_at(const uint32_t* base, int off) {
  const int i = off >> 2, sh = off & 3;
  return __builtin_amdgcn_alignbyte(base[i + 1], base[i], sh);
}

// Q6_K (210-byte block, 2-byte aligned in LDS at byte `blk` of `lds`): 64 of its elements against
// the activations a[0..64): half g, planes k = 2m and 2m + 1, every l in [0, 32) —
// e = 128 g + 32 k + l, q = (ql[64g + 32(k&1) + l] >> 4(k>>1)) & 15 | ((qh[32g + l] >> 2k) & 3) << 4,
// value d * sc[8g + 2k + (l>>4)] * (q - 32) (tools/gguf_reader.py:299-322), summed as
// d * sc * (sum a q - 32 sum a) per 16-element run.
__device__ __forceinline__ float q6k_lane64_dot(const uint32_t* lds, int blk, int g, int m, const float* a) {
  const int sh = blk & 3;
  uint32_t ql[16], qh[8];
  {
    const int o = (blk + 64 * g) >> 2;
    uint32_t w[17];
#pragma unroll
    for (int i = 0; i < 17; ++i) w[i] = lds[o + i];
#pragma unroll
    for (int i = 0; i < 16; ++i) ql[i] = __builtin_amdgcn_alignbyte(w[i + 1], w[i], sh);
  }
  {
    const int o = (blk + 128 + 32 * g) >> 2;
    uint32_t w[9];
#pragma unroll
    for (int i = 0; i < 9; ++i) w[i] = lds[o + i];
#pragma unroll
    for (int i = 0; i < 8; ++i) qh[i] = __builtin_amdgcn_alignbyte(w[i + 1], w[i], sh);
  }
  const uint32_t scw = lds_u32_at(lds, blk + 192 + 8 * g + 4 * m);
  const uint32_t dw = lds[(blk + 208) >> 2] >> (8 * ((blk + 208) & 3));
  const float d = f16_to_f32(dw & 0xFFFFu);
  const uint32_t shl = 4u * (uint32_t)m;
  float acc = 0.0f;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t shh = 4u * (uint32_t)m + 2u * (uint32_t)h;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      float dq = 0.0f, sa = 0.0f;
#pragma unroll
      for (int l = 16 * u; l < 16 * u + 16; ++l) {
        const uint32_t qlb = ql[(32 * h + l) >> 2] >> (8 * (l & 3));
        const uint32_t qhb = qh[l >> 2] >> (8 * (l & 3));
        const float q = (float)(((qlb >> shl) & 15u) | (((qhb >> shh) & 3u) << 4));
        const float av = a[32 * h + l];
        dq = fmaf(av, q, dq);
        sa += av;
      }
      const float sc = (float)(int8_t)(scw >> (8 * (2 * h + u)));
      acc += d * sc * (dq - 32.0f * sa);
    }
  }
  return acc;
}

// XDT: input x width; RDT: router row width (bf16, or f32 as the shipped artifact's ffn_gate_inp);
// DFMT: routed down format (Q4_K, Q5_K as the artifact's ffn_down_exps in 37 of 40 layers, or
// Q6_K as in its other 3, whose 2-byte-aligned 210-byte blocks are staged through LDS);
// SFMT: shared-expert rows (bf16, or Q8_0 as the artifact's ffn_*_shexp)
template <int XDT, int RDT, int DFMT, int SFMT>
__global__ __launch_bounds__(kThreads) void k_dec_layer(LayerArgs a) {
  constexpr int H = 2048, I = 512, E = 256, K = 8, IS = 512, ISX = IS / kXcd;
  __shared__ float s_x[H];
  __shared__ TopkLds tk;                 // the exact replay's scratch (ties only)
  __shared__ float s_k[I];               // routed activations of this XCD's slot
  // digit planes, exponents and float sums of the 16-element groups of s_k (Q4_K and Q5_K down dots)
  __shared__ uint4 s_kd[3][I / 16];
  __shared__ int s_ke[I / 16];
  __shared__ float s_ks[I / 16];
  __shared__ float s_sh[ISX];            // shared activations of this XCD's slice
  // the routed slots in ascending expert id: XCD x runs slot x (s_ids[x]); s_w its bf16 weight,
  // s_tslot its position in torch's slot order (stage outputs)
  __shared__ int s_ids[K];
  __shared__ float s_w[K];
  __shared__ int s_tslot[K];
  __shared__ int s_rid[K];               // ids in torch's slot order (the exact paths)
  __shared__ float s_wf[K];
  __shared__ uint16_t s_wb[K];
  __shared__ uint32_t s_lb[256];         // the logits' bf16 bits, for the weights wave
  __shared__ int s_wdone;                // the weights are in s_w already (an exact path ran)
  __shared__ uint32_t s_key[K];          // the set's keys (rank order of the weights wave)
  __shared__ float s_comb[2][K][8];      // [y | shared partial][slot | xcd][row]
  __shared__ float s_gate;
  __shared__ double s_red[2][kThreads / 64];
  __shared__ int s_role[2];               // the role's launch count, the test hook
  __shared__ int s_bad;                   // a wait of this workgroup gave up
  __shared__ uint4 s_occ[kOccPad];
  // Q8_0 shared rows staged for the lanes' block reads: waves 5-6 their gate and up rows (2176 B
  // each, dwords [1088 (wave - 5), +1088)), wave 4 the 64 rows' 68-byte slices of this XCD
  // (dwords [2176, 3264))
  __shared__ uint32_t s_q8[SFMT == MOE_FMT_Q8_0 ? 4 * 544 + 64 * 17 : 1];
  const int t = threadIdx.x;
  const int lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
  // 8 shared-expert weights held in a uint4 (bf16 x 8, or Q8_0 d / quants) dotted with x8
  auto shared_dot = [](uint4 w, const float* x8) -> float {
    if (SFMT == MOE_FMT_Q8_0) return q8_0_dot8(__uint_as_float(w.x), w.y, w.z, x8);
    return dot8_bf16(w, x8);
  };
  const int l16 = lane & 15;
  int* err = a.sync + kErrWord;
  // the role (x, r) from the launch's round-robin placement; the role's launch count is read
  // first, the input row and every routing-independent weight this role uses right behind it
  const int x = (int)blockIdx.x & (kXcd - 1), r = (int)blockIdx.x >> 3;
  const int j = kPer * x + r;            // combine rows [8j, 8j+8)
  int ep = 0, hook = 0;
  if (t == 0) {
    ep = aload(a.sync + kRoleEpoch + kPer * x + r);
    hook = aload(a.sync + kHookWord);
  }
  float4 xin;
  if (XDT == MOE_DT_F32) {
    xin = reinterpret_cast<const float4*>(a.x)[t];
  } else {
    const uint2 u = reinterpret_cast<const uint2*>(a.x)[t];
    xin = make_float4(bf16_to_f32(u.x & 0xFFFFu), bf16_to_f32(u.x >> 16),
                      bf16_to_f32(u.y & 0xFFFFu), bf16_to_f32(u.y >> 16));
  }
  const float4 nw = a.norm_w ? reinterpret_cast<const float4*>(a.norm_w)[t] : make_float4(1.f, 1.f, 1.f, 1.f);

  // ------------------------------------------------------------------ start: loads, x, norm --
  // routing-independent weights: router row 8r + wave; shared gate and up rows
  // i = 64x + 2r + (wave - 5) (waves 5-6); the scalar gate row (wave 7); shared-down rows
  // 64r + (lane >> 3) + 8q, cols 64x + 8 (lane & 7) .. +8 (wave 4, used while wave 0 selects the
  // experts). Wave 0, which polls the logits, carries none of the extras.
  // the router rows now; the shared expert's rows (waves 4-7, wx) once these and the input row
  // have landed (below): requested together, they would slow the loads the routing waits on
  uint4 wr4[RDT == MOE_DT_F32 ? 8 : 4], wx[8];
  if (RDT == MOE_DT_F32) {
    const float* wr = reinterpret_cast<const float*>(a.w_router) + (size_t)(8 * r + wave) * H;
#pragma unroll
    for (int c = 0; c < 8; ++c)
      wr4[c] = *reinterpret_cast<const uint4*>(wr + 512 * (c >> 1) + 8 * lane + 4 * (c & 1));
  } else {
    const uint16_t* wr = reinterpret_cast<const uint16_t*>(a.w_router) + (size_t)(8 * r + wave) * H;
#pragma unroll
    for (int c = 0; c < 4; ++c) wr4[c] = *reinterpret_cast<const uint4*>(wr + 512 * c + 8 * lane);
  }
  // waves 5-6: shared gate row wx[0..3], up row wx[4..7]; wave 7: the scalar gate row wx[0..3];
  // wave 4: shared-down rows 64r + (lane >> 3) + 8q at cols 64x + 8 (lane & 7), q = 0..7
  // the logit bias, read unconditionally (a device zero when there is none) after the weights, as
  // a global-address-space load: a flat load outstanding would make the compiler wait for every
  // earlier load (the router rows) before the first use of x
  typedef const __attribute__((address_space(1))) float gfloat;
  const float bias_e = *(gfloat*)(a.bias ? a.bias + 8 * r + wave : &kZeroBias);
  const float resid = (t < 8 && a.residual) ? a.residual[8 * j + t] : 0.0f;
  // norm: r = f32(1 / sqrt(mean(x^2) + eps)) in f64 (every square exact, one final rounding);
  // and sum (x_j nw_j)^2 (exact products, their squares rounded in f64) for the router's bound on
  // the normalized input's 2-norm: each element of x_n = (x r) nw is within two f32 roundings of
  // x_j r nw_j
  {
    double ss = (double)xin.x * xin.x + (double)xin.y * xin.y + (double)xin.z * xin.z + (double)xin.w * xin.w;
    double sa = 0.0;
    {
      const double p0 = (double)xin.x * nw.x, p1 = (double)xin.y * nw.y;
      const double p2 = (double)xin.z * nw.z, p3 = (double)xin.w * nw.w;
      sa = p0 * p0 + p1 * p1 + p2 * p2 + p3 * p3;
    }
    ss = wave_sum_f64_v(ss);
    sa = wave_sum_f64_v(sa);
    if (lane == 0) { s_red[0][wave] = ss; s_red[1][wave] = sa; }
  }
  if (t == 0) {
    s_role[0] = ep;
    s_role[1] = hook;
    s_bad = 0;
  }
  // the LDS footprint keeps one workgroup per CU; this never-true branch keeps the array
  const bool never = a.out == reinterpret_cast<float*>(a.sync);
  if (never) s_occ[t] = make_uint4(t, 0, 0, 0);
  __syncthreads();
  if (never) atomicOr(err, (int)s_occ[t ^ 1].x);
  const uint32_t epoch = (uint32_t)s_role[0] + 1u;
  const Spin sp{err, &s_bad, s_role[1]};
  // Q8_0 shared rows (34-byte blocks, 2-byte aligned; a row's block pairs are 4-byte aligned),
  // requested as contiguous bytes and staged through LDS (s_q8) just before use: waves 5-6 the gate
  // and up rows of their intermediate row (16-byte loads), wave 4 the 64 shared-down rows'
  // 68-byte slices of this XCD (consecutive dwords). Each lane then reads its own blocks from LDS.
  uint32_t wq[SFMT == MOE_FMT_Q8_0 ? 20 : 1];
  if (SFMT == MOE_FMT_Q8_0 && wave >= 4 && wave <= 6) {
    if (wave == 4) {
#pragma unroll
      for (int k = 0; k < 17; ++k) {
        const int g = lane + 64 * k, row = g / 17;
        wq[k] = *reinterpret_cast<const uint32_t*>(reinterpret_cast<const uint8_t*>(a.sd) +
                                                   (size_t)(64 * r + row) * (IS / 32 * 34) + 68 * x + 4 * (g - 17 * row));
      }
    } else {
      const size_t roff = (size_t)(ISX * x + 2 * r + (wave - 5)) * (H / 32 * 34);
      const uint4* g = reinterpret_cast<const uint4*>(reinterpret_cast<const uint8_t*>(a.sg) + roff);
      const uint4* u = reinterpret_cast<const uint4*>(reinterpret_cast<const uint8_t*>(a.su) + roff);
      // 136 uint4 per row, gate then up: chunk c = lane + 64 k, k < 4 for every lane, k = 4 for 16
#pragma unroll
      for (int k = 0; k < 5; ++k) {
        const int c = lane + 64 * k;
        const uint4 v = c < 136 ? g[c] : (c < 272 ? u[c - 136] : make_uint4(0u, 0u, 0u, 0u));
        wq[4 * k] = v.x; wq[4 * k + 1] = v.y; wq[4 * k + 2] = v.z; wq[4 * k + 3] = v.w;
      }
    }
  } else if (wave >= 4) {
    // one wave-uniform block with per-wave bases (p_lo: loads 0-3, p_hi: 4-7, stride st) rather
    // than a branch per wave, whose register reuse makes the compiler wait on loads the wave
    // never issued
    const uint16_t *p_lo, *p_hi;
    size_t st;
    if (wave == 4) {
      p_lo = a.sd + (size_t)(64 * r + (lane >> 3)) * IS + ISX * x + 8 * (lane & 7);
      p_hi = p_lo + (size_t)32 * IS;
      st = (size_t)8 * IS;
    } else if (wave == 7) {
      // bf16 row: 8 elements per load; f32 row: the first and second 4 of those 8 (p_hi)
      p_lo = a.ssg + (a.ssg_f32 ? 16 : 8) * lane;
      p_hi = p_lo + (a.ssg_f32 ? 8 : 0);
      st = a.ssg_f32 ? 1024 : 512;
    } else {
      const int i = ISX * x + 2 * r + (wave - 5);
      p_lo = a.sg + (size_t)i * H + 8 * lane;
      p_hi = a.su + (size_t)i * H + 8 * lane;
      st = 512;
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      wx[q] = *reinterpret_cast<const uint4*>(p_lo + st * q);
      wx[4 + q] = *reinterpret_cast<const uint4*>(p_hi + st * q);
    }
  }
  uint32_t* xb = a.xch + (epoch & 1u) * XW_BUF;          // this launch's words
  uint32_t* xn = a.xch + ((epoch & 1u) ^ 1u) * XW_BUF;   // the next launch's, zeroed here
  const __amdgpu_buffer_rsrc_t xr =
      __builtin_amdgcn_make_buffer_rsrc(xb, 0, XW_BUF * 4, 0x00020000);
  {
    double tot = 0.0, tsq = 0.0;
#pragma unroll
    for (int q = 0; q < kThreads / 64; ++q) { tot += s_red[0][q]; tsq += s_red[1][q]; }
    float4 v = xin;
    float rs = 1.0f;
    if (a.norm_w) {
      rs = (float)(1.0 / sqrt(tot / (double)H + (double)a.norm_eps));
      v = make_float4((v.x * rs) * nw.x, (v.y * rs) * nw.y, (v.z * rs) * nw.z, (v.w * rs) * nw.w);
    }
    reinterpret_cast<float4*>(s_x)[t] = v;
    __syncthreads();
    // the router's bound on |x_n|_2, after the barrier (nothing before it waits for this): the
    // f32 root of the f64 sum raised by 2^-15 (its rounding to f32), the root raised by 2^-20
    // (its error and the two f32 roundings of each normalized element)
    const double xl2 = (double)__builtin_sqrtf((float)tsq * (1.0f + 0x1p-15f)) * (1.0 + 0x1p-20) * (double)rs;

    // ---------------------------------------------------------------------------- phase 1 --
    // x at cols 512c + 8 lane (c = 0..3): f64 for the router dot, f32 for waves 5-7's dots
    float xv[4][8];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float4 u0 = *reinterpret_cast<const float4*>(s_x + 512 * c + 8 * lane);
      const float4 u1 = *reinterpret_cast<const float4*>(s_x + 512 * c + 8 * lane + 4);
      xv[c][0] = u0.x; xv[c][1] = u0.y; xv[c][2] = u0.z; xv[c][3] = u0.w;
      xv[c][4] = u1.x; xv[c][5] = u1.y; xv[c][6] = u1.z; xv[c][7] = u1.w;
    }
    double xd[4][8];
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int i = 0; i < 8; ++i) xd[c][i] = (double)xv[c][i];
    const int e = 8 * r + wave;
    const uint32_t bits = router_row_bits<RDT>(wr4, xd, (double)bias_e, xl2);
    if (lane == 0) lstore(xr, 4 * (XW_LOG + 256 * x + e), ~bits);
    if ((wave == 5 || wave == 6) && SFMT == MOE_FMT_Q8_0) {
      uint32_t* st = s_q8 + 1088 * (wave - 5);
#pragma unroll
      for (int k = 0; k < 5; ++k) {
        const int c = lane + 64 * k;
        if (c < 272) *reinterpret_cast<uint4*>(st + 4 * c) = make_uint4(wq[4 * k], wq[4 * k + 1], wq[4 * k + 2], wq[4 * k + 3]);
      }
      wave_sync();
      // block `lane` of both rows: the 9 dwords of its pair half, then elements 32 lane .. +31
      uint32_t bg[9], bu[9];
#pragma unroll
      for (int k = 0; k < 9; ++k) {
        bg[k] = st[17 * (lane >> 1) + 8 * (lane & 1) + k];
        bu[k] = st[544 + 17 * (lane >> 1) + 8 * (lane & 1) + k];
      }
      float xq[32];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const float4 u = reinterpret_cast<const float4*>(s_x + 32 * lane)[k];
        xq[4 * k] = u.x; xq[4 * k + 1] = u.y; xq[4 * k + 2] = u.z; xq[4 * k + 3] = u.w;
      }
      float ag = q8_0_block_dot(bg, lane & 1, xq), au = q8_0_block_dot(bu, lane & 1, xq);
      ag = wave_sum_f32_v(ag);
      au = wave_sum_f32_v(au);
      if (lane == 0) lstore(xr, 4 * (XW_SSH + ISX * x + 2 * r + (wave - 5)), xenc(silu_f32(ag) * au));
    } else if (wave == 5 || wave == 6) {
      float ag = 0.0f, au = 0.0f;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        ag += shared_dot(wx[c], xv[c]);
        au += shared_dot(wx[4 + c], xv[c]);
      }
      ag = wave_sum_f32_v(ag);
      au = wave_sum_f32_v(au);
      if (lane == 0) lstore(xr, 4 * (XW_SSH + ISX * x + 2 * r + (wave - 5)), xenc(silu_f32(ag) * au));
    } else if (wave == 7) {
      float gs = 0.0f;
      if (a.ssg_f32) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const float w8[8] = {__uint_as_float(wx[c].x), __uint_as_float(wx[c].y), __uint_as_float(wx[c].z),
                               __uint_as_float(wx[c].w), __uint_as_float(wx[4 + c].x), __uint_as_float(wx[4 + c].y),
                               __uint_as_float(wx[4 + c].z), __uint_as_float(wx[4 + c].w)};
          float s8 = fmaf(w8[0], xv[c][0], 0.0f);
#pragma unroll
          for (int i = 1; i < 8; ++i) s8 = fmaf(w8[i], xv[c][i], s8);
          gs += s8;
        }
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c) gs += dot8_bf16(wx[c], xv[c]);
      }
      gs = wave_sum_f32_v(gs);
      const float p = 1.0f / (1.0f + expf(-gs));
      if (lane == 0) {
        s_gate = p;
        if (j == 0 && a.gate_prob_out) a.gate_prob_out[0] = p;
      }
    }
  }

  // ------------------------------------------------------------------------------ phase 2 --
  if (wave == 0) {
    uint32_t lw[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) lw[q] = lload(xr, 4 * (XW_LOG + 256 * x + lane + 64 * q));
    for (int spins = 0;; ++spins) {
      const bool ok = lw[0] && lw[1] && lw[2] && lw[3];
      if (ok) break;
      if (spins >= kSpinLimit) {
        // a logit that never arrived counts as the lowest finite bf16 (-3.39e38), so no NaN
        // reaches the selection, whose indices stay in range whatever the values
        sp.give_up();
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (lw[q] == 0u) lw[q] = ~0xFF7Fu;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (lw[q] == 0u) lw[q] = lload(xr, 4 * (XW_LOG + 256 * x + lane + 64 * q));
    }
    sp.done();
    uint32_t lb[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) lb[q] = ~lw[q] & 0xFFFFu;
    if (j == 0 && a.logits_out) {
#pragma unroll
      for (int q = 0; q < 4; ++q) a.logits_out[64 * q + lane] = (uint16_t)lb[q];
    }
    // the set decides the expert loads; its weights are formed by wave 3 while those loads are in
    // flight. Otherwise (a tie or near tie at the K-th place) the probability-based selection and,
    // where it cannot settle, the exact replay run here, weights included.
    if (wave_topk_set<K>(lb, lane, s_ids)) {
#pragma unroll
      for (int q = 0; q < 4; ++q) s_lb[lane + 64 * q] = lb[q];
      if (lane == 0) s_wdone = 0;
    } else {
      float p[4];
      if (!wave_route_keys<K>(lb, lane, a.exact_order != 0, p, s_rid, s_wf, s_wb))
        route_replay_and_write(tk, p, E, K, lane, s_rid, s_wf, s_wb, nullptr);
      wave_sync();
      if (lane < K) {
        const int id = s_rid[lane];
        int pos = 0;
#pragma unroll
        for (int q = 0; q < K; ++q) pos += (s_rid[q] < id) ? 1 : 0;
        s_ids[pos] = id;                 // ascending expert id (ids are distinct)
        s_w[pos] = bf16_to_f32(s_wb[lane]);
        s_tslot[pos] = lane;
        if (j == 0) {
          if (a.ids_out) a.ids_out[lane] = id;
          if (a.w_f32_out) a.w_f32_out[lane] = s_wf[lane];
          if (a.w_bf16_out) a.w_bf16_out[lane] = s_wb[lane];
        }
      }
      if (lane == 0) s_wdone = 1;
    }
  }
  __syncthreads();
  const int e = s_ids[x];
  // phase-3 weights: down rows h = 64 r + 2 (t >> 4) + pass of expert e; 16 lanes per row,
  // lane: super-block b = l16 >> 3, 16-byte nibble chunk c = l16 & 7 (requested with phase 2's)
  // Q4_K: header + nibble chunk (two loads); Q5_K: also the chunk's 16 qh bytes (tools/gguf_reader.py:271-296)
  constexpr int kDB = DFMT == MOE_FMT_Q6_K ? 210 : DFMT == MOE_FMT_Q5_K ? 176 : 144;
  constexpr int kDQs = DFMT == MOE_FMT_Q5_K ? 48 : 16;
  constexpr size_t drowb = (I / 256) * kDB;
  // Q6_K: the workgroup's 64 down rows are one 16-byte-aligned run of 64 * 420 bytes, loaded as
  // uint4 (4 per thread, the index clamped so no load sits in a branch) and staged in s_occ
  constexpr int kQ6U4 = 64 * (int)drowb / 16;
  static_assert(DFMT != MOE_FMT_Q6_K || (kQ6U4 <= 4 * kThreads && 4 * kThreads <= kOccPad), "Q6_K staging");
  uint4 dh[2], dq[2], dqh[2];
  uint4 d60, d61, d62, d63;              // named, not an array: a loop-indexed array goes to LDS
  {
    // routed gate/up: intermediate rows i0, i0+1 (gate and up) per wave
    const int i0 = 16 * r + 2 * wave;
    const int b = lane >> 3, c = lane & 7, gq = c >> 1, l0 = 16 * (c & 1);
    constexpr size_t rowb = (H / 256) * 144;
    const uint8_t* gbase = a.gu + (size_t)e * a.gu_estride;
    const uint8_t* ubase = a.gu_up + (size_t)e * a.gu_estride;
    uint4 hdr[4], qs[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint8_t* p = ((q & 1) ? ubase : gbase) + (size_t)(i0 + (q >> 1)) * rowb + (size_t)b * 144;
      hdr[q] = *reinterpret_cast<const uint4*>(p);
      qs[q] = *reinterpret_cast<const uint4*>(p + 16 + 16 * c);
    }
    if (DFMT == MOE_FMT_Q6_K) {
      const uint4* src = reinterpret_cast<const uint4*>(a.dn + ((size_t)e * H + 64 * r) * drowb);
      d60 = src[t];
      d61 = src[min(t + kThreads, kQ6U4 - 1)];
      d62 = src[min(t + 2 * kThreads, kQ6U4 - 1)];
      d63 = src[min(t + 3 * kThreads, kQ6U4 - 1)];
    } else {
      const int db = l16 >> 3, dc = l16 & 7;
#pragma unroll
      for (int pass = 0; pass < 2; ++pass) {
        const int h = 64 * r + 2 * (t >> 4) + pass;
        const uint8_t* p = a.dn + ((size_t)e * H + h) * drowb + (size_t)db * kDB;
        dh[pass] = *reinterpret_cast<const uint4*>(p);
        dq[pass] = *reinterpret_cast<const uint4*>(p + kDQs + 16 * dc);
        if (DFMT == MOE_FMT_Q5_K) dqh[pass] = *reinterpret_cast<const uint4*>(p + 16 + 16 * (dc & 1));
      }
    }
    // wave 3, its rows requested: the routing weights of the set wave 0 chose
    if (wave == 3 && !s_wdone)
      wave_route_weights<K>(s_lb, s_ids, lane, a.exact_order != 0, tk, s_rid, s_wf, s_wb, s_w, s_tslot, s_key,
                            j == 0 ? RouteOut{a.ids_out, a.w_f32_out, a.w_bf16_out} : RouteOut{nullptr, nullptr, nullptr});
    float xl[16], xh[16];
    {
      const float* xp = s_x + 256 * b + 64 * gq + l0;
#pragma unroll
      for (int i = 0; i < 16; i += 4) {
        const float4 u0 = *reinterpret_cast<const float4*>(xp + i);
        const float4 u1 = *reinterpret_cast<const float4*>(xp + 32 + i);
        xl[i] = u0.x; xl[i + 1] = u0.y; xl[i + 2] = u0.z; xl[i + 3] = u0.w;
        xh[i] = u1.x; xh[i + 1] = u1.y; xh[i + 2] = u1.z; xh[i + 3] = u1.w;
      }
    }
    float sxl = 0.0f, sxh = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) { sxl += xl[i]; sxh += xh[i]; }
    float acc[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) acc[q] = wave_sum_f32_v(q4k_chunk_dot(hdr[q], qs[q], gq, xl, xh, sxl, sxh));
#pragma unroll
    for (int q = 0; q < 2; ++q)
      if (lane == q) lstore(xr, 4 * (XW_SR + I * x + i0 + q), xenc(silu_f32(acc[2 * q]) * acc[2 * q + 1]));
  }

  // wave 4, while waves 0-1 wait for the slot's activations: the shared-down partial over this
  // XCD's 64 shared activations (ready since phase 1), rows h = 64r + (lane >> 3) + 8q, published
  // to the combining workgroups (agent scope); off the routing's path to the expert loads
  if (wave == 4) {
    {
      const uint4 v = lane < ISX / 4 ? lwait4(xr, 4 * (XW_SSH + ISX * x) + 16 * lane, sp) : make_uint4(0, 0, 0, 0);
      if (lane < ISX / 4)
        reinterpret_cast<float4*>(s_sh)[lane] = make_float4(xdec(v.x), xdec(v.y), xdec(v.z), xdec(v.w));
    }
    wave_sync();
    if (SFMT == MOE_FMT_Q8_0) {
      uint32_t* st = s_q8 + 2176;
#pragma unroll
      for (int k = 0; k < 17; ++k) st[lane + 64 * k] = wq[k];
      wave_sync();
      // row 64 r + lane: its two blocks (this XCD's 64 shared activations) in one lane
      uint32_t bd[17];
#pragma unroll
      for (int k = 0; k < 17; ++k) bd[k] = st[17 * lane + k];
      float sq[64];
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        const float4 u = reinterpret_cast<const float4*>(s_sh)[k];
        sq[4 * k] = u.x; sq[4 * k + 1] = u.y; sq[4 * k + 2] = u.z; sq[4 * k + 3] = u.w;
      }
      const float acc = q8_0_block_dot(bd, 0, sq) + q8_0_block_dot(bd + 8, 1, sq + 32);
      xstore(xb + XW_SHP + H * x + 64 * r + lane, xenc(acc));
    }
    float sv[8];
    {
      const float4 u0 = *reinterpret_cast<const float4*>(s_sh + 8 * (lane & 7));
      const float4 u1 = *reinterpret_cast<const float4*>(s_sh + 8 * (lane & 7) + 4);
      sv[0] = u0.x; sv[1] = u0.y; sv[2] = u0.z; sv[3] = u0.w;
      sv[4] = u1.x; sv[5] = u1.y; sv[6] = u1.z; sv[7] = u1.w;
    }
#pragma unroll
    for (int q = 0; q < (SFMT == MOE_FMT_Q8_0 ? 0 : 8); ++q) {
      float acc = shared_dot(wx[q], sv);
      acc += dpp_f32<0xB1>(acc);
      acc += dpp_f32<0x4E>(acc);
      acc += dpp_f32<0x141>(acc);        // sum over the 8 lanes of the row
      if ((lane & 7) == 0) xstore(xb + XW_SHP + H * x + 64 * r + (lane >> 3) + 8 * q, xenc(acc));
    }
    }

  // ------------------------------------------------------------------------------ phase 3 --
  if (DFMT == MOE_FMT_Q6_K) {
    s_occ[t] = d60;
    s_occ[t + kThreads] = d61;
    s_occ[t + 2 * kThreads] = d62;
    s_occ[t + 3 * kThreads] = d63;
  }
  if (t < I / 4) {
    const uint4 v = lwait4(xr, 4 * (XW_SR + I * x) + 16 * t, sp);
    const float f[4] = {xdec(v.x), xdec(v.y), xdec(v.z), xdec(v.w)};
    reinterpret_cast<float4*>(s_k)[t] = make_float4(f[0], f[1], f[2], f[3]);
    if constexpr (DFMT == MOE_FMT_Q4_K || DFMT == MOE_FMT_Q5_K) {
      // the digit planes of the slot's activations: group t / 4 is the quad of lanes 4g .. 4g+3
      // (waves 0-1 whole, so the quad moves see every lane); its float sum in element order
      float m = fmaxf(fmaxf(fabsf(f[0]), fabsf(f[1])), fmaxf(fabsf(f[2]), fabsf(f[3])));
      m = fmaxf(m, dpp_f32<0xB1>(m));
      m = fmaxf(m, dpp_f32<0x4E>(m));
      const float s4 = ((f[0] + f[1]) + f[2]) + f[3];
      const float gsum = ((dpp_f32<0x00>(s4) + dpp_f32<0x55>(s4)) + dpp_f32<0xAA>(s4)) + dpp_f32<0xFF>(s4);
      const int e = group_exp(m);
      uint32_t w[3];
      digits4(f, e, w);
#pragma unroll
      for (int p = 0; p < 3; ++p) reinterpret_cast<uint32_t*>(&s_kd[p][0])[t] = w[p];
      if ((t & 3) == 0) {
        s_ke[t >> 2] = e;
        s_ks[t >> 2] = gsum;
      }
    }
  }
  __syncthreads();
  const int xslot = s_tslot[x];          // this XCD's slot in torch's order (expert_raw)
  if (DFMT == MOE_FMT_Q6_K) {
    // down row 64r + (t >> 3): 8 lanes per row, 64 elements each, from the staged rows
    const int rho = t >> 3, s8 = t & 7, b = s8 >> 2, g = (s8 >> 1) & 1, m = s8 & 1;
    float v = q6k_lane64_dot(reinterpret_cast<const uint32_t*>(s_occ), (int)drowb * rho + kDB * b, g, m,
                             s_k + 256 * b + 128 * g + 64 * m);
    v += dpp_f32<0xB1>(v);
    v += dpp_f32<0x4E>(v);
    v += dpp_f32<0x141>(v);              // the 8 lanes of the row
    if (s8 == 0) {
      const int h = 64 * r + rho;
      xstore(xb + XW_Y + H * x + h, xenc(v));
      if (a.expert_raw) a.expert_raw[(size_t)xslot * H + h] = v;
    }
  } else {
    const int b = l16 >> 3, c = l16 & 7, gq = c >> 1, l0 = 16 * (c & 1);
    // both rows before either store: a load wait placed after an agent-scope store would also
    // wait for that store's write-through (vmcnt counts both)
    float v[2];
    const int glo = 16 * b + 4 * gq + (l0 >> 4), ghi = glo + 2;
    uint4 zl[3], zh[3];
#pragma unroll
    for (int p = 0; p < 3; ++p) {
      zl[p] = s_kd[p][glo];
      zh[p] = s_kd[p][ghi];
    }
    const int el = s_ke[glo], eh = s_ke[ghi];
    const float sl = s_ks[glo], sh = s_ks[ghi];
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {
      uint32_t lo[4], hi[4];
      if (DFMT == MOE_FMT_Q5_K) q5k_bytes(dq[pass], dqh[pass], gq, lo, hi);
      else q4k_bytes(dq[pass], lo, hi);
      v[pass] = row16_sum_f32(kquant_chunk_dot_dig(dh[pass], lo, hi, gq, zl, zh, el, eh, sl, sh));
    }
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {
      if (l16 == 0) {
        const int h = 64 * r + 2 * (t >> 4) + pass;
        xstore(xb + XW_Y + H * x + h, xenc(v[pass]));
        if (a.expert_raw) a.expert_raw[(size_t)xslot * H + h] = v[pass];
      }
    }
  }

  // ------------------------------------------------------------------------------ phase 4 --
  // wave 0 collects its combine rows, waves 4-7 warm the next layer's router rows and norm weight
  // and clear the next launch's exchange words. Only what the next layer's routing waits on is
  // warmed: its shared-expert rows have slack there, and reading them here (6.3 MB more) slowed
  // this layer's combine exchange by more than they saved.
  if (wave >= 4) {
    if (a.nx_router) {
      // warm XCD x's L2 with what role (x, r) reads first in the next layer
      const int u = t - 256;
      uint32_t acc = 0;
      // rows 8r .. 8r + 7: 2048 uint4 of bf16, 4096 of f32
      const uint4* nr = reinterpret_cast<const uint4*>(a.nx_router) + (size_t)r * H * (a.nx_router_f32 ? 2 : 1);
#pragma unroll
      for (int q = 0; q < 8; ++q) acc ^= xor4(nr[u + 256 * q]);
      if (a.nx_router_f32) {
#pragma unroll
        for (int q = 8; q < 16; ++q) acc ^= xor4(nr[u + 256 * q]);
      }
      if (a.nx_norm) {
        const uint4* nn = reinterpret_cast<const uint4*>(a.nx_norm);
        acc ^= xor4(nn[u]) ^ xor4(nn[u + 256]);
      }
      if (acc == 0x9E3779B9u && a.out == reinterpret_cast<float*>(a.sync)) atomicOr(err, 0);
    }
    // the next launch's exchange words (its epoch parity), cleared last: nothing here waits on them
    if (t - 256 < kClearPerWg && kClearPerWg * j + t - 256 < XW_BUF) xstore(xn + kClearPerWg * j + t - 256, 0u);
  } else if (wave == 0) {
    // y[k][8j..8j+7] for the 8 slots and the 8 XCDs' shared partials (two 16-byte groups each)
    if (t < 32) {
      const int k = t >> 2, kind = (t >> 1) & 1, half = t & 1;
      const uint4 v = xwait4(xr, 4 * ((kind ? XW_SHP : XW_Y) + H * k + 8 * j) + 16 * half, sp);
      float* o = &s_comb[kind][k][4 * half];
      o[0] = xdec(v.x); o[1] = xdec(v.y); o[2] = xdec(v.z); o[3] = xdec(v.w);
    }
    wave_sync();
    if (t < 8) {
      const int h = 8 * j + t;
      float acc = 0.0f;
#pragma unroll
      for (int k = 0; k < K; ++k) acc = comb_madd(acc, s_w[k], s_comb[0][k][t]);   // ascending id
      float shr = 0.0f;
#pragma unroll
      for (int q = 0; q < kXcd; ++q) shr += s_comb[1][q][t];
      // a wait of this workgroup gave up: its rows are NaN (the status word says so too)
      const bool bad = s_bad != 0;
      const float nan = __builtin_nanf("");
      if (a.routed_sum) a.routed_sum[h] = bad ? nan : acc;
      if (a.shared_out) a.shared_out[h] = bad ? nan : s_gate * shr;
      a.out[h] = bad ? nan : comb_out(resid, acc, s_gate, shr);
    }
    // this role's launch count, for the next launch
    if (t == 0) astore(a.sync + kRoleEpoch + kPer * x + r, (int)epoch);
  }
}

}  // namespace moe

using namespace moe;

bool moe_layer_kernel_supported(int H, int I, int E, int K, int Is, int gu_fmt, int dn_fmt) {
  // the CU count of the current device, cached per device (0: unknown, -1 not yet asked)
  constexpr int kMaxDev = 64;
  static std::atomic<int> ncu_cache[kMaxDev];
  static std::once_flag once;
  std::call_once(once, [] { for (auto& c : ncu_cache) c.store(-1); });
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) return false;
  int ncu = ncu_cache[dev].load();
  if (ncu < 0) {
    if (hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) ncu = 0;
    ncu_cache[dev].store(ncu);
  }
  // 8 XCDs with at least 32 CUs each (MI355X: exactly 32)
  return ncu >= kG && ncu % kXcd == 0 && H == 2048 && I == 512 && E == 256 && K == 8 &&
         Is == 512 && gu_fmt == MOE_FMT_Q4_K &&
         (dn_fmt == MOE_FMT_Q4_K || dn_fmt == MOE_FMT_Q5_K || dn_fmt == MOE_FMT_Q6_K);
}

namespace {

template <int XDT, int RDT, int SFMT>
void launch_layer_sfmt(int dn_fmt, const LayerArgs& a, hipStream_t st) {
  if (dn_fmt == MOE_FMT_Q5_K)
    hipLaunchKernelGGL((k_dec_layer<XDT, RDT, MOE_FMT_Q5_K, SFMT>), dim3(kG), dim3(kThreads), 0, st, a);
  else if (dn_fmt == MOE_FMT_Q6_K)
    hipLaunchKernelGGL((k_dec_layer<XDT, RDT, MOE_FMT_Q6_K, SFMT>), dim3(kG), dim3(kThreads), 0, st, a);
  else
    hipLaunchKernelGGL((k_dec_layer<XDT, RDT, MOE_FMT_Q4_K, SFMT>), dim3(kG), dim3(kThreads), 0, st, a);
}

template <int XDT, int RDT>
void launch_layer_fmt(int dn_fmt, int sfmt, const LayerArgs& a, hipStream_t st) {
  if (sfmt == MOE_FMT_Q8_0) launch_layer_sfmt<XDT, RDT, MOE_FMT_Q8_0>(dn_fmt, a, st);
  else launch_layer_sfmt<XDT, RDT, MOE_FMT_BF16>(dn_fmt, a, st);
}

}  // namespace

size_t moe_layer_exchange_bytes() { return (size_t)2 * XW_BUF * 4; }

int moe_launch_decode_layer(const MoeDecodeLaunch& L, int* sync, uint32_t* xch, hipStream_t st) {
  LayerArgs a;
  a.x = L.x; a.residual = L.residual; a.w_router = L.w_router; a.bias = L.bias;
  a.gu = (const uint8_t*)L.gu; a.dn = (const uint8_t*)L.dn;
  {
    const size_t rowb = (size_t)(L.H / 256) * 144;
    a.gu_estride = L.gu_estride ? L.gu_estride : (size_t)2 * L.I * rowb;
    a.gu_up = L.gu_up ? (const uint8_t*)L.gu_up : a.gu + (size_t)L.I * rowb;
  }
  a.sg = (const uint16_t*)L.sg; a.su = (const uint16_t*)L.su; a.sd = (const uint16_t*)L.sd;
  a.ssg = (const uint16_t*)L.ssg;
  a.ssg_f32 = L.ssg_dt == MOE_DT_F32 ? 1 : 0;
  a.sync = sync; a.xch = xch;
  a.logits_out = L.logits; a.ids_out = L.ids; a.w_f32_out = L.w_f32; a.w_bf16_out = L.w_bf16;
  a.gate_prob_out = L.gate_prob; a.out = L.out; a.routed_sum = L.routed_sum;
  a.shared_out = L.shared_out; a.expert_raw = L.expert_raw;
  a.exact_order = (L.ids_out_requested || L.expert_raw) ? 1 : 0;
  a.norm_w = L.norm_w;
  a.norm_eps = L.norm_eps;
  a.nx_router = (const uint16_t*)L.nx_router;
  a.nx_router_f32 = L.nx_router_dt == MOE_DT_F32 ? 1 : 0;
  a.nx_norm = L.nx_router ? L.nx_norm : nullptr;
  const bool r32 = L.router_dt == MOE_DT_F32;
  if (L.x_dtype == MOE_DT_F32) {
    if (r32) launch_layer_fmt<MOE_DT_F32, MOE_DT_F32>(L.dn_fmt, L.sfmt, a, st);
    else launch_layer_fmt<MOE_DT_F32, MOE_DT_BF16>(L.dn_fmt, L.sfmt, a, st);
  } else {
    if (r32) launch_layer_fmt<MOE_DT_BF16, MOE_DT_F32>(L.dn_fmt, L.sfmt, a, st);
    else launch_layer_fmt<MOE_DT_BF16, MOE_DT_BF16>(L.dn_fmt, L.sfmt, a, st);
  }
  return moe_check_launch("decode_layer");
}
