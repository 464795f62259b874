// Internal declarations shared by the library's translation units (not part of the C-ABI).
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/moe_gfx950.h"

// thread-local error text behind moe_last_error()
int moe_set_error(int code, const char* fmt, ...);
// checks hipGetLastError() after a launch; returns MOE_OK or MOE_E_HIP
int moe_check_launch(const char* what);

// ---- launch helpers (each returns MOE_OK or an error code) ----------------------------------
int moe_launch_dequant(const void* blocks, int fmt, int64_t n_elts, void* out, int out_dtype,
                       hipStream_t st);

// scratch (may be NULL) of moe_router_i8_scratch_bytes(T, H, E) bytes lets T > 256 run on the
// int8 matrix cores; without it R1 runs on the f64 ones. The bits are the same either way.
int moe_launch_router_logits(const void* x, int x_dtype, const void* w, int w_dtype, const float* bias,
                             int T, int H, int E, uint16_t* logits, void* scratch,
                             size_t scratch_bytes, hipStream_t st);
size_t moe_router_i8_scratch_bytes(int T, int H, int E);
bool moe_router_i8_supported(int T, int H, int E);
int moe_launch_router_logits_i8(const void* x, int x_dtype, const void* w, int w_dtype,
                                const float* bias, int T, int H, int E, uint16_t* logits,
                                void* scratch, hipStream_t st);
// R1-R5 in one launch (8 <= T <= 256, E = 256, K = 8, H % 2048 == 0): scratch of
// moe_router_chain_scratch_bytes(T, E) bytes, sync = the workspace's sync words (arrival counters
// at kRouterCntWord, zero between launches). Same bits as router_logits + route_topk.
bool moe_router_chain_supported(int T, int H, int E, int K);
size_t moe_router_chain_scratch_bytes(int T, int E);
// x16 (NULL: skipped): also the f16 copy of x (k_to_f16's conversion)
struct MoeShJob;
// moe_launch_sort's outputs (P = T * K pairs, E = 256) and the MFMA tile list of bm-row tiles
// (bm <= 160), produced inside the single-launch router by the last 16-token group to finish its
// routing; P = 0: none (the caller sorts)
struct MoeSortJob {
  int P = 0;
  int32_t* offsets = nullptr;      // [E + 1]
  int32_t* sorted = nullptr;       // [P]
  int32_t* pos = nullptr;          // [P]
  int32_t* hits = nullptr;         // [E + 1]
  int32_t* tiles = nullptr;        // the packed tile list (moe_launch_build_tiles' layout)
  int bm = 0;
};
// sh (optional): the small-T shared expert's gate/up and scalar gate as extra blocks of the
// launch, reading x in its own dtype; srt (optional): the sort, as above
int moe_launch_router_chain(const void* x, int x_dtype, const void* w, int w_dtype, const float* bias,
                            int T, int H, int E, uint16_t* logits, float* probs, int32_t* ids,
                            float* w_f32, uint16_t* w_bf16, int32_t* heap_flag, bool exact_order,
                            void* scratch, int* sync, hipStream_t st, uint16_t* x16 = nullptr,
                            const MoeShJob* sh = nullptr, const MoeSortJob* srt = nullptr);
// bytes of router scratch that let every R1 form run (the int8 one, the single-launch chain)
size_t moe_router_scratch_bytes(int T, int H, int E);
int moe_launch_route_topk(const uint16_t* logits, int T, int E, int K, float* probs, int32_t* ids,
                          float* w_f32, uint16_t* w_bf16, int32_t* heap_flag, hipStream_t st,
                          bool exact_order = true);

// sort / permute; ws must hold moe_sort_ws_bytes(P, E) bytes. tiles != NULL: also the MFMA tile
// list of bm-row tiles (moe_launch_build_tiles' result), built inside the sort where it can be.
size_t moe_sort_ws_bytes(int P, int E);
int moe_launch_sort(const int32_t* ids, int P, int E, int32_t* offsets, int32_t* sorted_pairs,
                    int32_t* pair_pos, int32_t* hit_list, void* ws, hipStream_t st,
                    int32_t* tiles = nullptr, int bm = 0);

// MFMA tile list: [count, (expert, row0) x count], rows per tile = bm (MOE_GEMM_BM for gemm.hip,
// MOE_GEMM3_BM for gemm3.hip)
#define MOE_GEMM_BM 64
#define MOE_GEMM3_BM 160
#define MOE_GEMM6_BM 32
int moe_max_mtiles(int P, int E, int bm = MOE_GEMM_BM);
int moe_launch_build_tiles(const int32_t* offsets, const int32_t* hit_list, int E, int P,
                           int32_t* tiles, hipStream_t st, int bm = MOE_GEMM_BM);
// f16 activation operand of the MFMA paths: x [n] f32 / bf16 -> f16 (RNE, saturated)
int moe_launch_to_f16(const void* x, int x_dtype, size_t n, uint16_t* out, hipStream_t st);
// gemm3.hip: warp-specialized grouped GEMM (producer waves decode Q4_K / bf16 into LDS as f16,
// consumer waves run the MFMAs). x16: activations in f16 ([T,H]); S: [rows, I] f16; y: [rows, H]
// f32. tiles == NULL: identity rows 0..T-1 (shared expert). Formats: Q4_K and BF16 (others:
// gemm.hip).
bool moe_gemm3_supports(int fmt);          // gate_up formats of the 160-row kernels
bool moe_gemm3_down_supports(int fmt);     // down formats
int moe_launch_gemm3_gateup(const uint16_t* x16, const void* w_gate, const void* w_up, int fmt,
                            size_t expert_stride, const int32_t* tiles, int max_tiles, int T,
                            const int32_t* offsets, const int32_t* sorted_pairs, int K, int H,
                            int I, uint16_t* S, hipStream_t st);
// y: f32 rows, or f16 rows (saturated) when y16
int moe_launch_gemm3_down(const uint16_t* S, const void* w_down, int fmt, size_t expert_stride,
                          const int32_t* tiles, int max_tiles, int T, const int32_t* offsets,
                          int H, int I, void* y, int y16, hipStream_t st);

// gemm5.hip: the shared expert's dense GEMMs over all T rows with bf16 weights (f32
// accumulation): gate/up -> S = SiLU(gate) * up (f16 [T, I_s]) from bf16 rows a (a_bf16, bf16
// MFMA) or f16 rows, down -> y (f32 [T, H]).
bool moe_gemm5_supports(int H, int Is);
int moe_launch_gemm5_gateup(const void* a, int a_bf16, const void* w_gate, const void* w_up, int T,
                            int H, int Is, uint16_t* S, hipStream_t st);
int moe_launch_gemm5_down(const uint16_t* S, const void* w_down, int T, int H, int Is, float* y,
                          hipStream_t st);

// gemm5.hip, small T: one block per (64-row tile, narrow weight slab), K split over the waves.
// gate_up also writes gate_prob (sigmoid(x . wsg), NULL: skipped) and x16 (f16(x), NULL: skipped)
bool moe_gemm5s_supports(int H, int Is);
int moe_launch_gemm5s_gateup(const void* x, int x_dtype, const void* w_gate, const void* w_up,
                             const void* wsg, int gate_dtype, int T, int H, int Is, uint16_t* S,
                             float* gate_prob, uint16_t* x16, hipStream_t st);
int moe_launch_gemm5s_down(const uint16_t* S, const void* w_down, int T, int H, int Is, float* y,
                           hipStream_t st);

// gemm4.hip: Q4_K gate_up and down with the weight decode in the MFMA waves (persistent grid,
// direct global->LDS operand loads, two blocks per CU); same tiles (MOE_GEMM3_BM rows),
// arguments and results as the gemm3 launchers for Q4_K, within f32 rounding (another k order).
// Needs H >= 512 (gate_up) and I >= 512 (down).
int moe_launch_gemm4_gateup(const uint16_t* x16, const void* w_gate, const void* w_up,
                            size_t expert_stride, const int32_t* tiles, int max_tiles,
                            const int32_t* offsets, const int32_t* sorted_pairs, int K, int H,
                            int I, uint16_t* S, hipStream_t st);
int moe_launch_gemm4_down(const uint16_t* S, const void* w_down, size_t expert_stride,
                          const int32_t* tiles, int max_tiles, const int32_t* offsets, int H, int I,
                          void* y, int y16, hipStream_t st);
// gemm7.hip: the Q6_K down GEMM in gemm4's form (decode in the MFMA waves, raw super-block bytes
// in LDS half a super-block at a time); same tiles, arguments and results as gemm3's Q6_K down,
// within f32 rounding (another k order). Supported when H % 256 == 0, I % 256 == 0 and the tensor
// and its expert stride are 16-byte aligned (moe_gemm7_down_supports).
bool moe_gemm7_down_supports(const void* w_down, size_t expert_stride, int H, int I);
int moe_launch_gemm7_down(const uint16_t* S, const void* w_down, size_t expert_stride,
                          const int32_t* tiles, int max_tiles, const int32_t* offsets, int H, int I,
                          void* y, int y16, hipStream_t st);

// The small-T shared expert's blocks (shared_small.h), appended to another launch's grid: gate/up
// (with the scalar gate) in the single-launch router's, down in the gemm6 down launch's.
struct MoeShJob {
  int n = 0;                       // shared-expert blocks appended to the launch
  const void* x = nullptr;         // gate/up: x [T, H], read as it is
  int x_dtype = 0;
  const void* wsg = nullptr;       // the scalar gate's row and its dtype
  int gdt = 0;
  float* gate_prob = nullptr;
  const uint16_t* w0 = nullptr;    // gate/up: w_gate [Is, H]; down: w_down [H, Is]
  const uint16_t* w1 = nullptr;    // gate/up: w_up [Is, H]
  uint16_t* S = nullptr;           // gate/up: written; down: read (f16 [T, Is])
  float* y = nullptr;              // down: shared_raw (f32 [T, H])
  int T = 0, H = 0, Is = 0;
};
// gemm6.hip: the same GEMMs for few rows per expert: 32-row tiles (MOE_GEMM6_BM), one block per
// (tile, 256-row slab), activations and nibbles both requested three K steps ahead. sh (NULL or
// n == 0: none): the small-T shared expert's down blocks (4 waves), run after the routed ones.
int moe_launch_gemm6_gateup(const uint16_t* x16, const void* w_gate, const void* w_up,
                            size_t expert_stride, const int32_t* tiles, int max_tiles,
                            const int32_t* offsets, const int32_t* sorted_pairs, int K, int H,
                            int I, uint16_t* S, hipStream_t st);
int moe_launch_gemm6_down(const uint16_t* S, const void* w_down, size_t expert_stride,
                          const int32_t* tiles, int max_tiles, const int32_t* offsets, int H, int I,
                          void* y, int y16, hipStream_t st, const MoeShJob* sh = nullptr);
// shared-expert blocks of the router (gate/up) and down launches for T tokens (32-row token tiles x
// 16-column / 32-column slabs)
inline int moe_shjob_gateup_blocks(int T, int Is) { return (T + 31) / 32 * (Is / 16); }
inline int moe_shjob_down_blocks(int T, int H) { return (T + 31) / 32 * (H / 32); }

// decode GEMV path: S [P, I] f32 (sorted order), then y [P, H] f32
int moe_launch_gemv_gateup(const void* x, int x_dtype, const void* gate, const void* up, size_t estride,
                           int fmt, const int32_t* offsets, const int32_t* sorted_pairs,
                           const int32_t* hit_list, int max_hits, int H, int I, int K, float* S,
                           hipStream_t st);
int moe_launch_gemv_down(const float* S, const void* dn, int fmt, const int32_t* offsets,
                         const int32_t* hit_list, int max_hits, int H, int I, float* y,
                         hipStream_t st);

// MFMA path. A rows come from x (gathered through sorted_pairs / K) or, with tiles == NULL,
// are x rows / S rows 0..T-1 (the shared expert).
// op_bf16 = 0: f16 MFMA operands (default), 1: bf16 operands. S holds 16-bit operands.
int moe_launch_gemm_gateup(const void* x, int x_dtype, const void* w_gate, const void* w_up,
                           int fmt, size_t expert_stride, const int32_t* tiles, int max_tiles,
                           int T, const int32_t* offsets, const int32_t* sorted_pairs, int K,
                           int H, int I, int op_bf16, uint16_t* S, hipStream_t st);
int moe_launch_gemm_down(const uint16_t* S, const void* w_down, int fmt, size_t expert_stride,
                         const int32_t* tiles, int max_tiles, int T, const int32_t* offsets,
                         int H, int I, int op_bf16, float* y, hipStream_t st);

// shared expert
int moe_launch_shared_gemv(const void* x, int x_dtype, const void* wg, const void* wu,
                           const void* wd, int shared_fmt, const void* wsg, int gate_dtype, int T,
                           int H, int Is, float* s_tmp, float* shared_raw, float* gate_prob,
                           hipStream_t st);
// x16 (optional): also the f16 rows of x, as moe_launch_to_f16 writes them
int moe_launch_shared_gate(const void* x, int x_dtype, const void* wsg, int gate_dtype, int T, int H,
                           float* gate_prob, hipStream_t st, uint16_t* x16 = nullptr);

// combine
// y: the per-slot expert rows, f32 or (y16) f16
int moe_launch_combine(const void* y, int y16, const int32_t* pair_pos, const int32_t* ids,
                       const uint16_t* w_bf16, const float* shared_raw, const float* gate_prob,
                       const float* residual, int T, int K, int H, float* out, float* routed_sum,
                       float* shared_out, float* expert_raw, hipStream_t st);

// fused single-token decode (three launches); requires T == 1, K == 8, Q4_K gate_up
struct MoeDecodeLaunch {
  const void* x;
  int x_dtype;
  const float* residual;
  const void* w_router;
  int router_dt = MOE_DT_BF16;             // router weight dtype (bf16 or f32)
  const float* bias;
  const void* gu;                          // gate rows of expert e at gu + e * gu_estride
  const void* gu_up = nullptr;             // up rows likewise (NULL: fused, up = gate + I rows)
  size_t gu_estride = 0;                   // bytes per expert (0: fused, 2 I rows)
  const void* dn;
  int dn_fmt;
  const void *sg, *su, *sd, *ssg;
  int sfmt = MOE_FMT_BF16;                 // shared-expert rows: bf16 or Q8_0
  int ssg_dt = MOE_DT_BF16;                // scalar shared gate dtype (bf16 or f32)
  uint16_t* logits;
  int32_t* ids;
  float* w_f32;
  uint16_t* w_bf16;
  float *s_shared, *gate_prob, *shared_raw, *s_routed, *out, *routed_sum, *shared_out, *expert_raw;
  int* counter;
  int H, I, E, K, Is;
  int ids_out_requested;   // the caller asked for topk_ids / weights: keep torch's slot order
  const float* norm_w;     // post-attention RMSNorm weight [H] f32, or NULL (x is the input)
  float norm_eps;
  // the next layer's routing-independent weights (single-launch layer's L2 warm-up), or NULL
  const void* nx_router = nullptr;      // the next layer's router and norm weights (warm-up hint)
  int nx_router_dt = MOE_DT_BF16;
  const float* nx_norm = nullptr;
};
int moe_launch_decode_fused(const MoeDecodeLaunch& L, hipStream_t st);
// xn[T,H] f32 = (x * f32(1/sqrt(mean_f64(x^2) + eps))) * w   (norm.hip)
int moe_launch_rmsnorm(const void* x, int x_dtype, int T, int H, const float* w, float eps,
                       float* out, hipStream_t st);
int moe_launch_zero_words(int* p, int n, hipStream_t st);
// *out = *word; *word = 0 (one device-scope exchange)
int moe_launch_take_status(int* word, int32_t* out, hipStream_t st);

// The first kSyncBytes of every workspace hold the library's device-side sync words (block
// tickets, the decode layer's epoch, arrival counter and per-XCD tickets, its two exchange
// buffers). They must be zero before the first call (moe_workspace_init); calls keep them
// consistent.
constexpr size_t kSyncBytes = 524288;
// first sync word of the single-launch router's arrival counters (272 words; the decode layer's
// words end before it)
constexpr int kRouterCntWord = 120000;
// single-launch decode layer (decode_layer.hip): 256 co-resident workgroups, model geometry only
bool moe_layer_kernel_supported(int H, int I, int E, int K, int Is, int gu_fmt, int dn_fmt);
size_t moe_layer_exchange_bytes();
int moe_launch_decode_layer(const MoeDecodeLaunch& L, int* sync, uint32_t* xch, hipStream_t st);

// untied lm_head GEMV (lm_head.hip): H = 2048; Q6_K, Q8_0 or BF16 rows; B tokens in passes of 4
bool moe_lm_head_supported(int H, int fmt);
int moe_launch_lm_head(const void* h, int h_dtype, int B, const void* w, int fmt, long long V,
                       const int32_t* row_ids, long long n_rows, float* logits, hipStream_t st);

// workspace carving
struct MoeWs {
  char* p;
  size_t left;
  void* take(size_t bytes) {
    bytes = (bytes + 255) & ~size_t(255);
    if (bytes > left) {
      left = 0;   // sticky: nothing after a failed take (the sync words first of all) is handed out
      return nullptr;
    }
    void* r = p;
    p += bytes;
    left -= bytes;
    return r;
  }
};
