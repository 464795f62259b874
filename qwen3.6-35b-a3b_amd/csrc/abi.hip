// C-ABI entry points of libmoe_gfx950.so (declared in include/moe_gfx950.h): argument checks,
// workspace carving and stream-ordered launches. No entry point allocates, frees or synchronises.
#include <stdarg.h>
#include <stdio.h>

#include <algorithm>
#include <mutex>

#include "moe_internal.h"

static thread_local char g_err[512] = "";

int moe_set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int moe_check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return moe_set_error(MOE_E_HIP, "%s: %s", what, hipGetErrorString(e));
  return MOE_OK;
}

#define MOE_TRY(expr)            \
  do {                           \
    const int _rc = (expr);      \
    if (_rc != MOE_OK) return _rc; \
  } while (0)

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
static size_t r256(size_t b) { return (b + 255) & ~size_t(255); }

static int check_geom(int T, int H, int I, int E, int K, const char* who) {
  if (T < 1 || H < 1 || I < 1 || E < 1 || K < 1)
    return moe_set_error(MOE_E_ARG, "%s: non-positive dimension (T=%d H=%d I=%d E=%d K=%d)", who, T, H, I, E, K);
  if (E > 256 || K > 16 || K > E || K * 64 <= E)
    return moe_set_error(MOE_E_UNSUPPORTED, "%s: need E <= 256, K <= 16, K <= E and K*64 > E (E=%d K=%d)", who, E, K);
  if (H % 2048 || I % 512)
    return moe_set_error(MOE_E_UNSUPPORTED, "%s: need H %% 2048 == 0 and I %% 512 == 0 (H=%d I=%d)", who, H, I);
  return MOE_OK;
}

static int pick_path(int path, int T, int gate_up_fmt, int down_fmt) {
  if (path == MOE_PATH_GEMV_MULTI) return MOE_PATH_GEMV;
  if (path == MOE_PATH_GEMV || path == MOE_PATH_MFMA || path == MOE_PATH_MFMA_BF16) return path;
  // the GEMV kernels read Q4_K gate_up and GGUF-block down only
  if (gate_up_fmt != MOE_FMT_Q4_K || down_fmt == MOE_FMT_BF16) return MOE_PATH_MFMA;
  // measured crossover (block at 2..24 tokens, the shared expert on the second stream from 7):
  // the GEMV path reads every hit expert once per token group, the MFMA path once per tile
  return T <= 6 ? MOE_PATH_GEMV : MOE_PATH_MFMA;
}

// The grouped paths' shared expert depends on x alone, so from kForkMinT tokens on it runs on a
// library-owned second stream of the device (default priority, non-blocking) beside the router
// and the sort, whose small grids leave most CUs idle; the caller's stream waits for it before
// the routed GEMMs (their persistent grids take every CU). With bf16 rows the shared GEMMs read x
// itself and the routed GEMMs' f16 copy of x is made on that stream after them. The fork and join
// are events, so the pattern is legal under graph capture. One mutex serialises the enqueue
// sequence, because the stream and its two events are shared by every call on the device.
// Below kForkMinT the event round trip costs more than the overlap returns (measured: 2 tokens
// 53 -> 90 us with the fork, 8 tokens 124 -> 116, 64 tokens 184 -> 126)
constexpr int kForkMinT = 7;
constexpr int kMaxDevices = 64;
struct ForkRes {
  hipStream_t s = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
};
static ForkRes g_fork[kMaxDevices];
static std::mutex g_fork_mu;

// called with g_fork_mu held
static int fork_res(ForkRes*& r) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return moe_set_error(MOE_E_HIP, "moe_block_forward: no current device for the shared-expert stream");
  ForkRes& f = g_fork[dev];
  if (!f.s) {
    if (hipStreamCreateWithFlags(&f.s, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreateWithFlags(&f.fork, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&f.join, hipEventDisableTiming) != hipSuccess)
      return moe_set_error(MOE_E_HIP, "moe_block_forward: cannot create the shared-expert stream");
  }
  r = &f;
  return MOE_OK;
}

struct Carve {
  // every piece a T-token forward can need; sizes are upper bounds over both paths
  size_t logits, ids, wf, wb, offsets, sorted, pos, hits, sort_ws, tiles, S, y, sS, sraw, gprob, xn, x16, flag, rscr;
};

static Carve carve_sizes(int T, int H, int I, int E, int K, int Is) {
  const size_t P = (size_t)T * K;
  Carve c;
  c.logits = r256((size_t)T * E * 2);
  c.ids = r256(P * 4);
  c.wf = r256(P * 4);
  c.wb = r256(P * 2);
  c.offsets = r256((size_t)(E + 1) * 4);
  c.sorted = r256(P * 4);
  c.pos = r256(P * 4);
  c.hits = r256((size_t)(E + 1) * 4);
  c.sort_ws = moe_sort_ws_bytes((int)P, E);
  c.tiles = r256((size_t)(1 + 2 * moe_max_mtiles((int)P, E, MOE_GEMM6_BM)) * 4);
  // f32 rows (GEMV path) or f16 rows plus MOE_GEMM3_BM padding rows (the 160-row down kernels
  // read whole tiles past the last row)
  c.S = r256(std::max(P * I * 4, (P + MOE_GEMM3_BM) * I * 2));
  c.y = r256(P * H * 4);
  c.sS = r256((size_t)T * Is * 4);
  c.sraw = r256((size_t)T * H * 4);
  c.gprob = r256((size_t)T * 4);
  c.xn = r256((size_t)T * H * 4);
  c.x16 = r256((size_t)T * H * 2);
  c.flag = 256;
  c.rscr = moe_router_scratch_bytes(T, H, E);
  return c;
}

extern "C" {

int moe_abi_version(void) { return MOE_ABI_VERSION; }

const char* moe_last_error(void) { return g_err; }

size_t moe_workspace_bytes(int T, int H, int I, int E, int K, int I_s) {
  if (T < 1 || E < 1 || K < 1) return 0;
  const Carve c = carve_sizes(T, H, I, E, K, I_s);
  return kSyncBytes + c.logits + c.ids + c.wf + c.wb + c.offsets + c.sorted + c.pos + c.hits +
         c.sort_ws + c.tiles + c.S + c.y + c.sS + c.sraw + c.gprob + c.xn + c.x16 + c.flag + c.rscr;
}

size_t moe_router_workspace_bytes(int T, int H, int E) {
  if (T < 1 || H < 1 || E < 1) return 0;
  return kSyncBytes + r256((size_t)T * E * 2) + moe_router_scratch_bytes(T, H, E);
}

int moe_dequant(const void* blocks, int fmt, int64_t n_elts, void* out, int out_dtype,
                void* stream) {
  if (!blocks || !out) return moe_set_error(MOE_E_ARG, "moe_dequant: NULL pointer");
  if (n_elts <= 0 || n_elts % 256) return moe_set_error(MOE_E_ARG, "moe_dequant: n_elts must be a positive multiple of 256");
  if (out_dtype != MOE_DT_F32 && out_dtype != MOE_DT_BF16) return moe_set_error(MOE_E_ARG, "moe_dequant: bad out_dtype %d", out_dtype);
  if (fmt == MOE_FMT_Q4_K && !aligned16(blocks)) return moe_set_error(MOE_E_ARG, "moe_dequant: Q4_K blocks must be 16-byte aligned");
  if (fmt == MOE_FMT_Q6_K && (reinterpret_cast<uintptr_t>(blocks) & 1u)) return moe_set_error(MOE_E_ARG, "moe_dequant: Q6_K blocks must be 2-byte aligned");
  if (fmt == MOE_FMT_Q5_K && !aligned16(blocks)) return moe_set_error(MOE_E_ARG, "moe_dequant: Q5_K blocks must be 16-byte aligned");
  return moe_launch_dequant(blocks, fmt, n_elts, out, out_dtype, (hipStream_t)stream);
}

int moe_router_topk(const void* x, int x_dtype, const void* w_router, int w_dtype,
                    const float* logit_bias, int T, int H, int E, int K, void* logits_bf16, float* probs,
                    int32_t* topk_ids, float* w_f32, void* w_bf16, void* ws, size_t ws_bytes,
                    void* stream) {
  if (!x || !w_router || !topk_ids || !w_f32 || !w_bf16) return moe_set_error(MOE_E_ARG, "moe_router_topk: NULL pointer");
  if (x_dtype != MOE_DT_F32 && x_dtype != MOE_DT_BF16) return moe_set_error(MOE_E_ARG, "moe_router_topk: bad x_dtype %d", x_dtype);
  if (w_dtype != MOE_DT_F32 && w_dtype != MOE_DT_BF16) return moe_set_error(MOE_E_FORMAT, "moe_router_topk: router weights must be bf16 or f32 (got %d)", w_dtype);
  if (T < 1 || H < 1 || H % 512) return moe_set_error(MOE_E_UNSUPPORTED, "moe_router_topk: need T >= 1 and H %% 512 == 0");
  if (E < 1 || E > 256 || K < 1 || K > 16 || K > E || K * 64 <= E)
    return moe_set_error(MOE_E_UNSUPPORTED, "moe_router_topk: need E <= 256, K <= 16, K*64 > E (E=%d K=%d)", E, K);
  if (!aligned16(x) || !aligned16(w_router)) return moe_set_error(MOE_E_ARG, "moe_router_topk: x and w_router must be 16-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  uint16_t* logits = reinterpret_cast<uint16_t*>(logits_bf16);
  MoeWs w{reinterpret_cast<char*>(ws), ws ? ws_bytes : 0};
  w.take(kSyncBytes);
  if (!logits) {
    logits = reinterpret_cast<uint16_t*>(w.take((size_t)T * E * 2));
    if (!logits) return moe_set_error(MOE_E_WORKSPACE, "moe_router_topk: workspace too small for the logits");
  }
  // room for the int8 matrix-core R1 (large T) or the single-launch R1-R5 (small T), else the
  // f64 one; the bits are the same
  const size_t rsb = moe_router_scratch_bytes(T, H, E);
  void* rscr = w.take(rsb);
  if (rscr && moe_router_chain_supported(T, H, E, K))
    return moe_launch_router_chain(x, x_dtype, w_router, w_dtype, logit_bias, T, H, E, logits, probs,
                                   topk_ids, w_f32, reinterpret_cast<uint16_t*>(w_bf16), nullptr, true,
                                   rscr, reinterpret_cast<int*>(ws), st);
  MOE_TRY(moe_launch_router_logits(x, x_dtype, w_router, w_dtype, logit_bias, T, H, E, logits, rscr, rsb, st));
  return moe_launch_route_topk(logits, T, E, K, probs, topk_ids, w_f32,
                               reinterpret_cast<uint16_t*>(w_bf16), nullptr, st);
}

int moe_sort_permute(const int32_t* topk_ids, int T, int K, int E, int32_t* expert_offsets,
                     int32_t* sorted_pairs, int32_t* pair_pos, int32_t* hit_list, void* ws,
                     size_t ws_bytes, void* stream) {
  if (!topk_ids || !expert_offsets || !sorted_pairs || !pair_pos || !hit_list)
    return moe_set_error(MOE_E_ARG, "moe_sort_permute: NULL pointer");
  if (T < 1 || K < 1 || E < 1 || E > 256) return moe_set_error(MOE_E_UNSUPPORTED, "moe_sort_permute: need T, K >= 1 and 1 <= E <= 256");
  const int P = T * K;
  // the workspace's first kSyncBytes are the sync words every entry point leaves in place
  MoeWs w{reinterpret_cast<char*>(ws), ws ? ws_bytes : 0};
  void* sort_ws = nullptr;
  if (P > 64) {
    w.take(kSyncBytes);
    sort_ws = w.take(moe_sort_ws_bytes(P, E));
    if (!sort_ws)
      return moe_set_error(MOE_E_WORKSPACE, "moe_sort_permute: workspace needs %zu bytes",
                           kSyncBytes + moe_sort_ws_bytes(P, E));
  }
  return moe_launch_sort(topk_ids, P, E, expert_offsets, sorted_pairs, pair_pos, hit_list, sort_ws,
                         (hipStream_t)stream);
}

// x16: the rows already in f16 (the MFMA paths' activation operand), or NULL to convert here
// gate / up: the routed gate and up rows of expert e at gate + e * estride and up + e * estride
// the 160-row kernels for both GEMMs (gemm3 / gemm4)
static bool mfma_v2(int path, int H, int I, int gu_fmt, int dn_fmt) {
  return path == MOE_PATH_MFMA && moe_gemm3_supports(gu_fmt) && moe_gemm3_down_supports(dn_fmt) &&
         H % 256 == 0 && I % 256 == 0;
}
// Q4_K gate_up on gemm4 while the down format has no 160-row kernel (Q6_K): the down GEMM then
// runs on gemm.hip's 64-row tiles
static bool mfma_gu4_mixed(int path, int H, int I, int gu_fmt, int dn_fmt) {
  return path == MOE_PATH_MFMA && gu_fmt == MOE_FMT_Q4_K && H >= 512 && H % 256 == 0 && I % 128 == 0 &&
         !mfma_v2(path, H, I, gu_fmt, dn_fmt);
}

// Q4_K experts with few rows each (up to kSmallRowsMaxT tokens): the 32-row kernels (gemm6.hip),
// which keep three K steps of activations and nibbles in flight per item
constexpr int kSmallRowsMaxT = 256;
static bool mfma_small(int path, int T, int H, int I, int gu_fmt, int dn_fmt) {
  return mfma_v2(path, H, I, gu_fmt, dn_fmt) && gu_fmt == MOE_FMT_Q4_K && dn_fmt == MOE_FMT_Q4_K &&
         T <= kSmallRowsMaxT && H >= 512 && I >= 512;
}

// rows per MFMA tile of the first grouped GEMM experts_impl runs (0: a GEMV path)
static int mfma_tile_rows(int path, int T, int H, int I, int gu_fmt, int dn_fmt) {
  path = pick_path(path, T, gu_fmt, dn_fmt);
  if (path == MOE_PATH_GEMV) return 0;
  if (mfma_small(path, T, H, I, gu_fmt, dn_fmt)) return MOE_GEMM6_BM;
  return (mfma_v2(path, H, I, gu_fmt, dn_fmt) || mfma_gu4_mixed(path, H, I, gu_fmt, dn_fmt)) ? MOE_GEMM3_BM
                                                                                           : MOE_GEMM_BM;
}

// the routed down GEMM writes its rows as f16 (the block forward's combine operand: half the
// bytes written and read back) on the gemm3 / gemm4 path with the combine's K == 8 kernel
static bool y16_rows(int path, int T, int H, int I, int K, int gu_fmt, int dn_fmt) {
  path = pick_path(path, T, gu_fmt, dn_fmt);
  return path != MOE_PATH_GEMV && mfma_v2(path, H, I, gu_fmt, dn_fmt) && K == 8 && H % 4 == 0;
}

// ints of a tile-list buffer that holds the list of any tile height (the shortest tiles: most)
static size_t tile_list_ints(int P, int E) { return 1 + 2 * (size_t)moe_max_mtiles(P, E, MOE_GEMM6_BM); }

// tiles_pre: the tile list of mfma_tile_rows(...) rows, already built in a buffer of
// tile_list_ints(P, E) ints (NULL: built here)
static int experts_impl(const void* x, int x_dtype, const uint16_t* x16, const void* gate,
                        const void* up, size_t estride, int gu_fmt,
                        const void* dn, int dn_fmt, const int32_t* offsets,
                        const int32_t* sorted_pairs, const int32_t* hit_list, int T, int H, int I,
                        int E, int K, int path, void* y, MoeWs& w, hipStream_t st,
                        int32_t* tiles_pre = nullptr, int y16 = 0, const MoeShJob* shd = nullptr) {
  const int P = T * K;
  const int max_hits = P < E ? P : E;
  if (y16 && !y16_rows(path, T, H, I, K, gu_fmt, dn_fmt))
    return moe_set_error(MOE_E_UNSUPPORTED, "moe_experts: f16 expert rows need the gemm3/gemm4 MFMA path");
  path = pick_path(path, T, gu_fmt, dn_fmt);
  float* yf = reinterpret_cast<float*>(y);
  if (path == MOE_PATH_GEMV) {
    float* S = reinterpret_cast<float*>(w.take((size_t)P * I * 4));
    if (!S) return moe_set_error(MOE_E_WORKSPACE, "moe_experts: workspace too small");
    MOE_TRY(moe_launch_gemv_gateup(x, x_dtype, gate, up, estride, gu_fmt, offsets, sorted_pairs, hit_list, max_hits, H, I, K, S, st));
    return moe_launch_gemv_down(S, dn, dn_fmt, offsets, hit_list, max_hits, H, I, yf, st);
  }
  const size_t dn_row = dn_fmt == MOE_FMT_Q4_K ? (size_t)I / 256 * 144 : dn_fmt == MOE_FMT_Q5_K ? (size_t)I / 256 * 176
                      : dn_fmt == MOE_FMT_Q6_K ? (size_t)I / 256 * 210 : (size_t)I * 2;
  if (dn_fmt == MOE_FMT_Q5_K && path == MOE_PATH_MFMA_BF16)
    return moe_set_error(MOE_E_FORMAT, "moe_experts: Q5_K down runs on the GEMV and MFMA (f16) paths");
  const bool v2 = mfma_v2(path, H, I, gu_fmt, dn_fmt);
  const bool gu4 = mfma_gu4_mixed(path, H, I, gu_fmt, dn_fmt);
  const bool small = mfma_small(path, T, H, I, gu_fmt, dn_fmt);
  const int bm = small ? MOE_GEMM6_BM : (v2 || gu4) ? MOE_GEMM3_BM : MOE_GEMM_BM;
  const int max_tiles = moe_max_mtiles(P, E, bm);
  int32_t* tiles = tiles_pre;
  if (!tiles) {
    tiles = reinterpret_cast<int32_t*>(w.take(tile_list_ints(P, E) * 4));
    if (!tiles) return moe_set_error(MOE_E_WORKSPACE, "moe_experts: workspace too small");
    MOE_TRY(moe_launch_build_tiles(offsets, hit_list, E, P, tiles, st, bm));
  }
  uint16_t* S = reinterpret_cast<uint16_t*>(w.take((size_t)(P + MOE_GEMM3_BM) * I * 2));
  if (!S) return moe_set_error(MOE_E_WORKSPACE, "moe_experts: workspace too small");
  if (gu4) {
    if (!x16) {
      uint16_t* c = reinterpret_cast<uint16_t*>(w.take((size_t)T * H * 2));
      if (!c) return moe_set_error(MOE_E_WORKSPACE, "moe_experts: workspace too small");
      MOE_TRY(moe_launch_to_f16(x, x_dtype, (size_t)T * H, c, st));
      x16 = c;
    }
    MOE_TRY(moe_launch_gemm4_gateup(x16, gate, up, estride, tiles, max_tiles, offsets, sorted_pairs,
                                    K, H, I, S, st));
    // the down GEMM's 64-row list replaces the 160-row one in the same buffer (stream order)
    MOE_TRY(moe_launch_build_tiles(offsets, hit_list, E, P, tiles, st, MOE_GEMM_BM));
    return moe_launch_gemm_down(S, dn, dn_fmt, (size_t)H * dn_row, tiles, moe_max_mtiles(P, E, MOE_GEMM_BM), T,
                                offsets, H, I, 0, yf, st);
  }
  if (v2) {
    if (!x16) {
      uint16_t* c = reinterpret_cast<uint16_t*>(w.take((size_t)T * H * 2));
      if (!c) return moe_set_error(MOE_E_WORKSPACE, "moe_experts: workspace too small");
      MOE_TRY(moe_launch_to_f16(x, x_dtype, (size_t)T * H, c, st));
      x16 = c;
    }
    if (small) {
      MOE_TRY(moe_launch_gemm6_gateup(x16, gate, up, estride, tiles, max_tiles, offsets, sorted_pairs,
                                      K, H, I, S, st));
      return moe_launch_gemm6_down(S, dn, (size_t)H * dn_row, tiles, max_tiles, offsets, H, I, y, y16, st, shd);
    }
    // gemm4's persistent item stream needs two super-blocks per item (H, I >= 512)
    if (gu_fmt == MOE_FMT_Q4_K && H >= 512)
      MOE_TRY(moe_launch_gemm4_gateup(x16, gate, up, estride, tiles, max_tiles, offsets, sorted_pairs,
                                      K, H, I, S, st));
    else
      MOE_TRY(moe_launch_gemm3_gateup(x16, gate, up, gu_fmt, estride, tiles, max_tiles, T, offsets,
                                      sorted_pairs, K, H, I, S, st));
    if (dn_fmt == MOE_FMT_Q4_K && I >= 512)
      return moe_launch_gemm4_down(S, dn, (size_t)H * dn_row, tiles, max_tiles, offsets, H, I, y, y16, st);
    if (dn_fmt == MOE_FMT_Q6_K && moe_gemm7_down_supports(dn, (size_t)H * dn_row, H, I))
      return moe_launch_gemm7_down(S, dn, (size_t)H * dn_row, tiles, max_tiles, offsets, H, I, y, y16, st);
    return moe_launch_gemm3_down(S, dn, dn_fmt, (size_t)H * dn_row, tiles, max_tiles, T, offsets, H, I, y, y16, st);
  }
  const int opb = path == MOE_PATH_MFMA_BF16;
  MOE_TRY(moe_launch_gemm_gateup(x, x_dtype, gate, up, gu_fmt, estride, tiles, max_tiles, T, offsets,
                                 sorted_pairs, K, H, I, opb, S, st));
  return moe_launch_gemm_down(S, dn, dn_fmt, (size_t)H * dn_row, tiles, max_tiles, T, offsets, H, I, opb, yf, st);
}

// the formats the resolved routed path reads; checked before any launch is queued
static int check_path_fmt(int rpath, int gu_fmt, int dn_fmt, const char* who) {
  if (rpath == MOE_PATH_GEMV && gu_fmt != MOE_FMT_Q4_K)
    return moe_set_error(MOE_E_FORMAT, "%s: the GEMV path reads Q4_K gate_up only", who);
  if (rpath == MOE_PATH_GEMV && dn_fmt == MOE_FMT_BF16)
    return moe_set_error(MOE_E_FORMAT, "%s: the GEMV path reads Q4_K / Q5_K / Q6_K down only", who);
  if (rpath == MOE_PATH_MFMA_BF16 && dn_fmt == MOE_FMT_Q5_K)
    return moe_set_error(MOE_E_FORMAT, "%s: Q5_K down runs on the GEMV and MFMA (f16) paths", who);
  return MOE_OK;
}

static int check_wfmt(int gu_fmt, int dn_fmt, const void* gu, const void* up, const void* dn, const char* who) {
  if (gu_fmt != MOE_FMT_Q4_K && gu_fmt != MOE_FMT_Q6_K && gu_fmt != MOE_FMT_BF16)
    return moe_set_error(MOE_E_FORMAT, "%s: unsupported gate_up format %d", who, gu_fmt);
  if (dn_fmt != MOE_FMT_Q4_K && dn_fmt != MOE_FMT_Q5_K && dn_fmt != MOE_FMT_Q6_K && dn_fmt != MOE_FMT_BF16)
    return moe_set_error(MOE_E_FORMAT, "%s: unsupported down format %d", who, dn_fmt);
  if (!aligned16(gu) || !aligned16(dn) || (up && !aligned16(up)))
    return moe_set_error(MOE_E_ARG, "%s: expert weights must be 16-byte aligned", who);
  return MOE_OK;
}

static size_t gate_up_row_bytes(int fmt, int H) {
  return fmt == MOE_FMT_Q4_K ? (size_t)H / 256 * 144 : fmt == MOE_FMT_Q6_K ? (size_t)H / 256 * 210 : (size_t)H * 2;
}

// (gate, up, estride) of the routed gate/up rows: a fused record [E][2I rows] (up_q NULL, gate
// rows first) or the separate gate and up tensors [E][I rows] (engine/README.md: the artifact
// stores ffn_gate_exps and ffn_up_exps apart)
static void gate_up_bases(const void* gate_q, const void* up_q, int fmt, int H, int I,
                          const void*& gate, const void*& up, size_t& estride) {
  const size_t row = gate_up_row_bytes(fmt, H);
  gate = gate_q;
  if (up_q) {
    up = up_q;
    estride = (size_t)I * row;
  } else {
    up = reinterpret_cast<const uint8_t*>(gate_q) + (size_t)I * row;
    estride = (size_t)2 * I * row;
  }
}

int moe_experts(const void* x, int x_dtype, const void* gate_up_q, const void* up_q, int gate_up_fmt,
                const void* down_q, int down_fmt, const int32_t* expert_offsets,
                const int32_t* sorted_pairs, const int32_t* hit_list, int T, int H, int I, int E,
                int K, int path, float* y, void* ws, size_t ws_bytes, void* stream) {
  if (!x || !gate_up_q || !down_q || !expert_offsets || !sorted_pairs || !hit_list || !y)
    return moe_set_error(MOE_E_ARG, "moe_experts: NULL pointer");
  if (x_dtype != MOE_DT_F32 && x_dtype != MOE_DT_BF16) return moe_set_error(MOE_E_ARG, "moe_experts: bad x_dtype %d", x_dtype);
  MOE_TRY(check_geom(T, H, I, E, K, "moe_experts"));
  MOE_TRY(check_wfmt(gate_up_fmt, down_fmt, gate_up_q, up_q, down_q, "moe_experts"));
  MOE_TRY(check_path_fmt(pick_path(path, T, gate_up_fmt, down_fmt), gate_up_fmt, down_fmt, "moe_experts"));
  if (!aligned16(x)) return moe_set_error(MOE_E_ARG, "moe_experts: x must be 16-byte aligned");
  MoeWs w{reinterpret_cast<char*>(ws), ws ? ws_bytes : 0};
  w.take(kSyncBytes);
  const void *gate, *up;
  size_t estride;
  gate_up_bases(gate_up_q, up_q, gate_up_fmt, H, I, gate, up, estride);
  return experts_impl(x, x_dtype, nullptr, gate, up, estride, gate_up_fmt, down_q, down_fmt, expert_offsets,
                      sorted_pairs, hit_list, T, H, I, E, K, path, y, w, (hipStream_t)stream);
}

// The small-T shared-expert kernels (narrow slabs, K split over the waves) up to this many tokens;
// above it the 128 x 256 items keep every CU busy and reuse each weight tile over 128 rows.
constexpr int kSharedSkinnyMaxT = 256;
// the shared expert's own path: AUTO takes the GEMV kernels up to 16 tokens, MFMA above
static int shared_path(int path, int T) {
  return path == MOE_PATH_AUTO ? (T <= 16 ? MOE_PATH_GEMV : MOE_PATH_MFMA) : path;
}
static bool shared_skinny(int path, int sfmt, int T, int H, int Is) {
  return shared_path(path, T) == MOE_PATH_MFMA && sfmt == MOE_FMT_BF16 && T <= kSharedSkinnyMaxT &&
         moe_gemm5s_supports(H, Is);
}

// x16: the f16 rows of x when the caller already has them (else NULL); x16_make: where to write
// them for the caller (NULL: not wanted), made by the shared expert's own kernels where they can
static int shared_body(const void* x, int x_dtype, const uint16_t* x16, const void* wg,
                       const void* wu, const void* wd, int sfmt, const void* wsg, int gate_dtype, int T, int H,
                       int Is, int path, float* shared_raw, float* gate_prob, MoeWs& w, hipStream_t st,
                       uint16_t* x16_make, bool& made) {
  path = shared_path(path, T);
  if (path == MOE_PATH_GEMV || path == MOE_PATH_GEMV_MULTI) {
    float* s = reinterpret_cast<float*>(w.take((size_t)T * Is * 4));
    if (!s) return moe_set_error(MOE_E_WORKSPACE, "moe_shared_expert: workspace too small");
    return moe_launch_shared_gemv(x, x_dtype, wg, wu, wd, sfmt, wsg, gate_dtype, T, H, Is, s, shared_raw, gate_prob, st);
  }
  uint16_t* s = reinterpret_cast<uint16_t*>(w.take((size_t)T * Is * 2));
  if (!s) return moe_set_error(MOE_E_WORKSPACE, "moe_shared_expert: workspace too small");
  if (shared_skinny(path, sfmt, T, H, Is)) {
    MOE_TRY(moe_launch_gemm5s_gateup(x, x_dtype, wg, wu, wsg, gate_dtype, T, H, Is, s, gate_prob, x16_make, st));
    made = x16_make != nullptr;
    return moe_launch_gemm5s_down(s, wd, T, H, Is, shared_raw, st);
  }
  // bf16 shared weights on the MFMA path: the dense 128-row kernels, on bf16 rows as they are.
  // With bf16 rows the GEMMs go first and the gate kernel last; it reads every row anyway and
  // writes the f16 rows the caller asked for.
  const bool dense = path == MOE_PATH_MFMA && sfmt == MOE_FMT_BF16 && moe_gemm5_supports(H, Is);
  if (dense && x_dtype == MOE_DT_BF16) {
    MOE_TRY(moe_launch_gemm5_gateup(x, 1, wg, wu, T, H, Is, s, st));
    MOE_TRY(moe_launch_gemm5_down(s, wd, T, H, Is, shared_raw, st));
    made = x16_make != nullptr;
    return moe_launch_shared_gate(x, x_dtype, wsg, gate_dtype, T, H, gate_prob, st, x16_make);
  }
  MOE_TRY(moe_launch_shared_gate(x, x_dtype, wsg, gate_dtype, T, H, gate_prob, st));
  if (dense) {
    if (!x16) {
      uint16_t* c = x16_make ? x16_make : reinterpret_cast<uint16_t*>(w.take((size_t)T * H * 2));
      if (!c) return moe_set_error(MOE_E_WORKSPACE, "moe_shared_expert: workspace too small");
      MOE_TRY(moe_launch_to_f16(x, x_dtype, (size_t)T * H, c, st));
      made = c == x16_make;
      x16 = c;
    }
    MOE_TRY(moe_launch_gemm5_gateup(x16, 0, wg, wu, T, H, Is, s, st));
    return moe_launch_gemm5_down(s, wd, T, H, Is, shared_raw, st);
  }
  // Q8_0 shared weights take the 160-row f16 kernels on either MFMA path
  if ((path == MOE_PATH_MFMA || sfmt == MOE_FMT_Q8_0) && H % 256 == 0 && Is % 256 == 0) {
    if (!x16) {
      uint16_t* c = x16_make ? x16_make : reinterpret_cast<uint16_t*>(w.take((size_t)T * H * 2));
      if (!c) return moe_set_error(MOE_E_WORKSPACE, "moe_shared_expert: workspace too small");
      MOE_TRY(moe_launch_to_f16(x, x_dtype, (size_t)T * H, c, st));
      made = c == x16_make;
      x16 = c;
    }
    MOE_TRY(moe_launch_gemm3_gateup(x16, wg, wu, sfmt, 0, nullptr, 0, T, nullptr, nullptr, 1, H, Is, s, st));
    return moe_launch_gemm3_down(s, wd, sfmt, 0, nullptr, 0, T, nullptr, H, Is, shared_raw, 0, st);
  }
  if (sfmt != MOE_FMT_BF16)
    return moe_set_error(MOE_E_UNSUPPORTED, "moe_shared_expert: Q8_0 shared weights need H and I_s multiples of 256 on the MFMA paths");
  const int opb = path == MOE_PATH_MFMA_BF16;
  MOE_TRY(moe_launch_gemm_gateup(x, x_dtype, wg, wu, MOE_FMT_BF16, 0, nullptr, 0, T, nullptr, nullptr, 1, H, Is, opb, s, st));
  return moe_launch_gemm_down(s, wd, MOE_FMT_BF16, 0, nullptr, 0, T, nullptr, H, Is, opb, shared_raw, st);
}

static int shared_impl(const void* x, int x_dtype, const uint16_t* x16, const void* wg,
                       const void* wu, const void* wd, int sfmt, const void* wsg, int gate_dtype, int T, int H,
                       int Is, int path, float* shared_raw, float* gate_prob, MoeWs& w, hipStream_t st,
                       uint16_t* x16_make = nullptr) {
  bool made = false;
  MOE_TRY(shared_body(x, x_dtype, x16, wg, wu, wd, sfmt, wsg, gate_dtype, T, H, Is, path, shared_raw,
                      gate_prob, w, st, x16_make, made));
  if (x16_make && !made) return moe_launch_to_f16(x, x_dtype, (size_t)T * H, x16_make, st);
  return MOE_OK;
}

static int check_shared_fmt(int shared_fmt, int gate_dtype, const char* who) {
  if (shared_fmt != MOE_FMT_BF16 && shared_fmt != MOE_FMT_Q8_0)
    return moe_set_error(MOE_E_FORMAT, "%s: shared-expert weights must be bf16 or Q8_0 (got %d)", who, shared_fmt);
  if (gate_dtype != MOE_DT_BF16 && gate_dtype != MOE_DT_F32)
    return moe_set_error(MOE_E_FORMAT, "%s: the scalar shared gate must be bf16 or f32 (got %d)", who, gate_dtype);
  return MOE_OK;
}

int moe_shared_expert(const void* x, int x_dtype, const void* w_gate, const void* w_up,
                      const void* w_down, int shared_fmt, const void* w_scalar_gate, int gate_dtype,
                      int T, int H, int I_s, int path, float* shared_raw, float* gate_prob, void* ws,
                      size_t ws_bytes, void* stream) {
  if (!x || !w_gate || !w_up || !w_down || !w_scalar_gate || !shared_raw || !gate_prob)
    return moe_set_error(MOE_E_ARG, "moe_shared_expert: NULL pointer");
  if (x_dtype != MOE_DT_F32 && x_dtype != MOE_DT_BF16) return moe_set_error(MOE_E_ARG, "moe_shared_expert: bad x_dtype %d", x_dtype);
  MOE_TRY(check_shared_fmt(shared_fmt, gate_dtype, "moe_shared_expert"));
  if (T < 1 || H % 2048 || I_s % 512) return moe_set_error(MOE_E_UNSUPPORTED, "moe_shared_expert: need T >= 1, H %% 2048 == 0, I_s %% 512 == 0");
  if (!aligned16(x) || !aligned16(w_gate) || !aligned16(w_up) || !aligned16(w_down) || !aligned16(w_scalar_gate))
    return moe_set_error(MOE_E_ARG, "moe_shared_expert: pointers must be 16-byte aligned");
  MoeWs w{reinterpret_cast<char*>(ws), ws ? ws_bytes : 0};
  w.take(kSyncBytes);
  return shared_impl(x, x_dtype, nullptr, w_gate, w_up, w_down, shared_fmt, w_scalar_gate, gate_dtype, T,
                     H, I_s, path, shared_raw, gate_prob, w, (hipStream_t)stream);
}

int moe_combine(const float* y, const int32_t* pair_pos, const int32_t* topk_ids,
                const void* w_bf16, const float* shared_raw, const float* gate_prob, int T, int K,
                int H, float* out, float* routed_sum, float* shared_out, float* expert_raw,
                void* stream) {
  if (!y || !pair_pos || !topk_ids || !w_bf16 || !shared_raw || !gate_prob || !out)
    return moe_set_error(MOE_E_ARG, "moe_combine: NULL pointer");
  if (T < 1 || K < 1 || K > 16 || H < 1) return moe_set_error(MOE_E_ARG, "moe_combine: bad shape");
  return moe_launch_combine(y, 0, pair_pos, topk_ids, reinterpret_cast<const uint16_t*>(w_bf16),
                            shared_raw, gate_prob, nullptr, T, K, H, out, routed_sum, shared_out,
                            expert_raw, (hipStream_t)stream);
}

static int block_forward_impl(const void* x, int x_dtype, int T, int H, int I, int E, int K, int I_s,
                              const moe_layer_weights& Wt, float norm_eps, int path,
                              const float* residual, float* out, void* logits_bf16,
                              int32_t* topk_ids, void* topk_w_bf16, float* topk_w_f32,
                              float* routed_sum, float* shared_out, float* gate_prob,
                              float* expert_raw, void* ws, size_t ws_bytes, void* stream,
                              const moe_layer_weights* next, bool allow_fork = true) {
  const void* w_router = Wt.w_router;
  const float* logit_bias = Wt.logit_bias;
  const void* gate_up_q = Wt.gate_q;
  const int gate_up_fmt = Wt.gate_up_fmt;
  const void* down_q = Wt.down_q;
  const int down_fmt = Wt.down_fmt;
  const void *ws_gate = Wt.ws_gate, *ws_up = Wt.ws_up, *ws_down = Wt.ws_down;
  const void* ws_scalar_gate = Wt.ws_scalar_gate;
  const float* norm_w = Wt.norm_w;
  if (!x || !w_router || !gate_up_q || !down_q || !ws_gate || !ws_up || !ws_down || !ws_scalar_gate || !out)
    return moe_set_error(MOE_E_ARG, "moe_block_forward: NULL pointer");
  if (x_dtype != MOE_DT_F32 && x_dtype != MOE_DT_BF16) return moe_set_error(MOE_E_ARG, "moe_block_forward: bad x_dtype %d", x_dtype);
  if (Wt.router_dtype != MOE_DT_F32 && Wt.router_dtype != MOE_DT_BF16)
    return moe_set_error(MOE_E_FORMAT, "moe_block_forward: router weights must be bf16 or f32 (got %d)", Wt.router_dtype);
  MOE_TRY(check_shared_fmt(Wt.shared_fmt, Wt.scalar_gate_dtype, "moe_block_forward"));
  MOE_TRY(check_geom(T, H, I, E, K, "moe_block_forward"));
  MOE_TRY(check_wfmt(gate_up_fmt, down_fmt, gate_up_q, Wt.up_q, down_q, "moe_block_forward"));
  const void *gate, *up;
  size_t gu_estride;
  gate_up_bases(gate_up_q, Wt.up_q, gate_up_fmt, H, I, gate, up, gu_estride);
  if (I_s % 512) return moe_set_error(MOE_E_UNSUPPORTED, "moe_block_forward: need I_s %% 512 == 0");
  if (!aligned16(x) || !aligned16(w_router) || !aligned16(ws_gate) || !aligned16(ws_up) || !aligned16(ws_down) || !aligned16(ws_scalar_gate))
    return moe_set_error(MOE_E_ARG, "moe_block_forward: pointers must be 16-byte aligned");
  if (norm_w && (!aligned16(norm_w) || !(norm_eps >= 0.0f) || norm_eps > 1.0f))
    return moe_set_error(MOE_E_ARG, "moe_block_forward: norm_w must be 16-byte aligned and 0 <= norm_eps <= 1");
  const size_t need = moe_workspace_bytes(T, H, I, E, K, I_s);
  if (!ws || ws_bytes < need) return moe_set_error(MOE_E_WORKSPACE, "moe_block_forward: workspace needs %zu bytes", need);
  hipStream_t st = (hipStream_t)stream;
  const int P = T * K;
  MoeWs w{reinterpret_cast<char*>(ws), ws_bytes};
  int* sync = reinterpret_cast<int*>(w.take(kSyncBytes));
  const int rpath = pick_path(path, T, gate_up_fmt, down_fmt);
  MOE_TRY(check_path_fmt(rpath, gate_up_fmt, down_fmt, "moe_block_forward"));
  const bool decode = T == 1 && K == 8 && rpath == MOE_PATH_GEMV && gate_up_fmt == MOE_FMT_Q4_K &&
                      (down_fmt == MOE_FMT_Q4_K || down_fmt == MOE_FMT_Q5_K || down_fmt == MOE_FMT_Q6_K) &&
                      I_s % 128 == 0 && E % 4 == 0;
  const bool one_launch = decode && path != MOE_PATH_GEMV_MULTI &&
                          moe_layer_kernel_supported(H, I, E, K, I_s, gate_up_fmt, down_fmt);
  if (norm_w && !one_launch) {
    // every other path reads the normalized rows from the workspace (f32)
    float* xn = reinterpret_cast<float*>(w.take((size_t)T * H * 4));
    if (!xn) return moe_set_error(MOE_E_WORKSPACE, "moe_block_forward: workspace too small");
    MOE_TRY(moe_launch_rmsnorm(x, x_dtype, T, H, norm_w, norm_eps, xn, st));
    x = xn;
    x_dtype = MOE_DT_F32;
  }
  if (decode) {
    MoeDecodeLaunch L;
    L.x = x; L.x_dtype = x_dtype; L.residual = residual; L.w_router = w_router; L.bias = logit_bias;
    L.router_dt = Wt.router_dtype;
    L.gu = gate; L.gu_up = up; L.gu_estride = gu_estride;
    L.dn = down_q; L.dn_fmt = down_fmt;
    L.sg = ws_gate; L.su = ws_up; L.sd = ws_down; L.sfmt = Wt.shared_fmt;
    L.ssg = ws_scalar_gate; L.ssg_dt = Wt.scalar_gate_dtype;
    L.logits = logits_bf16 ? reinterpret_cast<uint16_t*>(logits_bf16) : reinterpret_cast<uint16_t*>(w.take((size_t)E * 2));
    L.ids = topk_ids ? topk_ids : reinterpret_cast<int32_t*>(w.take(K * 4));
    L.w_f32 = topk_w_f32 ? topk_w_f32 : reinterpret_cast<float*>(w.take(K * 4));
    L.w_bf16 = topk_w_bf16 ? reinterpret_cast<uint16_t*>(topk_w_bf16) : reinterpret_cast<uint16_t*>(w.take(K * 2));
    L.s_shared = reinterpret_cast<float*>(w.take((size_t)I_s * 4));
    L.gate_prob = gate_prob ? gate_prob : reinterpret_cast<float*>(w.take(4));
    L.shared_raw = reinterpret_cast<float*>(w.take((size_t)H * 4));
    L.s_routed = reinterpret_cast<float*>(w.take((size_t)K * I * 4));
    L.out = out; L.routed_sum = routed_sum; L.shared_out = shared_out; L.expert_raw = expert_raw;
    L.counter = sync;
    L.H = H; L.I = I; L.E = E; L.K = K; L.Is = I_s;
    L.ids_out_requested = (topk_ids || topk_w_bf16 || topk_w_f32) ? 1 : 0;
    L.norm_w = one_launch ? norm_w : nullptr;
    L.norm_eps = norm_eps;
    if (next && next->w_router && (next->router_dtype == MOE_DT_BF16 || next->router_dtype == MOE_DT_F32)) {
      L.nx_router = next->w_router;
      L.nx_router_dt = next->router_dtype;
      L.nx_norm = next->norm_w;
    }
    if (!L.logits || !L.ids || !L.w_f32 || !L.w_bf16 || !L.s_shared || !L.gate_prob || !L.shared_raw || !L.s_routed)
      return moe_set_error(MOE_E_WORKSPACE, "moe_block_forward: workspace too small");
    if (one_launch)
      return moe_launch_decode_layer(L, sync, reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(sync) + 256), st);
    return moe_launch_decode_fused(L, st);
  }
  uint16_t* logits = logits_bf16 ? reinterpret_cast<uint16_t*>(logits_bf16) : reinterpret_cast<uint16_t*>(w.take((size_t)T * E * 2));
  // torch's slot order among equal probabilities only matters to a caller that reads the routing
  // (ids, weights) or the per-slot expert rows
  const bool exact_order = topk_ids || topk_w_f32 || topk_w_bf16 || expert_raw;
  int32_t* ids = topk_ids ? topk_ids : reinterpret_cast<int32_t*>(w.take((size_t)P * 4));
  float* wf = topk_w_f32 ? topk_w_f32 : reinterpret_cast<float*>(w.take((size_t)P * 4));
  uint16_t* wb = topk_w_bf16 ? reinterpret_cast<uint16_t*>(topk_w_bf16) : reinterpret_cast<uint16_t*>(w.take((size_t)P * 2));
  int32_t* offsets = reinterpret_cast<int32_t*>(w.take((size_t)(E + 1) * 4));
  int32_t* sorted = reinterpret_cast<int32_t*>(w.take((size_t)P * 4));
  int32_t* pos = reinterpret_cast<int32_t*>(w.take((size_t)P * 4));
  int32_t* hits = reinterpret_cast<int32_t*>(w.take((size_t)(E + 1) * 4));
  void* sort_ws = w.take(moe_sort_ws_bytes(P, E));
  // the per-slot expert rows: f16 where the down GEMM can write them so
  const int y16 = y16_rows(path, T, H, I, K, gate_up_fmt, down_fmt) ? 1 : 0;
  void* y = w.take((size_t)P * H * (y16 ? 2 : 4));
  float* sraw = reinterpret_cast<float*>(w.take((size_t)T * H * 4));
  float* gp = gate_prob ? gate_prob : reinterpret_cast<float*>(w.take((size_t)T * 4));
  if (!logits || !ids || !wf || !wb || !offsets || !sorted || !pos || !hits || !y || !sraw || !gp)
    return moe_set_error(MOE_E_WORKSPACE, "moe_block_forward: workspace too small");
  // the grouped GEMMs' tile list, built by the sort
  const int bm = mfma_tile_rows(path, T, H, I, gate_up_fmt, down_fmt);
  int32_t* tiles = nullptr;
  if (bm) {
    tiles = reinterpret_cast<int32_t*>(w.take(tile_list_ints(P, E) * 4));
    if (!tiles) return moe_set_error(MOE_E_WORKSPACE, "moe_block_forward: workspace too small");
  }
  // the MFMA path's f16 activation operand, converted once for the shared and routed GEMMs;
  // with bf16 rows and the shared expert forked, the shared GEMMs read the rows as they are and
  // the conversion runs on the shared expert's stream after them (off the router's path)
  const bool fork = T >= kForkMinT && allow_fork;
  // Few rows per expert (the 32-row routed kernels) with the narrow-slab shared expert: no second
  // stream. The single-launch router also writes the f16 copy of x and runs the shared gate/up
  // blocks, and the shared down blocks run inside the routed down launch: both grids leave CUs
  // idle at this size, and the fork and join cost more than the shared expert's time left after
  // that overlap.
  const bool fuse = rpath == MOE_PATH_MFMA && Wt.shared_fmt == MOE_FMT_BF16 && H % 2048 == 0 &&
                    I_s % 256 == 0 && mfma_small(rpath, T, H, I, gate_up_fmt, down_fmt) &&
                    shared_skinny(path, Wt.shared_fmt, T, H, I_s) && moe_router_chain_supported(T, H, E, K);
  uint16_t* x16 = nullptr;
  bool x16_late = false;
  if (rpath == MOE_PATH_MFMA) {
    x16 = reinterpret_cast<uint16_t*>(w.take((size_t)T * H * 2));
    if (!x16) return moe_set_error(MOE_E_WORKSPACE, "moe_block_forward: workspace too small");
    // made on the shared expert's stream: beside (or after) its GEMMs, off the router's path
    x16_late = !fuse && fork && Wt.shared_fmt == MOE_FMT_BF16 &&
               (x_dtype == MOE_DT_BF16 || shared_skinny(path, Wt.shared_fmt, T, H, I_s));
    if (!x16_late && !fuse) MOE_TRY(moe_launch_to_f16(x, x_dtype, (size_t)T * H, x16, st));
  }
  if (fuse) {
    uint16_t* ssh = reinterpret_cast<uint16_t*>(w.take((size_t)T * I_s * 2));
    MoeWs wr = w;   // the router's scratch is dead before the experts take theirs (same stream)
    const size_t rsb = moe_router_scratch_bytes(T, H, E);
    void* rscr = wr.take(rsb);
    if (!ssh || !rscr) return moe_set_error(MOE_E_WORKSPACE, "moe_block_forward: workspace too small");
    // the shared gate/up (and scalar gate) as extra blocks of the router launch, which leaves CUs
    // idle once its partial tiles are in; the shared down as extra blocks of the routed down
    MoeShJob g, d;
    g.n = moe_shjob_gateup_blocks(T, I_s);
    g.x = x; g.x_dtype = x_dtype; g.wsg = ws_scalar_gate; g.gdt = Wt.scalar_gate_dtype;
    g.gate_prob = gp; g.w0 = reinterpret_cast<const uint16_t*>(ws_gate);
    g.w1 = reinterpret_cast<const uint16_t*>(ws_up); g.S = ssh; g.T = T; g.H = H; g.Is = I_s;
    d.n = moe_shjob_down_blocks(T, H);
    d.w0 = reinterpret_cast<const uint16_t*>(ws_down); d.S = ssh; d.y = sraw; d.T = T; d.H = H; d.Is = I_s;
    // the sort and the tile list inside the router launch, by its last group to finish routing
    MoeSortJob sj;
    if (tiles && bm >= 32 && bm <= 160) {
      sj.P = P; sj.offsets = offsets; sj.sorted = sorted; sj.pos = pos; sj.hits = hits;
      sj.tiles = tiles; sj.bm = bm;
    }
    MOE_TRY(moe_launch_router_chain(x, x_dtype, w_router, Wt.router_dtype, logit_bias, T, H, E, logits,
                                    nullptr, ids, wf, wb, nullptr, exact_order, rscr, sync, st, x16, &g, &sj));
    if (!sj.P) MOE_TRY(moe_launch_sort(ids, P, E, offsets, sorted, pos, hits, sort_ws, st, tiles, bm));
    MOE_TRY(experts_impl(x, x_dtype, x16, gate, up, gu_estride, gate_up_fmt, down_q, down_fmt, offsets,
                         sorted, hits, T, H, I, E, K, path, y, w, st, tiles, y16, &d));
    return moe_launch_combine(y, y16, pos, ids, wb, sraw, gp, residual, T, K, H, out, routed_sum,
                              shared_out, expert_raw, st);
  }
  if (!fork) {
    MOE_TRY(moe_launch_router_logits(x, x_dtype, w_router, Wt.router_dtype, logit_bias, T, H, E, logits, nullptr, 0, st));
    MOE_TRY(moe_launch_route_topk(logits, T, E, K, nullptr, ids, wf, wb, nullptr, st, exact_order));
    MOE_TRY(moe_launch_sort(ids, P, E, offsets, sorted, pos, hits, sort_ws, st, tiles, bm));
    MoeWs w2 = w;   // the shared expert's scratch is dead before the experts' is taken
    MOE_TRY(shared_impl(x, x_dtype, x16, ws_gate, ws_up, ws_down, Wt.shared_fmt, ws_scalar_gate,
                        Wt.scalar_gate_dtype, T, H, I_s, path, sraw, gp, w2, st));
    MOE_TRY(experts_impl(x, x_dtype, x16, gate, up, gu_estride, gate_up_fmt, down_q, down_fmt, offsets, sorted,
                         hits, T, H, I, E, K, path, y, w, st, tiles, y16));
    return moe_launch_combine(y, y16, pos, ids, wb, sraw, gp, residual, T, K, H, out, routed_sum,
                              shared_out, expert_raw, st);
  }
  // the shared expert on the second stream, its scratch taken before (and disjoint from) the
  // routed experts'; the join is enqueued on every path out, so the caller's stream never runs
  // ahead of work still reading this call's workspace
  std::lock_guard<std::mutex> lock(g_fork_mu);
  ForkRes* f = nullptr;
  MOE_TRY(fork_res(f));
  if (hipEventRecord(f->fork, st) != hipSuccess || hipStreamWaitEvent(f->s, f->fork, 0) != hipSuccess)
    return moe_set_error(MOE_E_HIP, "moe_block_forward: cannot fork the shared-expert stream");
  int rc = shared_impl(x, x_dtype, x16_late ? nullptr : x16, ws_gate, ws_up, ws_down, Wt.shared_fmt,
                       ws_scalar_gate, Wt.scalar_gate_dtype, T, H, I_s, path, sraw, gp, w, f->s,
                       x16_late ? x16 : nullptr);
  // the router's scratch is dead before the experts take theirs (same stream)
  MoeWs wr = w;
  const size_t rsb = moe_router_scratch_bytes(T, H, E);
  void* rscr = wr.take(rsb);
  if (rc == MOE_OK && rscr && moe_router_chain_supported(T, H, E, K)) {
    rc = moe_launch_router_chain(x, x_dtype, w_router, Wt.router_dtype, logit_bias, T, H, E, logits,
                                 nullptr, ids, wf, wb, nullptr, exact_order, rscr, sync, st);
  } else {
    if (rc == MOE_OK) rc = moe_launch_router_logits(x, x_dtype, w_router, Wt.router_dtype, logit_bias, T, H, E, logits, rscr, rsb, st);
    if (rc == MOE_OK) rc = moe_launch_route_topk(logits, T, E, K, nullptr, ids, wf, wb, nullptr, st, exact_order);
  }
  if (rc == MOE_OK) rc = moe_launch_sort(ids, P, E, offsets, sorted, pos, hits, sort_ws, st, tiles, bm);
  // joined before the routed GEMMs: their persistent grids take every CU and each block owns a
  // fixed share of the items, so a block kept waiting by a still-running shared-expert kernel
  // would stretch the whole grid
  if (hipEventRecord(f->join, f->s) != hipSuccess || hipStreamWaitEvent(st, f->join, 0) != hipSuccess)
    return moe_set_error(MOE_E_HIP, "moe_block_forward: cannot join the shared-expert stream");
  if (rc == MOE_OK)
    rc = experts_impl(x, x_dtype, x16, gate, up, gu_estride, gate_up_fmt, down_q, down_fmt, offsets,
                      sorted, hits, T, H, I, E, K, path, y, w, st, tiles, y16);
  if (rc != MOE_OK) return rc;
  return moe_launch_combine(y, y16, pos, ids, wb, sraw, gp, residual, T, K, H, out, routed_sum,
                            shared_out, expert_raw, st);
}

static moe_layer_weights bf16_layer(const float* norm_w, const void* w_router, const float* logit_bias,
                                    const void* gate_up_q, int gate_up_fmt, const void* down_q,
                                    int down_fmt, const void* ws_gate, const void* ws_up,
                                    const void* ws_down, const void* ws_scalar_gate) {
  moe_layer_weights W;
  W.w_router = w_router; W.router_dtype = MOE_DT_BF16; W.logit_bias = logit_bias;
  W.gate_q = gate_up_q; W.up_q = nullptr; W.gate_up_fmt = gate_up_fmt;
  W.down_q = down_q; W.down_fmt = down_fmt;
  W.ws_gate = ws_gate; W.ws_up = ws_up; W.ws_down = ws_down; W.shared_fmt = MOE_FMT_BF16;
  W.ws_scalar_gate = ws_scalar_gate; W.scalar_gate_dtype = MOE_DT_BF16;
  W.norm_w = norm_w;
  return W;
}

int moe_block_forward(const void* x, int x_dtype, int T, int H, int I, int E, int K, int I_s,
                      const float* norm_w, float norm_eps,
                      const void* w_router, const float* logit_bias, const void* gate_up_q,
                      int gate_up_fmt, const void* down_q, int down_fmt, const void* ws_gate,
                      const void* ws_up, const void* ws_down, const void* ws_scalar_gate,
                      int path, const float* residual, float* out, void* logits_bf16,
                      int32_t* topk_ids, void* topk_w_bf16, float* topk_w_f32, float* routed_sum,
                      float* shared_out, float* gate_prob, float* expert_raw, void* ws,
                      size_t ws_bytes, void* stream) {
  const moe_layer_weights W = bf16_layer(norm_w, w_router, logit_bias, gate_up_q, gate_up_fmt, down_q,
                                         down_fmt, ws_gate, ws_up, ws_down, ws_scalar_gate);
  return block_forward_impl(x, x_dtype, T, H, I, E, K, I_s, W, norm_eps, path, residual, out, logits_bf16,
                            topk_ids, topk_w_bf16, topk_w_f32, routed_sum, shared_out, gate_prob,
                            expert_raw, ws, ws_bytes, stream, nullptr);
}

int moe_block_forward_prefetch(const void* x, int x_dtype, int T, int H, int I, int E, int K, int I_s,
                      const float* norm_w, float norm_eps,
                      const void* w_router, const float* logit_bias, const void* gate_up_q,
                      int gate_up_fmt, const void* down_q, int down_fmt, const void* ws_gate,
                      const void* ws_up, const void* ws_down, const void* ws_scalar_gate,
                      int path, const float* residual, float* out, void* logits_bf16,
                      int32_t* topk_ids, void* topk_w_bf16, float* topk_w_f32, float* routed_sum,
                      float* shared_out, float* gate_prob, float* expert_raw, void* ws,
                      size_t ws_bytes, void* stream,
                               const moe_next_layer* next) {
  const moe_layer_weights W = bf16_layer(norm_w, w_router, logit_bias, gate_up_q, gate_up_fmt, down_q,
                                         down_fmt, ws_gate, ws_up, ws_down, ws_scalar_gate);
  moe_layer_weights N{};
  if (next)
    N = bf16_layer(next->norm_w, next->w_router, nullptr, nullptr, MOE_FMT_Q4_K, nullptr, MOE_FMT_Q4_K,
                   nullptr, nullptr, nullptr, nullptr);
  return block_forward_impl(x, x_dtype, T, H, I, E, K, I_s, W, norm_eps, path, residual, out, logits_bf16,
                            topk_ids, topk_w_bf16, topk_w_f32, routed_sum, shared_out, gate_prob,
                            expert_raw, ws, ws_bytes, stream, next ? &N : nullptr);
}

int moe_block_forward_w(const void* x, int x_dtype, int T, int H, int I, int E, int K, int I_s,
                        const moe_layer_weights* w, float norm_eps, int path, const float* residual,
                        float* out, void* logits_bf16, int32_t* topk_ids, void* topk_w_bf16,
                        float* topk_w_f32, float* routed_sum, float* shared_out, float* gate_prob,
                        float* expert_raw, void* ws, size_t ws_bytes, void* stream,
                        const moe_layer_weights* next) {
  if (!w) return moe_set_error(MOE_E_ARG, "moe_block_forward_w: NULL weights");
  return block_forward_impl(x, x_dtype, T, H, I, E, K, I_s, *w, norm_eps, path, residual, out, logits_bf16,
                            topk_ids, topk_w_bf16, topk_w_f32, routed_sum, shared_out, gate_prob,
                            expert_raw, ws, ws_bytes, stream, next);
}

}  // extern "C"

// ------------------------------------------------------------------ the allocation-free entry --
// moe_block_forward_w_noalloc's scratch: one array per device (each GPU the library runs on holds
// its own copy until the process ends). Host code never passes `scratch` itself to a kernel (its
// name is a host-side stand-in there): the device address comes from hipGetSymbolAddress, once
// per device, on that device's first call, and is kept per device.
static __device__ __align__(256) unsigned char scratch[MOE_NOALLOC_SCRATCH_BYTES];

struct ScratchDev {
  void* ptr = nullptr;      // the device's copy of `scratch`
  bool zeroed = false;      // its sync words cleared (stream-ordered before the first use)
};
static ScratchDev g_scratch[kMaxDevices];
static std::mutex g_scratch_mu;

static int scratch_for_device(hipStream_t st, void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return moe_set_error(MOE_E_HIP, "moe_block_forward_w_noalloc: no current device");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  ScratchDev& d = g_scratch[dev];
  if (!d.ptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return moe_set_error(MOE_E_HIP, "moe_block_forward_w_noalloc: hipGetSymbolAddress(scratch) on device %d: %s",
                           dev, hipGetErrorString(e));
    d.ptr = p;
  }
  if (!d.zeroed) {
    // the sync words must start at zero; every later call leaves them valid for the next
    MOE_TRY(moe_launch_zero_words(reinterpret_cast<int*>(d.ptr), (int)(kSyncBytes / 4), st));
    d.zeroed = true;
  }
  *out = d.ptr;
  return MOE_OK;
}

extern "C" {

int moe_block_forward_w_noalloc(const void* x, int x_dtype, int T, int H, int I, int E, int K, int I_s,
                                const moe_layer_weights* w, float norm_eps, int path, const float* residual,
                                float* out, void* logits_bf16, int32_t* topk_ids, void* topk_w_bf16,
                                float* topk_w_f32, float* routed_sum, float* shared_out, float* gate_prob,
                                float* expert_raw, void* stream, const moe_layer_weights* next) {
  if (!w) return moe_set_error(MOE_E_ARG, "moe_block_forward_w_noalloc: NULL weights");
  MOE_TRY(check_geom(T, H, I, E, K, "moe_block_forward_w_noalloc"));
  const size_t need = moe_workspace_bytes(T, H, I, E, K, I_s);
  if (need > (size_t)MOE_NOALLOC_SCRATCH_BYTES)
    return moe_set_error(MOE_E_WORKSPACE,
                         "moe_block_forward_w_noalloc: a %d-token step needs %zu scratch bytes, the static "
                         "scratch holds %zu (at most %d tokens at H=2048, I=512, E=256, K=8, I_s=512)",
                         T, need, (size_t)MOE_NOALLOC_SCRATCH_BYTES, MOE_NOALLOC_MAX_T);
  hipStream_t st = (hipStream_t)stream;
  void* ws = nullptr;
  MOE_TRY(scratch_for_device(st, &ws));
  // one stream: the shared expert runs on the caller's stream (the fork's second stream and
  // events would be created on first use)
  return block_forward_impl(x, x_dtype, T, H, I, E, K, I_s, *w, norm_eps, path, residual, out, logits_bf16,
                            topk_ids, topk_w_bf16, topk_w_f32, routed_sum, shared_out, gate_prob,
                            expert_raw, ws, (size_t)MOE_NOALLOC_SCRATCH_BYTES, stream, next, false);
}

int moe_lm_head(const void* h, int h_dtype, int B, int H, const void* w, int w_fmt, int64_t V,
                const int32_t* row_ids, int64_t n_rows, float* logits, void* stream) {
  if (!h || !w || !logits) return moe_set_error(MOE_E_ARG, "moe_lm_head: NULL pointer");
  if (h_dtype != MOE_DT_F32 && h_dtype != MOE_DT_BF16) return moe_set_error(MOE_E_ARG, "moe_lm_head: bad h_dtype %d", h_dtype);
  if (w_fmt != MOE_FMT_Q6_K && w_fmt != MOE_FMT_Q8_0 && w_fmt != MOE_FMT_BF16)
    return moe_set_error(MOE_E_FORMAT, "moe_lm_head: table format %d (want Q6_K, Q8_0 or BF16)", w_fmt);
  if (B < 1 || B > 8 || V < 1 || n_rows < 1 || (!row_ids && n_rows > V))
    return moe_set_error(MOE_E_ARG, "moe_lm_head: need 1 <= B <= 8, V >= 1, 1 <= n_rows (<= V when dense)");
  if (!moe_lm_head_supported(H, w_fmt)) return moe_set_error(MOE_E_UNSUPPORTED, "moe_lm_head: need H == 2048 (got %d)", H);
  if (!aligned16(w) || (reinterpret_cast<uintptr_t>(h) & (h_dtype == MOE_DT_F32 ? 3u : 1u)) ||
      (reinterpret_cast<uintptr_t>(logits) & 3u) || (row_ids && (reinterpret_cast<uintptr_t>(row_ids) & 3u)))
    return moe_set_error(MOE_E_ARG, "moe_lm_head: W must be 16-byte aligned, h / logits / row_ids element aligned");
  return moe_launch_lm_head(h, h_dtype, B, w, w_fmt, (long long)V, row_ids, (long long)n_rows, logits,
                            (hipStream_t)stream);
}

int moe_workspace_status(void* ws, size_t ws_bytes, int32_t* status, void* stream) {
  if (!ws || ws_bytes < kSyncBytes) return moe_set_error(MOE_E_ARG, "moe_workspace_status: workspace smaller than %zu bytes", kSyncBytes);
  if (!status || (reinterpret_cast<uintptr_t>(status) & 3u)) return moe_set_error(MOE_E_ARG, "moe_workspace_status: status must be an aligned int32 pointer");
  return moe_launch_take_status(reinterpret_cast<int*>(ws) + MOE_STATUS_WORD, status, (hipStream_t)stream);
}

int moe_workspace_init(void* ws, size_t ws_bytes, void* stream) {
  if (!ws || ws_bytes < kSyncBytes) return moe_set_error(MOE_E_ARG, "moe_workspace_init: workspace smaller than %zu bytes", kSyncBytes);
  return moe_launch_zero_words(reinterpret_cast<int*>(ws), (int)(kSyncBytes / 4), (hipStream_t)stream);
}

}  // extern "C"
