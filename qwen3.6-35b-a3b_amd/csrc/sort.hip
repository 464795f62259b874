// Stable token->expert grouping (speccheck/moe_ref.py:433-439 grouped form; engine/m3_forward.py:
// 448-452): pairs p = t*K + k ordered by expert id, equal ids in ascending p — the permutation
// torch.argsort(ids.flatten(), stable=True) returns. Integer work only, so bit-exact by design.
//
// P <= 64 (decode): one wave ranks every pair directly. P <= 1024: one block runs the three
// phases below. (The block forward at 8 <= T <= 256 with the single-launch router sorts inside
// that launch instead: chain_sort in router.hip, the same positions and tile list.) Otherwise two launches: per-chunk histograms, then per chunk one block that sums
// the histograms itself (totals, scan, its own chunk's start positions) and scatters its chunk
// stably, where ranks inside a 256-pair round come from wave-level id matching (8 ballots on the
// id bits) and a per-wave count table, so no atomics decide any position. sort_chunk() sets the
// chunk length: 512 pairs (two rounds per block) up to 128 chunks, above that the smallest multiple
// of 256 that keeps 128 chunks, so each block reads at most 128 counts per expert. (At 32K pairs
// 512-pair chunks measured 3-4 us faster per config-3 step than 1024-pair ones; 256-pair chunks
// were slower, each block reading four times the counts of the 1024-pair form.)
#include "common.h"
#include "moe_internal.h"

namespace moe {

constexpr int kOneMax = 1024;   // pairs the one-block sort takes
constexpr int kMaxChunks = 128;
// pairs per chunk: a multiple of 256, at most kMaxChunks chunks
__host__ __device__ inline int sort_chunk(int P) {
  const int per = (P + kMaxChunks - 1) / kMaxChunks;
  return per <= 512 ? 512 : (per + 255) / 256 * 256;
}

__global__ __launch_bounds__(64) void k_sort_small(const int32_t* __restrict__ ids, int P, int E,
                                                   int32_t* __restrict__ offsets,
                                                   int32_t* __restrict__ sorted_pairs,
                                                   int32_t* __restrict__ pair_pos,
                                                   int32_t* __restrict__ hit_list) {
  __shared__ int sid[64];
  __shared__ int sfirst[64];
  const int lane = threadIdx.x;
  int e = lane < P ? ids[lane] : 0x7FFFFFFF;
  const bool valid = lane < P && e >= 0 && e < E;   // out-of-range ids are dropped, never indexed
  if (!valid) e = 0x7FFFFFFF;
  sid[lane] = e;
  __syncthreads();
  int rank = 0;
  bool first = valid;
  for (int q = 0; q < P; ++q) {
    const int o = sid[q];
    rank += (o < e) || (o == e && q < lane);
    if (o == e && q < lane) first = false;
  }
  sfirst[lane] = first ? 1 : 0;
  if (valid) {
    sorted_pairs[rank] = lane;
    pair_pos[lane] = rank;
  } else if (lane < P) {
    pair_pos[lane] = -1;
  }
  __syncthreads();
  // hit list: distinct ids ascending
  int dist_below = 0, nhit = 0;
  for (int q = 0; q < P; ++q) {
    if (sfirst[q]) {
      ++nhit;
      if (sid[q] < e) ++dist_below;
    }
  }
  if (first) hit_list[1 + dist_below] = e;
  if (lane == 0) hit_list[0] = nhit;
  // offsets[x] = # pairs with id < x
  for (int x = lane; x <= E; x += 64) {
    int c = 0;
    for (int q = 0; q < P; ++q) c += sid[q] < x;
    offsets[x] = c;
  }
}

// row stride (ints) of the chunk histograms: hist[e][c], rows padded to 16 bytes
__host__ __device__ inline int hist_stride(int nchunks) { return (nchunks + 3) & ~3; }

// phase 1: histogram of each chunk -> hist[e][chunk] (an expert's counts contiguous)
__global__ __launch_bounds__(256) void k_sort_hist(const int32_t* __restrict__ ids, int P, int E,
                                                   int32_t* __restrict__ hist, int hs, int chunk) {
  __shared__ int h[256];
  for (int i = threadIdx.x; i < E; i += 256) h[i] = 0;
  __syncthreads();
  const int base = blockIdx.x * chunk;
  for (int i = threadIdx.x; i < chunk; i += 256) {
    const int p = base + i;
    if (p < P) {
      const int e = ids[p];
      if (e >= 0 && e < E) atomicAdd(&h[e], 1);
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < E; i += 256) hist[(size_t)i * hs + blockIdx.x] = h[i];
  // the row padding reads as zero
  if (blockIdx.x == 0)
    for (int i = threadIdx.x; i < E; i += 256)
      for (int c = gridDim.x; c < hs; ++c) hist[(size_t)i * hs + c] = 0;
}

// block-wide exclusive scan of one int per thread (256 threads): wave scans by lane shuffles, then
// the four wave totals through LDS (two barriers); tmp holds at least 4 ints
__device__ int block_exclusive_scan(int v, int* tmp, int* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int incl = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int n = __shfl_up(incl, o, 64);
    if (lane >= o) incl += n;
  }
  if (lane == 63) tmp[wave] = incl;
  __syncthreads();
  int base = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    base += w < wave ? tmp[w] : 0;
    tot += tmp[w];
  }
  *total = tot;
  __syncthreads();
  return base + incl - v;
}

// Stable scatter of the pairs [base, base + len) given the start position of the chunk's pairs
// of every expert (start_row[e]): ranks inside a 256-pair round come from wave-level id matching
// and per-wave counts, run[e] carries them across rounds. run (LDS, 256 ints) must be zero.
__device__ void scatter_chunk(const int32_t* __restrict__ ids, int P, int E, int base, int len,
                              const int32_t* start_row, int32_t* __restrict__ sorted_pairs,
                              int32_t* __restrict__ pair_pos, int* run, int (*wcnt)[256]) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint64_t lt = (lane == 0) ? 0ull : ((~0ull) >> (64 - lane));
  for (int r = 0; r < len; r += 256) {
    for (int i = tid; i < 4 * 256; i += 256) (&wcnt[0][0])[i] = 0;
    __syncthreads();
    const int p = base + r + tid;
    int e = p < P ? ids[p] : 0;
    const bool valid = p < P && e >= 0 && e < E;
    if (!valid) e = 0;
    if (p < P && !valid) pair_pos[p] = -1;
    uint64_t peers = __ballot(valid);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const bool bit = (e >> b) & 1;
      const uint64_t m = __ballot(bit);
      peers &= bit ? m : ~m;
    }
    const int rank_w = __popcll(peers & lt);
    const bool leader = valid && rank_w == 0;
    if (leader) wcnt[wave][e] = __popcll(peers);
    __syncthreads();
    if (valid) {
      int before = 0;
      for (int w2 = 0; w2 < wave; ++w2) before += wcnt[w2][e];
      const int dest = start_row[e] + run[e] + before + rank_w;
      sorted_pairs[dest] = p;
      pair_pos[p] = dest;
    }
    __syncthreads();
    if (leader) atomicAdd(&run[e], __popcll(peers));
    __syncthreads();
  }
}

// exclusive scan of a 64-bit value over a 256-thread block (wave shuffles, then the four wave
// totals); *total gets the block sum
__device__ uint64_t block_exclusive_scan64(uint64_t v, uint64_t* tmp, uint64_t* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  uint64_t incl = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint64_t n = __shfl_up(incl, o, 64);
    if (lane >= o) incl += n;
  }
  if (lane == 63) tmp[wave] = incl;
  __syncthreads();
  uint64_t base = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    base += w < wave ? tmp[w] : 0;
    tot += tmp[w];
  }
  *total = tot;
  __syncthreads();
  return base + incl - v;
}

// Largest tile count the one-scan builder takes (12-bit fields of a 64-bit scan)
constexpr int kTilesPacked = 4095;

// MFMA work list from the per-expert row counts (thread e of a 256-thread block holds expert e's
// rows and first sorted row): ceil(rows / bm) tiles of bm rows per expert, listed by decreasing
// 32-row group count (full tiles first, then the experts' partial last tiles; within a group
// count by ascending expert, an expert's full tiles before its partial one), so that the work a
// grid takes up last is the smallest. One 64-bit scan carries the five per-group-count prefix
// counts (12 bits each). Needs bm <= 160 and at most kTilesPacked tiles.
__device__ void build_tiles_block(int rows, int first_row, int e, int bm, int32_t* __restrict__ tiles,
                                  uint64_t* tmp) {
  const int ngmax = (bm + 31) / 32;
  const int nfull = rows / bm, rem = rows - nfull * bm;
  const int grem = rem > 0 ? (rem + 31) / 32 : 0;
  const uint64_t packed = ((uint64_t)nfull << (12 * (ngmax - 1))) + (grem ? (1ull << (12 * (grem - 1))) : 0ull);
  uint64_t tot;
  const uint64_t pre = block_exclusive_scan64(packed, tmp, &tot);
  auto field = [](uint64_t v, int g) { return (int)((v >> (12 * (g - 1))) & 4095u); };
  int start[6] = {0, 0, 0, 0, 0, 0};   // start[g]: first position of the tiles with g groups
  int acc = 0;
  for (int g = ngmax; g >= 1; --g) {
    start[g] = acc;
    acc += field(tot, g);
  }
  const int p_full = start[ngmax] + field(pre, ngmax);
  for (int i = 0; i < nfull; ++i) {
    tiles[1 + 2 * (p_full + i)] = e;
    tiles[2 + 2 * (p_full + i)] = first_row + i * bm;
  }
  if (grem) {
    const int p = start[grem] + field(pre, grem) + (grem == ngmax ? nfull : 0);
    tiles[1 + 2 * p] = e;
    tiles[2 + 2 * p] = first_row + nfull * bm;
  }
  if (threadIdx.x == 0) tiles[0] = acc;
}

// phases 2 and 3 in one launch: every block sums the chunk histograms itself (expert totals and
// its own chunk's prefix, 16-byte loads of an expert's contiguous counts), scans the totals, and
// scatters its chunk; block 0 also writes the offsets, the hit list and (tiles != NULL) the MFMA
// tile list of bm-row tiles. hist is only read.
__global__ __launch_bounds__(256) void k_sort_scan_scatter(const int32_t* __restrict__ ids, int P, int E,
                                                           const int32_t* __restrict__ hist, int hs,
                                                           int32_t* __restrict__ offsets,
                                                           int32_t* __restrict__ sorted_pairs,
                                                           int32_t* __restrict__ pair_pos,
                                                           int32_t* __restrict__ hit_list,
                                                           int32_t* __restrict__ tiles, int bm, int chunk) {
  __shared__ int start[256], tmp[256], run[256];
  __shared__ int wcnt[4][256];
  __shared__ uint64_t tmp64[4];
  const int e = threadIdx.x, c0 = blockIdx.x;
  run[e] = 0;
  int tot = 0, pre = 0;
  if (e < E) {
    const int4* row = reinterpret_cast<const int4*>(hist + (size_t)e * hs);
#pragma unroll 8
    for (int q = 0; q < hs / 4; ++q) {
      const int4 v = row[q];
      const int c = 4 * q;
      tot += v.x + v.y + v.z + v.w;
      pre += (c < c0 ? v.x : 0) + (c + 1 < c0 ? v.y : 0) + (c + 2 < c0 ? v.z : 0) + (c + 3 < c0 ? v.w : 0);
    }
  }
  int tsum;
  const int base = block_exclusive_scan(e < E ? tot : 0, tmp, &tsum);
  start[e] = base + pre;
  if (c0 == 0) {
    if (e < E) offsets[e] = base;
    if (e == 0) offsets[E] = tsum;   // == P unless out-of-range ids were dropped
  }
  int hsum;
  const int hidx = block_exclusive_scan((e < E && tot > 0) ? 1 : 0, tmp, &hsum);
  if (c0 == 0) {
    if (e < E && tot > 0) hit_list[1 + hidx] = e;
    if (e == 0) hit_list[0] = hsum;
    if (tiles) build_tiles_block(e < E ? tot : 0, base, e, bm, tiles, tmp64);
  }
  __syncthreads();
  scatter_chunk(ids, P, E, c0 * chunk, chunk, start, sorted_pairs, pair_pos, run, wcnt);
}

// 64 < P <= kOneMax: the three phases in one block (histogram, scan, the one chunk's scatter), so
// a small batch pays one launch instead of three; same positions as the three-kernel form. With
// tiles != NULL the block also writes the MFMA tile list (build_tiles_block).
__global__ __launch_bounds__(256) void k_sort_one(const int32_t* __restrict__ ids, int P, int E,
                                                  int32_t* __restrict__ offsets,
                                                  int32_t* __restrict__ sorted_pairs,
                                                  int32_t* __restrict__ pair_pos,
                                                  int32_t* __restrict__ hit_list,
                                                  int32_t* __restrict__ tiles, int bm) {
  __shared__ int h[256], start[256], tmp[256], run[256];
  __shared__ int wcnt[4][256];
  __shared__ uint64_t tmp64[4];
  const int e = threadIdx.x;
  h[e] = 0;
  run[e] = 0;
  __syncthreads();
  for (int i = threadIdx.x; i < P; i += 256) {
    const int id = ids[i];
    if (id >= 0 && id < E) atomicAdd(&h[id], 1);
  }
  __syncthreads();
  const int tot = e < E ? h[e] : 0;
  int tsum;
  const int base = block_exclusive_scan(tot, tmp, &tsum);
  start[e] = base;
  if (e < E) offsets[e] = base;
  if (e == 0) offsets[E] = tsum;   // == P unless out-of-range ids were dropped
  int hsum;
  const int hidx = block_exclusive_scan((e < E && tot > 0) ? 1 : 0, tmp, &hsum);
  if (e < E && tot > 0) hit_list[1 + hidx] = e;
  if (e == 0) hit_list[0] = hsum;
  if (tiles) build_tiles_block(tot, base, e, bm, tiles, tmp64);
  __syncthreads();
  scatter_chunk(ids, P, E, 0, P, start, sorted_pairs, pair_pos, run, wcnt);
}

// the tile list of build_tiles_block from the expert offsets (E <= 256), one scan
__global__ __launch_bounds__(256) void k_build_tiles_packed(const int32_t* __restrict__ offsets, int E,
                                                            int32_t* __restrict__ tiles, int bm) {
  __shared__ uint64_t tmp64[4];
  const int e = threadIdx.x;
  const int first = e < E ? offsets[e] : 0;
  const int rows = e < E ? offsets[e + 1] - first : 0;
  build_tiles_block(rows, first, e, bm, tiles, tmp64);
}

// MFMA work list: for every hit expert ceil(n_e / BM) tiles of BM sorted rows, listed by
// decreasing 32-row group count (full tiles first, then the experts' partial last tiles; within a
// group count by ascending expert), so that the work a grid takes up last is the smallest.
__global__ __launch_bounds__(256) void k_build_tiles(const int32_t* __restrict__ offsets,
                                                     const int32_t* __restrict__ hit_list,
                                                     int32_t* __restrict__ tiles, int bm) {
  __shared__ int tmp[256];
  const int nhit = hit_list[0];
  const int ngmax = (bm + 31) / 32;
  int written = 0;
  for (int g = ngmax; g >= 1; --g) {
    for (int h0 = 0; h0 < nhit; h0 += 256) {
      const int h = h0 + threadIdx.x;
      int e = 0, nfull = 0, rem = 0, n = 0;
      if (h < nhit) {
        e = hit_list[1 + h];
        const int rows = offsets[e + 1] - offsets[e];
        nfull = rows / bm;
        rem = rows - nfull * bm;
        // full tiles have ngmax groups; the remainder tile ceil(rem / 32)
        n = (g == ngmax ? nfull : 0) + ((rem > 0 && (rem + 31) / 32 == g) ? 1 : 0);
      }
      int tot;
      const int pre = block_exclusive_scan(n, tmp, &tot);
      for (int i = 0; i < n; ++i) {
        const int ti = (g == ngmax && i < nfull) ? i : nfull;   // tile index within the expert
        tiles[1 + 2 * (written + pre + i)] = e;
        tiles[2 + 2 * (written + pre + i)] = offsets[e] + ti * bm;
      }
      written += tot;
    }
  }
  if (threadIdx.x == 0) tiles[0] = written;
}

}  // namespace moe

using namespace moe;

size_t moe_sort_ws_bytes(int P, int E) {
  const size_t nchunks = (size_t)(P + sort_chunk(P) - 1) / sort_chunk(P);
  return ((size_t)hist_stride((int)nchunks) * E * sizeof(int32_t) + 255) & ~size_t(255);
}

int moe_launch_sort(const int32_t* ids, int P, int E, int32_t* offsets, int32_t* sorted_pairs,
                    int32_t* pair_pos, int32_t* hit_list, void* ws, hipStream_t st,
                    int32_t* tiles, int bm) {
  const bool fuse_tiles = tiles && P > 64 && E <= 256 && bm <= 160 &&
                          moe_max_mtiles(P, E, bm) <= kTilesPacked;
  if (P <= 64) {
    hipLaunchKernelGGL(k_sort_small, dim3(1), dim3(64), 0, st, ids, P, E, offsets, sorted_pairs,
                       pair_pos, hit_list);
  } else if (P <= kOneMax) {
    hipLaunchKernelGGL(k_sort_one, dim3(1), dim3(256), 0, st, ids, P, E, offsets, sorted_pairs,
                       pair_pos, hit_list, fuse_tiles ? tiles : nullptr, bm);
  } else {
    const int chunk = sort_chunk(P);
    const int nchunks = (P + chunk - 1) / chunk, hs = hist_stride(nchunks);
    int32_t* hist = reinterpret_cast<int32_t*>(ws);
    hipLaunchKernelGGL(k_sort_hist, dim3(nchunks), dim3(256), 0, st, ids, P, E, hist, hs, chunk);
    hipLaunchKernelGGL(k_sort_scan_scatter, dim3(nchunks), dim3(256), 0, st, ids, P, E, hist, hs,
                       offsets, sorted_pairs, pair_pos, hit_list, fuse_tiles ? tiles : nullptr, bm, chunk);
  }
  if (tiles && !fuse_tiles) return moe_launch_build_tiles(offsets, hit_list, E, P, tiles, st, bm);
  return moe_check_launch("sort");
}

int moe_max_mtiles(int P, int E, int bm) {
  const int hits = P < E ? P : E;
  return (P + bm - 1) / bm + hits;
}

int moe_launch_build_tiles(const int32_t* offsets, const int32_t* hit_list, int E, int P,
                           int32_t* tiles, hipStream_t st, int bm) {
  if (E <= 256 && bm <= 160 && moe_max_mtiles(P, E, bm) <= kTilesPacked)
    hipLaunchKernelGGL(k_build_tiles_packed, dim3(1), dim3(256), 0, st, offsets, E, tiles, bm);
  else
    hipLaunchKernelGGL(k_build_tiles, dim3(1), dim3(256), 0, st, offsets, hit_list, tiles, bm);
  return moe_check_launch("build_tiles");
}
