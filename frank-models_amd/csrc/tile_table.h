// Device code of the per-launch tile schedule of the 256x256-tile grouped
// GEMM (gemm_tiled256.hip), shared by the GEMM's own one-block table kernel
// and the permutation kernels, which build it beside their scatter
// (permute.hip) so that it costs no launch of its own.
//
// The GEMM's in-kernel schedule gives each XCD an equal count of row tiles;
// with skewed expert row counts that leaves whole XCDs short of work and
// each XCD's last round partly empty.  The table deals the work longest
// first instead: a chunk is one (K piece, column group of group_cols tiles,
// expert) with all the expert's row tiles, costed per row tile as
// 375 + rows (a full tile 631: fixed setup, prologue, epilogue and weight
// stream, plus its rows' MFMAs), scaled by the piece's share of the K
// stages (the two pieces of a split may differ).  Chunks are sorted by cost into 255
// buckets (a stable counting sort, largest first; empty chunks last) and
// dealt to the XCDs in snake order (0..7, 7..0, ...); each XCD runs its
// chunks in that order, a chunk's tiles row tile by row tile over its
// columns, so tiles sharing token rows or a weight slab stay on one L2.
// Entry 1 + b of the table is hardware block b's tile (XCD b % 8, position
// b / 8 in that XCD's list): {expert, first row, rows, column | split << 16},
// expert -1 for no tile, kTakeFromPool for a block that takes the next tile
// of the shared pool (entries 1 + 8 * (bpx + steal) on; entry 0 holds the
// pool's size and the claim counter, cleared here).  If an XCD's list
// outgrows the grid, every entry reads -2 and the GEMM falls back to its
// in-kernel schedule.
#pragma once
#include "common.h"
#include "launch.h"
#include "permute_block.h"

namespace fmoe {
namespace {
namespace ttab {

constexpr int kBM = 256;        // assignment rows per tile
constexpr int kPoolDiv = 12;    // 1/12 of each XCD's list (its tail) goes to the shared pool
constexpr int kTakeFromPool = -3;  // block entry: take the next tile of the pool
constexpr int kChunks = 2048;   // chunks a table covers (permute_block's limit)
constexpr int kBuckets = 256;
constexpr int kMaxExperts = 256;
static_assert(kMaxExperts <= perm::kThreads, "one thread per expert");

__host__ __device__ inline int blocks_per_xcd(int row_tiles_bound, int n_col, int ksplit) {
  const int per = (row_tiles_bound * n_col * ksplit + 7) / 8;
  return per + per / 4 + 1;
}

// Blocks per XCD beyond bpx that take their tile from the pool: the pool
// holds at most 8 * bpx / kPoolDiv tiles, within its 4 * steal entries.
__host__ __device__ inline int steal_per_xcd(int bpx) { return (bpx + 5) / 6; }
static_assert(kPoolDiv >= 12, "the pool's entries: 4 * steal_per_xcd(bpx) >= 8 * bpx / kPoolDiv");

// Column tiles per chunk.  A chunk's tiles run side by side on one XCD; 8
// columns x an expert's ~4 row tiles share more of each stage's token rows
// and weight slabs in L2 than 4 x 4 (measured at Mixtral's gate/up, 112
// columns: 5.08 against 6.63 GB fetched per launch, the same time), but on
// a narrow GEMM the coarser chunks balance the XCDs worse (Mixtral's down,
// 16 columns: 766 against 754 us; 2-column chunks there: 740 against 737 us).
__host__ __device__ inline int group_cols(int n_col) { return n_col >= 64 ? 8 : 4; }

// Chunks of a table (K splits x column groups x experts).
__host__ __device__ inline int64_t n_chunks(int n_col, int ksplit, int n_expert) {
  const int gc = group_cols(n_col);
  return static_cast<int64_t>(ksplit) * ((n_col + gc - 1) / gc) * n_expert;
}

__device__ __forceinline__ int tile_cost(int rows) { return 375 + rows; }

// K stages of piece sp of a tile split ksplit ways (the 256-tile kernel's
// split_boundary: a two-way split at first64 / 64 of the stages, rounded down
// to even; otherwise equal pieces).
__device__ __forceinline__ int piece_stages(int kblocks, int ksplit, int first64, int sp) {
  auto bound = [&](int s) {
    if (s >= ksplit) return kblocks;
    if (ksplit == 2 && s == 1) return (kblocks * first64 / 64) & ~1;
    return (s * kblocks / ksplit) & ~1;
  };
  return bound(sp + 1) - bound(sp);
}

// Position in the sorted chunk order of the m-th chunk XCD x receives.
__device__ __forceinline__ int snake_pos(int x, int m) { return m * 8 + ((m & 1) ? 7 - x : x); }

// The table of a GEMM over n_col column tiles and ksplit K splits whose
// experts hold e_rows[e] rows (LDS, n_expert <= kMaxExperts entries, visible
// to the whole block), in expert order; 8 * bpx entries.  Called by every
// thread of a perm::kThreads block; with n_parts blocks on one table, each
// sorts the chunks and writes part `part` of the entries.
__device__ __forceinline__ void build(const int* e_rows_in, int n_expert, const TileTableReq& req,
                                      int4* __restrict__ table, int part = 0, int n_parts = 1) {
  const int n_col = req.n_col, ksplit = req.ksplit, bpx = req.bpx;
  const int kblocks = req.kblocks > 0 ? req.kblocks : ksplit;
  // a chunk's cost scales with its K piece (the pieces of a two-way split may differ)
  int max_piece = 0;
  for (int sp = 0; sp < ksplit; ++sp) max_piece = max(max_piece, piece_stages(kblocks, ksplit, req.ksplit_first64, sp));
  __shared__ int e_off[kMaxExperts], e_rows[kMaxExperts], e_cost[kMaxExperts];
  __shared__ int bucket[kChunks], srt[kChunks], boff[kBuckets + 1], berr;
  __shared__ int pref[8][kChunks / 8 + 1];
  __shared__ int max_cost;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1), wave = tid / kWave;
  const int gcols = group_cols(n_col);
  const int n_groups = (n_col + gcols - 1) / gcols;
  const int n_chunks = ksplit * n_groups * n_expert;
  if (wave == 0) {
    // e_off: exclusive scan of the row counts; max_cost: the largest chunk's cost
    int running = 0, mc = 0;
    for (int c = 0; c < n_expert; c += kWave) {
      const int e = c + lane;
      const int r = e < n_expert ? e_rows_in[e] : 0;
      const int incl = wave_inclusive_scan(r);
      const int nt = (r + kBM - 1) / kBM;
      const int cost = nt == 0 ? 0 : (nt - 1) * tile_cost(kBM) + tile_cost(r - (nt - 1) * kBM);
      if (e < n_expert) {
        e_off[e] = running + incl - r;
        e_rows[e] = r;
        e_cost[e] = cost;
      }
      mc = max(mc, cost);
      running += __shfl(incl, kWave - 1, kWave);
    }
    for (int o = kWave / 2; o > 0; o >>= 1) mc = max(mc, __shfl_xor(mc, o, kWave));
    if (lane == 0) max_cost = static_cast<int>(static_cast<int64_t>(mc) * gcols * max_piece / kblocks);
  }
  __syncthreads();
  // bucket 0 = the most expensive chunks, kBuckets - 2 the cheapest, kBuckets - 1 empty
  for (int c = tid; c < n_chunks; c += perm::kThreads) {
    const int e = c % n_expert, g = (c / n_expert) % n_groups, sp = c / (n_expert * n_groups);
    const int cost = static_cast<int>(static_cast<int64_t>(e_cost[e]) * min(gcols, n_col - g * gcols) *
                                      piece_stages(kblocks, ksplit, req.ksplit_first64, sp) / kblocks);
    bucket[c] = cost == 0 ? kBuckets - 1
                          : kBuckets - 2 - static_cast<int>(static_cast<int64_t>(cost) * (kBuckets - 2) /
                                                            (max_cost + 1));
  }
  __syncthreads();
  perm::permute_block(bucket, n_chunks, kBuckets, srt, boff, &berr);
  __syncthreads();
  // pref[x][m]: tiles of XCD x's chunks before its m-th (one wave per XCD)
  const int per_x = (n_chunks + 7) / 8;
  if (wave < 8) {
    const int x = wave;
    int running = 0;
    for (int m0 = 0; m0 < per_x; m0 += kWave) {
      const int m = m0 + lane;
      const int q = snake_pos(x, m);
      int nt = 0;
      if (m < per_x && q < n_chunks) {
        const int c = srt[q];
        const int e = c % n_expert, g = (c / n_expert) % n_groups;
        nt = (e_rows[e] + kBM - 1) / kBM * min(gcols, n_col - g * gcols);
      }
      const int incl = wave_inclusive_scan(nt);
      if (m < per_x) pref[x][m] = running + incl - nt;
      running += __shfl(incl, kWave - 1, kWave);
    }
    if (lane == 0) pref[x][per_x] = running;
  }
  __syncthreads();
  bool fits = true;
#pragma unroll
  for (int x = 0; x < 8; ++x) fits = fits && pref[x][per_x] <= bpx;
  // keep[x]: the tiles XCD x runs as dealt.  With steal slots, the last
  // 1/kPoolDiv of its list (its cheapest chunks) goes to the shared pool,
  // from which the blocks past keep[x] on every XCD take one tile each, so
  // the XCDs that run faster take more (the XCDs of one part run the same
  // tiles 3-4% apart).
  __shared__ int keep[8], pbase[9];
  if (tid == 0) {
    int acc = 0;
    for (int x = 0; x < 8; ++x) {
      const int L = pref[x][per_x];
      keep[x] = req.steal > 0 ? L - L / kPoolDiv : L;
      pbase[x] = acc;
      acc += L - keep[x];
    }
    pbase[8] = acc;
  }
  __syncthreads();
  // tile at position p of XCD x's list
  auto entry = [&](int x, int p) {
    int lo = 0, hi = per_x - 1;  // the last m with pref[x][m] <= p
    while (lo < hi) {
      const int mid = (lo + hi + 1) / 2;
      if (pref[x][mid] <= p) lo = mid; else hi = mid - 1;
    }
    const int c = srt[snake_pos(x, lo)];
    const int e = c % n_expert, g = (c / n_expert) % n_groups, sp = c / (n_expert * n_groups);
    const int cig = min(gcols, n_col - g * gcols);
    const int t = p - pref[x][lo];
    const int r = t / cig;
    return make_int4(e, e_off[e] + r * kBM, min(kBM, e_rows[e] - r * kBM), (g * gcols + t % cig) | (sp << 16));
  };
  const int n_blocks = 8 * (bpx + req.steal);
  const int n_ent = 1 + n_blocks + 4 * req.steal;  // header, one per block, pool
  const int per_part = (n_ent + n_parts - 1) / n_parts;
  const int i_end = min(n_ent, (part + 1) * per_part);
  for (int i = part * per_part + tid; i < i_end; i += perm::kThreads) {
    int4 ent = make_int4(fits ? -1 : -2, 0, 0, 0);
    if (i == 0) {
      ent = make_int4(fits ? pbase[8] : 0, 0, 0, 0);  // pool size, claim counter
    } else if (i <= n_blocks) {
      const int b = i - 1, x = b % 8, p = b / 8;
      if (fits && p < keep[x]) ent = entry(x, p);
      else if (fits && req.steal > 0) ent = make_int4(kTakeFromPool, 0, 0, 0);
    } else if (fits) {
      const int j = i - 1 - n_blocks;
      if (j < pbase[8]) {
        int x = 0;
        while (pbase[x + 1] <= j) ++x;
        ent = entry(x, keep[x] + j - pbase[x]);
      }
    }
    table[i] = ent;
  }
}

}  // namespace ttab
}  // namespace
}  // namespace fmoe
