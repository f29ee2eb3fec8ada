// Token -> expert permutation: a stable counting sort of the slot-major flat
// assignment ids f = s*n_tokens + t by expert.
//
// The reference has no explicit permutation: mul_mat_id gathers one whole
// expert matrix per assignment in the flat order of
// `tensor.collapse_shape %ids [[0, 1]]` (components/moe/mul_mat_id.mlir:50-61).
// Grouping that order by expert, stably, lets every expert's weights be read
// once per row tile instead of once per assignment.
//
// Small batches (n <= kChunk): one block of 1024 threads (16 waves):
//   1. histogram with LDS atomics (counts are order-independent),
//   2. exclusive scan of the counts -> offsets,
//   3. tiles of 1024 ids in flat order: each wave ranks its lanes among the
//      lanes holding the same expert (ballots over the expert id bits), a
//      per-(wave, expert) count table gives the rank among earlier waves,
//      and a running per-expert base gives the rank among earlier tiles.
//      Position = offset + earlier tiles + earlier waves + rank in wave,
//      which is exactly the stable order.
// Larger batches split the flat order into chunks of kChunk ids, one block
// each, in two launches:
//   a. per-chunk expert histograms (and a count of invalid ids),
//   b. each chunk's block sums the histograms into the expert offsets and
//      its own per-expert base (offset + the counts of earlier chunks), then
//      runs step 3 over its chunk.  Chunk 0 writes the offsets.
// A caller may also ask for the tile schedules of 256-tile GEMMs over the
// resulting offsets (tile_table.h): kTableParts extra blocks per schedule in
// the same launch count the rows per expert themselves and build it while the
// scatter runs, each writing a part of its entries.
#include "common.h"
#include "launch.h"
#include "permute_block.h"
#include "tile_table.h"

namespace fmoe {
namespace {

using perm::kThreads;
using perm::kWaves;
using perm::kMaxExpert;
using perm::scatter_range;
constexpr int kHistThreads = 256;

struct TileTables {
  TileTableReq r[kPermuteMaxTables];
};
// Blocks per schedule: each sorts the chunks and writes a part of the entries.
constexpr int kTableParts = 4;

// Blocks 1.. of the launch (TABLES): the tile schedule over the counts of
// the valid ids per expert (the offsets block 0 writes).  Without TABLES the
// kernel holds none of the schedule's LDS.
template <bool TABLES>
__global__ __launch_bounds__(kThreads) void permute_kernel(const int* __restrict__ ids, int n,
                                                           int n_expert, int* __restrict__ order,
                                                           int* __restrict__ offsets,
                                                           int* __restrict__ err_count, TileTables tt) {
  if (TABLES && blockIdx.x > 0) {
    __shared__ int rows[ttab::kMaxExperts];
    for (int e = threadIdx.x; e < n_expert; e += kThreads) rows[e] = 0;
    __syncthreads();
    for (int f = threadIdx.x; f < n; f += kThreads) {
      const int e = ids[f];
      if (e >= 0 && e < n_expert) atomicAdd(&rows[e], 1);
    }
    __syncthreads();
    const int i = static_cast<int>(blockIdx.x) - 1;
    const TileTableReq r = tt.r[i / kTableParts];
    ttab::build(rows, n_expert, r, reinterpret_cast<int4*>(r.table), i % kTableParts, kTableParts);
    return;
  }
  perm::permute_block(ids, n, n_expert, order, offsets, err_count);
}

// counts[c * (n_expert + 1) + e]: ids of expert e in chunk c; entry n_expert
// counts the invalid ids.
__global__ __launch_bounds__(kHistThreads) void chunk_hist_kernel(const int* __restrict__ ids, int n,
                                                                  int n_expert, int* __restrict__ counts) {
  __shared__ int h[kMaxExpert + 1];
  for (int e = threadIdx.x; e <= n_expert; e += kHistThreads) h[e] = 0;
  __syncthreads();
  const int f0 = blockIdx.x * kPermuteChunk;
  const int f1 = min(n, f0 + kPermuteChunk);
  // All of a thread's ids are loaded before the first count (one memory
  // round trip per chunk, not one per id).
  constexpr int kPer = kPermuteChunk / kHistThreads;
  int ev[kPer];
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    const int f = f0 + q * kHistThreads + static_cast<int>(threadIdx.x);
    ev[q] = f < f1 ? ids[f] : 0;
  }
#pragma unroll
  for (int q = 0; q < kPer; ++q)
    if (f0 + q * kHistThreads + static_cast<int>(threadIdx.x) < f1)
      atomicAdd(&h[(ev[q] >= 0 && ev[q] < n_expert) ? ev[q] : n_expert], 1);
  __syncthreads();
  for (int e = threadIdx.x; e <= n_expert; e += kHistThreads)
    counts[static_cast<int64_t>(blockIdx.x) * (n_expert + 1) + e] = h[e];
}

template <bool TABLES>
__global__ __launch_bounds__(kThreads) void chunk_scatter_kernel(const int* __restrict__ ids, int n,
                                                                 int n_expert, const int* __restrict__ counts,
                                                                 int n_chunks, int* __restrict__ order,
                                                                 int* __restrict__ offsets,
                                                                 int* __restrict__ err_count, TileTables tt) {
  __shared__ int base[kMaxExpert];
  __shared__ int total[kMaxExpert];
  __shared__ int wcnt[kWaves][kMaxExpert];
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int chunk = blockIdx.x;
  const int stride = n_expert + 1;

  if (TABLES && chunk >= n_chunks) {
    // a tile schedule over the per-expert totals of the histograms
    for (int e = tid; e < n_expert; e += kThreads) {
      int tot = 0;
      for (int c0 = 0; c0 < n_chunks; c0 += 8) {
        int v[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) v[q] = c0 + q < n_chunks ? counts[(c0 + q) * stride + e] : 0;
#pragma unroll
        for (int q = 0; q < 8; ++q) tot += v[q];
      }
      total[e] = tot;
    }
    __syncthreads();
    const int i = chunk - n_chunks;
    const TileTableReq r = tt.r[i / kTableParts];
    ttab::build(total, n_expert, r, reinterpret_cast<int4*>(r.table), i % kTableParts, kTableParts);
    return;
  }
  for (int e = tid; e < n_expert; e += kThreads) {
    // eight chunks' counts in flight at a time
    int tot = 0, pre = 0;
    for (int c0 = 0; c0 < n_chunks; c0 += 8) {
      int v[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) v[q] = c0 + q < n_chunks ? counts[(c0 + q) * stride + e] : 0;
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        tot += v[q];
        pre += c0 + q < chunk ? v[q] : 0;
      }
    }
    total[e] = tot;
    base[e] = pre;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) wcnt[w][e] = 0;
  }
  __syncthreads();
  if (wave == 0) {
    int running = 0;
    for (int c = 0; c < n_expert; c += kWave) {
      const int e = c + lane;
      const int v = e < n_expert ? total[e] : 0;
      const int incl = wave_inclusive_scan(v);
      if (e < n_expert) {
        const int off = running + incl - v;
        base[e] += off;
        if (chunk == 0) offsets[e] = off;
      }
      running += __shfl(incl, kWave - 1, kWave);
    }
    if (chunk == 0) {
      int bad = 0;
      for (int c = lane; c < n_chunks; c += kWave) bad += counts[c * stride + n_expert];
      bad = wave_sum(bad);
      if (lane == 0) {
        offsets[n_expert] = running;
        err_count[0] = bad;
      }
    }
  }
  __syncthreads();
  const int f0 = chunk * kPermuteChunk;
  scatter_range(ids, f0, min(n, f0 + kPermuteChunk), n_expert, base, wcnt, order);
}

}  // namespace

size_t permute_scratch_bytes(int n_assign, int n_expert) {
  if (n_assign <= kPermuteChunk) return 0;
  const int64_t chunks = (static_cast<int64_t>(n_assign) + kPermuteChunk - 1) / kPermuteChunk;
  return static_cast<size_t>(chunks * (n_expert + 1)) * sizeof(int);
}

hipError_t launch_permute(const int* ids, int n_assign, int n_expert, int* order, int* offsets,
                          int* err_count, int* scratch, hipStream_t stream, const TileTableReq* tables,
                          int n_tables) {
  if (n_expert > kMaxExpert || n_expert <= 0) return hipErrorInvalidValue;
  if (n_tables < 0 || n_tables > kPermuteMaxTables || (n_tables > 0 && !tables)) return hipErrorInvalidValue;
  TileTables tt;
  for (int i = 0; i < n_tables; ++i) {
    const TileTableReq& r = tables[i];
    const int64_t chunks = ttab::n_chunks(r.n_col, r.ksplit, n_expert);
    if (!r.table || r.n_col <= 0 || r.n_col >= (1 << 16) || r.ksplit <= 0 || r.bpx <= 0 ||
        n_expert > ttab::kMaxExperts || chunks > ttab::kChunks ||
        r.bpx != ttab::blocks_per_xcd(max_row_tiles(n_assign, n_expert, ttab::kBM), r.n_col, r.ksplit) ||
        (r.steal != 0 && r.steal != ttab::steal_per_xcd(r.bpx)))
      return hipErrorInvalidValue;
    tt.r[i] = r;
  }
  if (n_assign <= kPermuteChunk) {
    if (n_tables > 0)
      hipLaunchKernelGGL(permute_kernel<true>, dim3(1 + kTableParts * n_tables), dim3(kThreads), 0, stream, ids, n_assign,
                         n_expert, order, offsets, err_count, tt);
    else
      hipLaunchKernelGGL(permute_kernel<false>, dim3(1), dim3(kThreads), 0, stream, ids, n_assign, n_expert, order,
                         offsets, err_count, tt);
    return hipGetLastError();
  }
  if (!scratch) return hipErrorInvalidValue;
  const int chunks = (n_assign + kPermuteChunk - 1) / kPermuteChunk;
  hipLaunchKernelGGL(chunk_hist_kernel, dim3(chunks), dim3(kHistThreads), 0, stream, ids, n_assign, n_expert,
                     scratch);
  if (n_tables > 0)
    hipLaunchKernelGGL(chunk_scatter_kernel<true>, dim3(chunks + kTableParts * n_tables), dim3(kThreads), 0, stream, ids,
                       n_assign, n_expert, scratch, chunks, order, offsets, err_count, tt);
  else
    hipLaunchKernelGGL(chunk_scatter_kernel<false>, dim3(chunks), dim3(kThreads), 0, stream, ids, n_assign,
                       n_expert, scratch, chunks, order, offsets, err_count, tt);
  return hipGetLastError();
}

}  // namespace fmoe
