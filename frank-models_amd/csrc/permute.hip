// Token -> expert permutation: a stable counting sort of the slot-major flat
// assignment ids f = s*n_tokens + t by expert.
//
// The reference has no explicit permutation: mul_mat_id gathers one whole
// expert matrix per assignment in the flat order of
// `tensor.collapse_shape %ids [[0, 1]]` (components/moe/mul_mat_id.mlir:50-61).
// Grouping that order by expert, stably, lets every expert's weights be read
// once per row tile instead of once per assignment.
//
// One block of 1024 threads (16 waves):
//   1. histogram with LDS atomics (counts are order-independent),
//   2. exclusive scan of the counts -> offsets,
//   3. tiles of 1024 ids in flat order: each wave ranks its lanes among the
//      lanes holding the same expert (ballots over the expert id bits), a
//      per-(wave, expert) count table gives the rank among earlier waves,
//      and a running per-expert base gives the rank among earlier tiles.
//      Position = offset + earlier tiles + earlier waves + rank in wave,
//      which is exactly the stable order.
#include "common.h"
#include "launch.h"

namespace fmoe {
namespace {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / kWave;
constexpr int kMaxExpert = 512;

__global__ __launch_bounds__(kThreads) void permute_kernel(const int* __restrict__ ids, int n,
                                                           int n_expert, int* __restrict__ order,
                                                           int* __restrict__ offsets,
                                                           int* __restrict__ err_count) {
  __shared__ int base[kMaxExpert];
  __shared__ int wcnt[kWaves][kMaxExpert];
  __shared__ int bad;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;

  for (int e = tid; e < n_expert; e += kThreads) {
    base[e] = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) wcnt[w][e] = 0;
  }
  if (tid == 0) bad = 0;
  __syncthreads();

  for (int f = tid; f < n; f += kThreads) {
    const int e = ids[f];
    if (e < 0 || e >= n_expert)
      atomicAdd(&bad, 1);
    else
      atomicAdd(&base[e], 1);
  }
  __syncthreads();

  if (wave == 0) {
    int running = 0;
    for (int c = 0; c < n_expert; c += kWave) {
      const int e = c + lane;
      const int v = e < n_expert ? base[e] : 0;
      const int incl = wave_inclusive_scan(v);
      if (e < n_expert) {
        offsets[e] = running + incl - v;
        base[e] = running + incl - v;
      }
      running += __shfl(incl, kWave - 1, kWave);
    }
    if (lane == 0) {
      offsets[n_expert] = running;
      err_count[0] = bad;
    }
  }
  __syncthreads();

  int nbits = 0;
  while ((1 << nbits) < n_expert) ++nbits;
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (kWave - lane));

  for (int f0 = 0; f0 < n; f0 += kThreads) {
    const int f = f0 + tid;
    const int e = f < n ? ids[f] : -1;
    const bool valid = e >= 0 && e < n_expert;
    uint64_t peers = __ballot(valid);
    for (int b = 0; b < nbits; ++b) {
      const bool bit = valid && ((e >> b) & 1);
      const uint64_t m = __ballot(bit);
      peers &= bit ? m : ~m;
    }
    const int rank = __popcll(peers & lt_mask);
    if (valid && rank == 0) wcnt[wave][e] = __popcll(peers);
    __syncthreads();
    if (valid) {
      int pre = 0;
      for (int w = 0; w < wave; ++w) pre += wcnt[w][e];
      order[base[e] + pre + rank] = f;
    }
    __syncthreads();
    for (int ee = tid; ee < n_expert; ee += kThreads) {
      int tot = 0;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        tot += wcnt[w][ee];
        wcnt[w][ee] = 0;
      }
      base[ee] += tot;
    }
    __syncthreads();
  }
}

}  // namespace

hipError_t launch_permute(const int* ids, int n_assign, int n_expert, int* order, int* offsets,
                          int* err_count, hipStream_t stream) {
  if (n_expert > kMaxExpert || n_expert <= 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(permute_kernel, dim3(1), dim3(kThreads), 0, stream, ids, n_assign, n_expert,
                     order, offsets, err_count);
  return hipGetLastError();
}

}  // namespace fmoe
