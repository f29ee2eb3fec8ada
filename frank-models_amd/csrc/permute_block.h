// Device code of the single-block token -> expert permutation (a stable
// counting sort of the slot-major flat assignment ids by expert), shared by
// the permutation kernels and the fused decode router.  The algorithm is
// described in permute.hip.
#pragma once
#include "common.h"
#include "launch.h"

namespace fmoe {
namespace {
namespace perm {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / kWave;
constexpr int kMaxExpert = 512;

// Step 3 over ids [f_begin, f_end): base[e] holds the position of the first
// id of expert e at or after f_begin; wcnt[][] must be zero on entry and is
// zero on exit.
__device__ __forceinline__ void scatter_range(const int* __restrict__ ids, int f_begin, int f_end, int n_expert,
                                              int* base, int (*wcnt)[kMaxExpert], int* __restrict__ order) {
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  int nbits = 0;
  while ((1 << nbits) < n_expert) ++nbits;
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (kWave - lane));

  for (int f0 = f_begin; f0 < f_end; f0 += kThreads) {
    const int f = f0 + tid;
    const int e = f < f_end ? ids[f] : -1;
    const bool valid = e >= 0 && e < n_expert;
    uint64_t peers = __ballot(valid);
    for (int b = 0; b < nbits; ++b) {
      const bool bit = valid && ((e >> b) & 1);
      const uint64_t m = __ballot(bit);
      peers &= bit ? m : ~m;
    }
    const int rank = __popcll(peers & lt_mask);
    if (valid && rank == 0) wcnt[wave][e] = __popcll(peers);
    lds_barrier();
    if (valid) {
      int pre = 0;
      for (int w = 0; w < wave; ++w) pre += wcnt[w][e];
      order[base[e] + pre + rank] = f;
    }
    lds_barrier();
    for (int ee = tid; ee < n_expert; ee += kThreads) {
      int tot = 0;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        tot += wcnt[w][ee];
        wcnt[w][ee] = 0;
      }
      base[ee] += tot;
    }
    lds_barrier();
  }
}

// The whole permutation of n <= kPermuteChunk ids by one block of kThreads
// threads: histogram, offsets, stable scatter.  ids must be visible to the
// whole block on entry.  The threads share data through LDS only (the
// order/offsets/err_count stores are not read back), so the barriers do not
// wait for global stores.
__device__ __forceinline__ void permute_block(const int* __restrict__ ids, int n, int n_expert,
                                              int* __restrict__ order, int* __restrict__ offsets,
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
  lds_barrier();

  for (int f = tid; f < n; f += kThreads) {
    const int e = ids[f];
    if (e < 0 || e >= n_expert)
      atomicAdd(&bad, 1);
    else
      atomicAdd(&base[e], 1);
  }
  lds_barrier();

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
  lds_barrier();
  scatter_range(ids, 0, n, n_expert, base, wcnt, order);
}

}  // namespace perm
}  // namespace
}  // namespace fmoe
