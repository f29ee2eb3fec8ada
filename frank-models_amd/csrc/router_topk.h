// Softmax + top-k of decode-sized router batches, shared by the router's
// kernels (router.hip) and the decode gate/up GEMM that recomputes the
// routing of up to 4 tokens in its blocks (gemm_mfma.hip): the same code, so
// the same ids and weights bit for bit.
#pragma once
#include "common.h"

namespace fmoe {
namespace {

// Row rotation within 16-lane DPP rows (row_ror:N), for reductions over a
// row without going through LDS.
template <int N>
__device__ __forceinline__ int ror16(int v) {
  return __builtin_amdgcn_update_dpp(0, v, 0x120 + N, 0xF, 0xF, false);
}
template <int N>
__device__ __forceinline__ float ror16(float v) {
  return __builtin_bit_cast(float, ror16<N>(__builtin_bit_cast(int, v)));
}

// Softmax + top-k (k <= 16, n_expert <= 16 NV <= 256) of four tokens at
// once, one per 16-lane row: row g takes token t0 + g, whose logits are
// lg[g * ld + e]; lane j of the row holds experts j, j + 16, ... (NV each:
// each is a few VALU instructions per slot, at 4 cycles each for a wave).  Reductions over the row
// use DPP rotations.  The selection runs on the fp32 probabilities, as the
// reference's top-k does: logits a few ulps apart can round to one
// probability, and that tie goes to the lower expert index.  Larger first,
// lower expert index on ties.  Each token's denominator is the one its
// lane 0 summed.  ids / weights null: nothing is stored in global memory
// (ids_copy, when given, still receives the flat ids).
template <int NV>
__device__ void softmax_topk4(const float* lg, int ld, int t0, int n_tokens, int n_expert, int k, bool normalize,
                              int* ids, float* weights, int* ids_copy = nullptr) {
  const int lane = threadIdx.x & (kWave - 1);
  const int g = lane >> 4, j = lane & 15;
  const int t = t0 + g;
  const float* row = lg + g * ld;
  float v[NV];
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int e = j + 16 * i;
    v[i] = e < n_expert ? row[e] : -INFINITY;
    m = fmaxf(m, v[i]);
  }
  m = fmaxf(m, ror16<8>(m));
  m = fmaxf(m, ror16<4>(m));
  m = fmaxf(m, ror16<2>(m));
  m = fmaxf(m, ror16<1>(m));
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    v[i] = j + 16 * i < n_expert ? expf(v[i] - m) : 0.f;
    s += v[i];
  }
  s += ror16<8>(s);
  s += ror16<4>(s);
  s += ror16<2>(s);
  s += ror16<1>(s);
  s = __shfl(s, lane & ~15, kWave);
  // Probabilities; -1 marks an expert that cannot be selected (absent, or
  // already taken).
#pragma unroll
  for (int i = 0; i < NV; ++i) v[i] = j + 16 * i < n_expert ? v[i] / s : -1.f;
  float my_w = 0.f;
  int my_id = 0;
  for (int slot = 0; slot < k; ++slot) {
    float bv = -1.f;
    int bi = 0x7FFFFFFF;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      if (v[i] > bv) {  // i ascending: ties keep the lower expert
        bv = v[i];
        bi = j + 16 * i;
      }
    }
#define FMOE_TOPK_STEP(N)                                   \
    {                                                       \
      const float ov = ror16<N>(bv);                        \
      const int oi = ror16<N>(bi);                          \
      if (ov > bv || (ov == bv && oi < bi)) {               \
        bv = ov;                                            \
        bi = oi;                                            \
      }                                                     \
    }
    FMOE_TOPK_STEP(8)
    FMOE_TOPK_STEP(4)
    FMOE_TOPK_STEP(2)
    FMOE_TOPK_STEP(1)
#undef FMOE_TOPK_STEP
#pragma unroll
    for (int i = 0; i < NV; ++i)
      if (j + 16 * i == bi) v[i] = -1.f;
    if (j == slot) {
      my_w = bv;
      my_id = bi;
    }
  }
  if (normalize) {
    // Sum in slot order (the linalg reduction of moe_ffn_block.mlir:97-107).
    float wsum = 0.f;
    for (int slot = 0; slot < k; ++slot) wsum += __shfl(my_w, (lane & ~15) + slot, kWave);
    my_w = my_w / wsum;
  }
  if (j < k && t < n_tokens) {
    if (ids) {
      ids[static_cast<int64_t>(j) * n_tokens + t] = my_id;
      weights[static_cast<int64_t>(j) * n_tokens + t] = my_w;
    }
    if (ids_copy) ids_copy[j * n_tokens + t] = my_id;
  }
}

// The calling wave's share of the decode top-k of up to 4 tokens: lane
// (g, j) sums the split partial logits (part[s][t][e], n_split splits of
// n_tokens x n_expert) of token g's experts j, j + 16, ... in split order
// into lg[g * (16 NV + 1) + e], then softmax_topk4 selects (ids / weights
// stored unless null; the k * n_tokens flat ids, slot-major, into idl).
// softmax_topk4 reads back only the lane's own lg entries; other lanes read
// idl only after a barrier.
template <int NV>
__device__ __forceinline__ void wave_topk4_splits(const float* __restrict__ part, int n_split, int n_tokens,
                                                  int n_expert, int k, bool normalize, float* lg, int* ids,
                                                  float* weights, int* idl) {
  constexpr int ld = 16 * NV + 1;
  const int lane = threadIdx.x & (kWave - 1);
  const int g = lane >> 4, j = lane & 15;
  const int t = min(g, n_tokens - 1);
  const int64_t plane = static_cast<int64_t>(n_tokens) * n_expert;
  const float* src = part + static_cast<int64_t>(t) * n_expert;
  float v[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) v[i] = 0.f;
  for (int s0 = 0; s0 < n_split; s0 += 4) {
    float pv[4][NV];
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int e = j + 16 * i;
        pv[q][i] = s0 + q < n_split && e < n_expert ? src[(s0 + q) * plane + e] : 0.f;
      }
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int i = 0; i < NV; ++i)
        if (s0 + q < n_split) v[i] += pv[q][i];
  }
#pragma unroll
  for (int i = 0; i < NV; ++i) lg[g * ld + j + 16 * i] = v[i];
  softmax_topk4<NV>(lg, ld, 0, n_tokens, n_expert, k, normalize, ids, weights, idl);
}

// The stable grouping of the n <= 64 flat ids in idl by the calling wave:
// lane f's id goes to position (ids of lower experts) + (its expert's ids
// before f), the stable counting sort's order; offsets[e] = the ids below e.
__device__ __forceinline__ void wave_permute(const int* idl, int n, int n_expert, int* order, int* offsets) {
  const int lane = threadIdx.x & (kWave - 1);
  const int e = lane < n ? idl[lane] : 0x7FFFFFFF;
  int pos = 0;
  for (int f = 0; f < n; ++f) {
    const int ef = idl[f];
    pos += (ef < e || (ef == e && f < lane)) ? 1 : 0;
  }
  if (lane < n) order[pos] = lane;
  for (int ee = lane; ee <= n_expert; ee += kWave) {
    int below = 0;
    for (int f = 0; f < n; ++f) below += idl[f] < ee ? 1 : 0;
    offsets[ee] = below;
  }
}

}  // namespace
}  // namespace fmoe
