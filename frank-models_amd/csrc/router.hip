// Router: logits = W_router @ x^T (fp32 accumulate), softmax over experts in
// fp32, top-k with exact ties to the lower expert index, optional slot-sum
// renormalisation.
//
// Reference: components/moe/moe_ffn_block.mlir:50-128 (transpose + matmul,
// linalg.softmax dimension(0), iree_linalg_ext.topk with `ogt`, scf.if
// renormalisation); oracles/moe.py:86-105.
//
// Kernels by shape (launch_router, launch_router_prefill, launch_router_decode):
//   * router_mfma_bf16_kernel: bf16, up to 128 experts (the prefill choice up
//     to 32), one block per kTok = 16 tokens, 16 waves splitting the hidden
//     axis;
//   * router_tile_bf16_kernel: bf16, 33-128 experts, token rows and router
//     rows staged as whole 256-byte row segments through an LDS ring; at
//     prefill sizes split over hidden-axis ranges, with router_part_topk_kernel
//     summing the ranges' partial logits;
//   * router_split_logits_kernel + router_topk_permute_kernel: decode-sized
//     batches (logits split over many blocks, one block for top-k and the
//     permutation: one wave up to 4 tokens (router_topk_permute_wave_kernel);
//     above 64 experts and 32 tokens router_part_topk_kernel over blocks,
//     then the permutation's own launch);
//   * router_simt_kernel: fp32 and the shapes above that none takes.
// Softmax + top-k run four tokens per wave (16 lanes each, DPP row
// reductions) for k <= 16, or one token per wave over its 64 lanes.
#include "common.h"
#include "launch.h"
#include "permute_block.h"
#include "router_topk.h"

namespace fmoe {
namespace {

constexpr int kTok = 16;
constexpr int kThreads = 256;
constexpr int kMaxExpert = 256;    // lanes hold up to 4 experts each
constexpr int kMfmaMaxExpert = 128;

// Softmax + top-k + optional renormalisation of token t, whose logits are
// lg[0 .. n_expert), by one wave with the expert axis spread over its lanes.
__device__ void softmax_topk_token(const float* lg, int t, int n_tokens, int n_expert, int k, bool normalize,
                                   int* ids, float* weights) {
  const int lane = threadIdx.x & (kWave - 1);
  float p[4];
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = lane + i * kWave;
    p[i] = e < n_expert ? lg[e] : -INFINITY;
    m = fmaxf(m, p[i]);
  }
  m = wave_max(m);
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = lane + i * kWave;
    p[i] = e < n_expert ? expf(p[i] - m) : 0.f;
    s += p[i];
  }
  s = wave_sum(s);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = lane + i * kWave;
    p[i] = e < n_expert ? p[i] / s : -1.f;  // -1 marks "not selectable"
  }
  // Lane `slot` keeps the slot's expert and probability.
  float my_w = 0.f;
  int my_id = 0;
  for (int slot = 0; slot < k; ++slot) {
    // lane-local best: larger value, then lower index (i ascending -> e ascending)
    float bv = -1.f;
    int bi = 0x7FFFFFFF;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (p[i] > bv) {
        bv = p[i];
        bi = lane + i * kWave;
      }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float ov = __shfl_xor(bv, o, kWave);
      const int oi = __shfl_xor(bi, o, kWave);
      if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (lane + i * kWave == bi) p[i] = -1.f;
    if (lane == slot) {
      my_w = bv;
      my_id = bi;
    }
  }
  if (normalize) {
    // Sum in slot order (the linalg reduction of moe_ffn_block.mlir:97-107).
    float wsum = 0.f;
    for (int slot = 0; slot < k; ++slot) wsum += __shfl(my_w, slot, kWave);
    my_w = my_w / wsum;
  }
  if (lane < k) {
    ids[static_cast<int64_t>(lane) * n_tokens + t] = my_id;
    weights[static_cast<int64_t>(lane) * n_tokens + t] = my_w;
  }
}

// Softmax + top-k of the kTok tokens from tok0 whose logits are in
// lds_logits[kTok][ld]; the block's n_waves waves take tokens wave,
// wave + n_waves, ...
// NV bounds the experts per lane of the four-token path (n_expert <= 16 NV).
template <int NV>
__device__ void softmax_topk(const float* lds_logits, int ld, int tok0, int n_tokens, int n_expert, int k,
                             bool normalize, int* ids, float* weights, int n_waves) {
  const int wave = threadIdx.x / kWave;
  if (k <= 16) {
    // four tokens per wave, 16 lanes each
    for (int q = wave; q < kTok / 4; q += n_waves) {
      if (tok0 + 4 * q >= n_tokens) break;
      softmax_topk4<NV>(lds_logits + 4 * q * ld, ld, tok0 + 4 * q, n_tokens, n_expert, k, normalize, ids, weights);
    }
    return;
  }
  for (int tt = wave; tt < kTok; tt += n_waves) {
    const int t = tok0 + tt;
    if (t >= n_tokens) break;
    softmax_topk_token(lds_logits + tt * ld, t, n_tokens, n_expert, k, normalize, ids, weights);
  }
}

template <typename T>
__device__ __forceinline__ float ld_f32(const T* p, int64_t i);
template <>
__device__ __forceinline__ float ld_f32<float>(const float* p, int64_t i) { return p[i]; }
template <>
__device__ __forceinline__ float ld_f32<bf16_t>(const bf16_t* p, int64_t i) { return bf16_to_f32(p[i]); }

// SIMT logits: any n_embd, any dtype.  Thread pairs (token, expert) walk
// the hidden axis in order.
template <typename T>
__global__ __launch_bounds__(kThreads) void router_simt_kernel(
    const T* __restrict__ x, const T* __restrict__ wr, int n_tokens, int n_embd,
    int n_expert, int k, int normalize, int* __restrict__ ids, float* __restrict__ weights) {
  extern __shared__ float lds[];
  const int ld = n_expert + 1;
  const int tok0 = blockIdx.x * kTok;
  for (int idx = threadIdx.x; idx < kTok * n_expert; idx += kThreads) {
    const int tt = idx / n_expert;
    const int e = idx - tt * n_expert;
    const int t = tok0 + tt;
    float acc = 0.f;
    if (t < n_tokens) {
      const T* xr = x + static_cast<int64_t>(t) * n_embd;
      const T* wrr = wr + static_cast<int64_t>(e) * n_embd;
      for (int h = 0; h < n_embd; ++h) acc = fmaf(ld_f32(wrr, h), ld_f32(xr, h), acc);
    }
    lds[tt * ld + e] = acc;
  }
  __syncthreads();
  softmax_topk<kMaxExpert / 16>(lds, ld, tok0, n_tokens, n_expert, k, normalize != 0, ids, weights, kThreads / kWave);
}

// MFMA logits for bf16 inputs, n_embd % 32 == 0, n_expert <= 128.
// v_mfma_f32_16x16x32_bf16 with A = 16 tokens x 32 hidden, B = 32 hidden x
// 16 experts.  The 16 waves of the block split the hidden axis (wave w takes
// 32-wide chunks w, w+16, ...), so a decode-sized batch still spreads its
// dot products over a whole block; partial logits are summed in wave order.
constexpr int kMfmaWaves = 16;
constexpr int kMfmaThreads = kMfmaWaves * kWave;

// NCH: 16-expert chunks the kernel is built for (1, 2, or 8 for up to 128
// experts, then only the first ceil(E / 16) are used).  Each wave loads
// kRouterDepth trips (32-wide hidden chunks kMfmaWaves * 32 apart) before
// its first MFMA: at 4096 hidden columns and up to 32 experts that is all
// of its 8 trips in one round trip.  With more experts the operands of one
// trip already fill the register budget (more would spill), so it loads one
// trip at a time; that case only serves inputs the tile router cannot take.
template <int NCH>
constexpr int router_depth() {
  return NCH <= 2 ? 8 : 1;
}

template <int NCH>
__global__ __launch_bounds__(kMfmaThreads) void router_mfma_bf16_kernel(
    const bf16_t* __restrict__ x, const bf16_t* __restrict__ wr, int n_tokens, int n_embd,
    int n_expert, int k, int normalize, int* __restrict__ ids, float* __restrict__ weights) {
  extern __shared__ float part[];  // [kMfmaWaves][kTok][ld], then logits [kTok][ld]
  const int ld = ((n_expert + 15) / 16) * 16 + 1;
  float* logits = part + kMfmaWaves * kTok * ld;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int tok0 = blockIdx.x * kTok;
  const int n_chunks = (n_expert + 15) / 16;

  f32x4_t acc[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) acc[c] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int row = lane & 15;         // token (A) / expert-in-chunk (B)
  const int kofs = (lane >> 4) * 8;  // 8 consecutive hidden elements
  const int t = tok0 + row;
  const bool t_ok = t < n_tokens;
  const bf16_t* xrow = x + static_cast<int64_t>(t_ok ? t : 0) * n_embd + kofs;
  // Operands of one 32-wide chunk of the hidden axis: the token fragment and
  // one router fragment per 16 experts; chunks past the hidden axis load
  // zeros (their MFMAs add exact zeros).  The trips accumulate in hidden
  // order, as one trip at a time would.
  const u32x4_t zero{0u, 0u, 0u, 0u};
  constexpr int kStep = kMfmaWaves * 32;
  constexpr int D = router_depth<NCH>();
  for (int h0 = wave * 32; h0 < n_embd; h0 += D * kStep) {
    u32x4_t av[D], bv[D][NCH];
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int h = h0 + d * kStep;
      const bool in = h < n_embd;
      av[d] = (t_ok && in) ? *reinterpret_cast<const u32x4_t*>(xrow + h) : zero;
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        const int e = c * 16 + row;
        bv[d][c] = (c < n_chunks && e < n_expert && in)
                       ? *reinterpret_cast<const u32x4_t*>(wr + static_cast<int64_t>(e) * n_embd + h + kofs)
                       : zero;
      }
    }
#pragma unroll
    for (int d = 0; d < D; ++d)
#pragma unroll
      for (int c = 0; c < NCH; ++c)
        if (c < n_chunks)
          acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, av[d]),
                                                           __builtin_bit_cast(bf16x8_t, bv[d][c]), acc[c], 0, 0, 0);
  }
  // D[token][expert]: lane holds expert (lane & 15), tokens 4*(lane>>4)+i.
  float* mine = part + wave * kTok * ld;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    if (c < n_chunks) {
#pragma unroll
      for (int i = 0; i < 4; ++i) mine[((lane >> 4) * 4 + i) * ld + c * 16 + (lane & 15)] = acc[c][i];
    }
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < kTok * n_expert; idx += kMfmaThreads) {
    const int tt = idx / n_expert;
    const int e = idx - tt * n_expert;
    float v = part[tt * ld + e];
    for (int w = 1; w < kMfmaWaves; ++w) v += part[(w * kTok + tt) * ld + e];
    logits[tt * ld + e] = v;
  }
  __syncthreads();
  softmax_topk<kMfmaMaxExpert / 16>(logits, ld, tok0, n_tokens, n_expert, k, normalize != 0, ids, weights,
                                    kMfmaWaves);
}

// ---- Prefill logits for 32 < n_expert <= 128 (bf16, n_embd % 128 == 0,
// k <= 16): one 512-thread block per TT 16-token tiles (32 or 64 tokens) and
// per range of the hidden axis.  The block stages its token rows and the
// router rows through an LDS ring by global_load_lds, in stages of 128
// hidden columns (a 3-deep ring, two stages in flight): TT * 16 token rows
// then NCP * 16 router rows, 256 bytes each.  Each load instruction moves
// four whole 256-byte row segments (16 lanes per row), which a CU streams
// about 1.6x faster than 16-row x 64-byte MFMA-shaped gathers.  The row's
// 16-byte chunks sit at chunk ^ (row & 15), so the MFMA operand reads
// (lane l: row l % 16, inputs 8 (l / 16) .. +8 of a 32-input step) hit 16
// distinct bank groups.  Wave w owns expert chunk w % NCP and TT * NCP / 8
// token tiles, so no partial logits cross waves.
//   part == nullptr (one range over the whole hidden axis): softmax + top-k
//   in the block.  Otherwise range blockIdx.y writes its partial logits to
//   part[(blockIdx.y * T + t) * E + e] for router_part_topk_kernel.
constexpr int kTileCols = 128;
constexpr int kTileRing = 3;

template <int NCP, int TT>
constexpr int tile_stage_bytes() {
  return (TT + NCP) * 16 * 256;
}

// One wave's loads of stage st: its 1 KiB blocks wave, wave + 8, ... (four
// rows each) into the stage's ring buffer.
template <int NPW>
__device__ __forceinline__ void tile_issue(const bf16_t* const (&src)[NPW], unsigned char* smem, int st, int buf,
                                           int wave, int stage_bytes) {
  unsigned char* dst = smem + buf * stage_bytes;
#pragma unroll
  for (int j = 0; j < NPW; ++j)
    __builtin_amdgcn_global_load_lds(src[j] + st * kTileCols, dst + (wave + 8 * j) * 1024, 16, 0, 0);
}

template <int NCP, int TT>
__global__ __launch_bounds__(512) void router_tile_bf16_kernel(const bf16_t* __restrict__ x,
                                                               const bf16_t* __restrict__ wr, int n_tokens,
                                                               int n_embd, int n_expert, int k, int normalize,
                                                               int stages_per_range, int* __restrict__ ids,
                                                               float* __restrict__ weights, float* __restrict__ part) {
  static_assert(NCP == 4 || NCP == 8, "8 waves over NCP expert chunks");
  static_assert((TT == 2 || TT == 4) && (TT * NCP) % 8 == 0, "whole token tiles per wave");
  extern __shared__ __align__(16) unsigned char smem[];
  constexpr int kTok = TT * 16;
  constexpr int kTTW = TT * NCP / 8;          // token tiles per wave
  constexpr int kStage = tile_stage_bytes<NCP, TT>();
  constexpr int kBlocks = kStage / 1024;      // 1 KiB blocks (four rows) per stage
  constexpr int kPerWave = kBlocks / 8;       // loads per wave per stage
  static_assert(kBlocks % 8 == 0, "stage blocks split evenly over 8 waves");
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int tok0 = blockIdx.x * kTok;
  const int chunk = wave % NCP;
  const int tt0 = (wave / NCP) * kTTW;
  const int r16 = lane & 15;

  // Block b holds stage rows 4 b .. 4 b + 3 (token rows first, then router
  // rows); lane l loads row 4 b + l / 16, physical chunk l % 16, i.e. the
  // logical chunk (l % 16) ^ (row & 15).  Rows past the batch or the expert
  // count read the last valid row (their logits are never used).
  const bf16_t* src[kPerWave];
#pragma unroll
  for (int j = 0; j < kPerWave; ++j) {
    const int r = 4 * (wave + 8 * j) + (lane >> 4);
    const int c = r16 ^ (r & 15);
    if (r < kTok) {
      const int t = min(tok0 + r, n_tokens - 1);
      src[j] = x + static_cast<int64_t>(t) * n_embd + c * 8;
    } else {
      const int e = min(r - kTok, n_expert - 1);
      src[j] = wr + static_cast<int64_t>(e) * n_embd + c * 8;
    }
  }

  f32x4_t acc[kTTW];
#pragma unroll
  for (int q = 0; q < kTTW; ++q) acc[q] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const int n_st_all = n_embd / kTileCols;
  const int st0 = blockIdx.y * stages_per_range;
  const int n_st = min(stages_per_range, n_st_all - st0);
  tile_issue<kPerWave>(src, smem, st0, 0, wave, kStage);
  if (n_st > 1) tile_issue<kPerWave>(src, smem, st0 + 1, 1, wave, kStage);
  // Operand reads: row (lane & 15) of a 16-row tile, logical chunk
  // 4 s + lane / 16 of step s, stored at that chunk ^ (lane & 15).
  const int rd_lane = r16 * 256;
  for (int st = 0; st < n_st; ++st) {
    // Stage st + 2 refills the buffer of stage st - 1, released by the
    // barrier that ended the last iteration.
    if (st + 2 < n_st) {
      tile_issue<kPerWave>(src, smem, st0 + st + 2, (st + 2) % kTileRing, wave, kStage);
      __builtin_amdgcn_s_waitcnt(wait_vm(2 * kPerWave, false));
    } else if (st + 1 < n_st) {
      __builtin_amdgcn_s_waitcnt(wait_vm(kPerWave, false));
    } else {
      __builtin_amdgcn_s_waitcnt(wait_vm(0, false));
    }
    asm volatile("s_barrier" ::: "memory");
    const unsigned char* cur = smem + (st % kTileRing) * kStage;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int off = rd_lane + (((4 * s + (lane >> 4)) ^ r16) << 4);
      const u32x4_t b = *reinterpret_cast<const u32x4_t*>(cur + (kTok + chunk * 16) * 256 + off);
#pragma unroll
      for (int q = 0; q < kTTW; ++q) {
        const u32x4_t a = *reinterpret_cast<const u32x4_t*>(cur + (tt0 + q) * 16 * 256 + off);
        acc[q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                         __builtin_bit_cast(bf16x8_t, b), acc[q], 0, 0, 0);
      }
    }
    // This buffer's reads are done before it is refilled (no wait on the
    // stages still in flight).
    __builtin_amdgcn_s_waitcnt(wait_vm(63, true));
    asm volatile("s_barrier" ::: "memory");
  }
  __builtin_amdgcn_s_waitcnt(wait_vm(0, true));
  // D[token][expert]: the lane holds expert r16 of its chunk, tokens
  // 4 (lane / 16) + i of each of its tiles.
  const int e = chunk * 16 + r16;
  if (part) {
    float* dst = part + static_cast<int64_t>(blockIdx.y) * n_tokens * n_expert;
#pragma unroll
    for (int q = 0; q < kTTW; ++q)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = tok0 + (tt0 + q) * 16 + 4 * (lane >> 4) + i;
        if (t < n_tokens && e < n_expert) dst[static_cast<int64_t>(t) * n_expert + e] = acc[q][i];
      }
    return;
  }
  // The logits overwrite the ring.
  constexpr int ld = NCP * 16 + 1;
  float* logits = reinterpret_cast<float*>(smem);
#pragma unroll
  for (int q = 0; q < kTTW; ++q)
#pragma unroll
    for (int i = 0; i < 4; ++i) logits[((tt0 + q) * 16 + 4 * (lane >> 4) + i) * ld + e] = acc[q][i];
  __syncthreads();
  for (int g = wave; g < kTok / 4; g += 8) {
    if (tok0 + 4 * g >= n_tokens) break;
    softmax_topk4<NCP>(logits + 4 * g * ld, ld, tok0 + 4 * g, n_tokens, n_expert, k, normalize != 0, ids, weights);
  }
}

// Softmax + top-k of prefill logits split over hidden ranges: each wave
// takes four tokens, sums their n_split partial logits in range order
// (four ranges' loads in flight at a time) into its LDS rows, then runs the
// four-token top-k.  n_expert <= 16 NV <= 128.
constexpr int kPartWaves = 4;

template <int NV>
__global__ __launch_bounds__(kPartWaves * kWave) void router_part_topk_kernel(
    const float* __restrict__ part, int n_split, int n_tokens, int n_expert, int k, int normalize,
    int* __restrict__ ids, float* __restrict__ weights) {
  constexpr int ld = 16 * NV + 1;
  __shared__ float lg[kPartWaves][4 * ld];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int t0 = (static_cast<int>(blockIdx.x) * kPartWaves + wave) * 4;
  if (t0 >= n_tokens) return;
  const int g = lane >> 4, j = lane & 15;
  const int t = min(t0 + g, n_tokens - 1);
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
  float* row = lg[wave];
#pragma unroll
  for (int i = 0; i < NV; ++i) row[g * ld + j + 16 * i] = v[i];
  // softmax_topk4 reads back only this lane's own values
  softmax_topk4<NV>(row, ld, t0, n_tokens, n_expert, k, normalize != 0, ids, weights);
}

// Hidden ranges of the split prefill router: at least one block per CU over
// the 64-token tiles, whole 128-column stages per range.
struct PrefillSplit {
  int n_split, stages_per_range;
};

PrefillSplit prefill_split(int n_tokens, int n_embd) {
  const int n_tt = (n_tokens + 63) / 64;
  const int n_st = n_embd / kTileCols;
  const int want = std::min(n_st, std::max(1, (256 + n_tt - 1) / n_tt));
  const int sps = (n_st + want - 1) / want;
  return {(n_st + sps - 1) / sps, sps};
}

// ---- Decode-sized batches (T <= kDecodeMaxTokens, bf16, k <= 16,
// n_expert <= 256): the logits are split over many blocks instead of
// streaming the whole router matrix through one CU, and one block finishes
// the softmax, top-k and the token -> expert permutation.
//
// router_split_logits_kernel: block (token group of 16, expert chunk of 16,
// column split of kSplitCols hidden columns); 4 waves take 128 columns each
// (4 trips of 32, all loaded before the first MFMA) and are summed in wave
// order.  part[(split * T + t) * E + e] holds the split's partial logit.
constexpr int kSplitCols = 512;
constexpr int kSplitWaves = 4;

__device__ __forceinline__ u32x4_t ld16(const bf16_t* p) { return *reinterpret_cast<const u32x4_t*>(p); }

__global__ __launch_bounds__(kSplitWaves * kWave) void router_split_logits_kernel(
    const bf16_t* __restrict__ x, const bf16_t* __restrict__ wr, int n_tokens, int n_embd, int n_expert,
    float* __restrict__ part) {
  __shared__ f32x4_t red[kSplitWaves][kWave];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int row = lane & 15, kofs = (lane >> 4) * 8;
  const int t = min(static_cast<int>(blockIdx.x) * 16 + row, n_tokens - 1);   // rows past the end repeat
  const int e = min(static_cast<int>(blockIdx.y) * 16 + row, n_expert - 1);   // the last token / expert
  const bf16_t* xr = x + static_cast<int64_t>(t) * n_embd + kofs;
  const bf16_t* wrow = wr + static_cast<int64_t>(e) * n_embd + kofs;
  const int h0 = static_cast<int>(blockIdx.z) * kSplitCols + wave * 128;
  const u32x4_t zero{0u, 0u, 0u, 0u};
  u32x4_t a[4], b[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int h = h0 + 32 * j;
    a[j] = h < n_embd ? ld16(xr + h) : zero;
    b[j] = h < n_embd ? ld16(wrow + h) : zero;
  }
  f32x4_t acc{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < 4; ++j)
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a[j]), __builtin_bit_cast(bf16x8_t, b[j]),
                                                  acc, 0, 0, 0);
  red[wave][lane] = acc;
  __syncthreads();
  if (wave == 0) {
    f32x4_t v = red[0][lane];
#pragma unroll
    for (int w = 1; w < kSplitWaves; ++w) v += red[w][lane];
    // D[token][expert]: lane holds expert (lane & 15), tokens 4*(lane>>4)+i.
    const int ee = static_cast<int>(blockIdx.y) * 16 + (lane & 15);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int tt = static_cast<int>(blockIdx.x) * 16 + (lane >> 4) * 4 + i;
      if (tt < n_tokens && ee < n_expert)
        part[(static_cast<int64_t>(blockIdx.z) * n_tokens + tt) * n_expert + ee] = v[i];
    }
  }
}

// One block: logits = the splits' partials summed in split order, softmax +
// top-k four tokens per wave (n_expert <= 16 NV), then the permutation of the
// k * T slot-major ids, read back from an LDS copy.  The partials of kSumU
// logits x kSumS splits are loaded before any is added, so a thread waits
// for memory once per group rather than once per partial.
constexpr int kSumU = 4, kSumS = 8;

size_t topk_permute_lds_bytes(int n_tokens, int n_expert, int k) {
  return (static_cast<size_t>((n_tokens + 3) / 4 * 4) * (n_expert + 1) + static_cast<size_t>(k) * n_tokens) * 4;
}

template <int NV>
__global__ __launch_bounds__(perm::kThreads) void router_topk_permute_kernel(
    const float* __restrict__ part, int n_split, int n_tokens, int n_expert, int k, int normalize,
    int* __restrict__ ids, float* __restrict__ weights, int* __restrict__ order, int* __restrict__ offsets,
    int* __restrict__ err_count) {
  extern __shared__ float lg[];  // [roundup(T, 4)][n_expert + 1] logits, then k * T ids
  const int ld = n_expert + 1;
  int* ids_lds = reinterpret_cast<int*>(lg + (n_tokens + 3) / 4 * 4 * ld);
  const int n = n_tokens * n_expert;
  for (int i0 = threadIdx.x; i0 < n; i0 += kSumU * perm::kThreads) {
    float acc[kSumU];
#pragma unroll
    for (int u = 0; u < kSumU; ++u) acc[u] = 0.f;
    for (int s0 = 0; s0 < n_split; s0 += kSumS) {
      float pv[kSumU][kSumS];
#pragma unroll
      for (int u = 0; u < kSumU; ++u)
#pragma unroll
        for (int q = 0; q < kSumS; ++q) {
          const int idx = i0 + u * perm::kThreads;
          pv[u][q] = idx < n && s0 + q < n_split ? part[static_cast<int64_t>(s0 + q) * n + idx] : 0.f;
        }
#pragma unroll
      for (int u = 0; u < kSumU; ++u)
#pragma unroll
        for (int q = 0; q < kSumS; ++q)
          if (s0 + q < n_split) acc[u] += pv[u][q];
    }
#pragma unroll
    for (int u = 0; u < kSumU; ++u) {
      const int idx = i0 + u * perm::kThreads;
      if (idx < n) {
        const int t = idx / n_expert;
        lg[t * ld + idx - t * n_expert] = acc[u];
      }
    }
  }
  lds_barrier();
  const int wave = threadIdx.x / kWave;
  for (int q = wave; 4 * q < n_tokens; q += perm::kWaves)
    softmax_topk4<NV>(lg + 4 * q * ld, ld, 4 * q, n_tokens, n_expert, k, normalize != 0, ids, weights, ids_lds);
  lds_barrier();
  perm::permute_block(ids_lds, k * n_tokens, n_expert, order, offsets, err_count);
}

// Batches of at most 4 tokens and 64 assignments: one wave does what
// router_topk_permute_kernel does with 16 (measured, whole block calls,
// cold: C4 T=1 39.8 -> 38.85 us, T=4 80.2 -> 79.5 us).  Lane (g, j) sums
// the partials of token g's experts j, j + 16, ... in split order (the same
// sums, so the same ids); the permutation ranks each flat id f among the
// others: its position is the number of ids of lower experts plus those of
// its expert before f, the stable counting sort's order.  Top-k ids are
// always valid experts, so the invalid-id count is zero.
template <int NV>
__global__ __launch_bounds__(kWave) void router_topk_permute_wave_kernel(
    const float* __restrict__ part, int n_split, int n_tokens, int n_expert, int k, int normalize,
    int* __restrict__ ids, float* __restrict__ weights, int* __restrict__ order, int* __restrict__ offsets,
    int* __restrict__ err_count) {
  __shared__ float lg[4 * (16 * NV + 1)];
  __shared__ int idl[kWave];
  wave_topk4_splits<NV>(part, n_split, n_tokens, n_expert, k, normalize != 0, lg, ids, weights, idl);
  __syncthreads();
  wave_permute(idl, k * n_tokens, n_expert, order, offsets);
  if (threadIdx.x == 0) err_count[0] = 0;
}

template <int NV>
hipError_t launch_topk_permute(const float* part, int n_split, int n_tokens, int n_expert, int k, bool normalize,
                               int* ids, float* weights, int* order, int* offsets, int* err, hipStream_t stream) {
  const size_t lds = topk_permute_lds_bytes(n_tokens, n_expert, k);
  // Up to 64 x 257 logits and 1024 ids, a little over the 64 KiB default.
  static const hipError_t attr = hipFuncSetAttribute(
      reinterpret_cast<const void*>(router_topk_permute_kernel<NV>), hipFuncAttributeMaxDynamicSharedMemorySize,
      static_cast<int>(topk_permute_lds_bytes(kDecodeMaxTokens, 256, 16)));
  (void)attr;
  hipLaunchKernelGGL((router_topk_permute_kernel<NV>), dim3(1), dim3(perm::kThreads), lds, stream, part, n_split,
                     n_tokens, n_expert, k, normalize ? 1 : 0, ids, weights, order, offsets, err);
  return hipGetLastError();
}

template <int NCH>
void launch_router_mfma(const void* x, const void* wr, int n_tokens, int n_embd, int n_expert, int k, bool normalize,
                        int* ids, float* weights, size_t lds, hipStream_t stream) {
  static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(router_mfma_bf16_kernel<NCH>),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
  (void)attr;
  hipLaunchKernelGGL((router_mfma_bf16_kernel<NCH>), dim3((n_tokens + kTok - 1) / kTok), dim3(kMfmaThreads), lds,
                     stream, static_cast<const bf16_t*>(x), static_cast<const bf16_t*>(wr), n_tokens, n_embd,
                     n_expert, k, normalize ? 1 : 0, ids, weights);
}

template <int NCP, int TT>
void launch_router_tile(const bf16_t* x, const bf16_t* wr, int n_tokens, int n_embd, int n_expert, int k,
                        bool normalize, int n_split, int stages_per_range, int* ids, float* weights, float* part,
                        hipStream_t stream) {
  constexpr int lds = kTileRing * tile_stage_bytes<NCP, TT>();
  static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(router_tile_bf16_kernel<NCP, TT>),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  (void)attr;
  hipLaunchKernelGGL((router_tile_bf16_kernel<NCP, TT>), dim3((n_tokens + TT * 16 - 1) / (TT * 16), n_split),
                     dim3(512), lds, stream, x, wr, n_tokens, n_embd, n_expert, k, normalize ? 1 : 0,
                     stages_per_range, ids, weights, part);
}

}  // namespace

hipError_t launch_router(const void* x, const void* wr, int n_tokens, int n_embd, int n_expert,
                         int k, bool normalize, int dtype, int* ids, float* weights,
                         hipStream_t stream) {
  if (n_tokens == 0) return hipSuccess;
  if (n_expert > kMaxExpert) return hipErrorInvalidValue;
  const dim3 grid((n_tokens + kTok - 1) / kTok);
  const bool aligned = (reinterpret_cast<uintptr_t>(x) % 16 == 0) &&
                       (reinterpret_cast<uintptr_t>(wr) % 16 == 0);
  if (dtype == DT_BF16 && n_embd % kTileCols == 0 && n_expert > 32 && n_expert <= kMfmaMaxExpert && k <= 16 &&
      aligned) {
    const int n_st = n_embd / kTileCols;
    if (n_expert <= 64)
      launch_router_tile<4, 2>(static_cast<const bf16_t*>(x), static_cast<const bf16_t*>(wr), n_tokens, n_embd,
                               n_expert, k, normalize, 1, n_st, ids, weights, nullptr, stream);
    else
      launch_router_tile<8, 2>(static_cast<const bf16_t*>(x), static_cast<const bf16_t*>(wr), n_tokens, n_embd,
                               n_expert, k, normalize, 1, n_st, ids, weights, nullptr, stream);
  } else if (dtype == DT_BF16 && n_embd % 32 == 0 && n_expert <= kMfmaMaxExpert && aligned) {
    const int ld = ((n_expert + 15) / 16) * 16 + 1;
    const size_t lds = static_cast<size_t>(kMfmaWaves + 1) * kTok * ld * sizeof(float);
    const int n_chunks = (n_expert + 15) / 16;
    if (n_chunks == 1)
      launch_router_mfma<1>(x, wr, n_tokens, n_embd, n_expert, k, normalize, ids, weights, lds, stream);
    else if (n_chunks == 2)
      launch_router_mfma<2>(x, wr, n_tokens, n_embd, n_expert, k, normalize, ids, weights, lds, stream);
    else
      launch_router_mfma<kMfmaMaxExpert / 16>(x, wr, n_tokens, n_embd, n_expert, k, normalize, ids, weights, lds,
                                              stream);
  } else {
    const size_t lds = static_cast<size_t>(kTok) * (n_expert + 1) * sizeof(float);
    if (dtype == DT_BF16) {
      hipLaunchKernelGGL(router_simt_kernel<bf16_t>, grid, dim3(kThreads), lds, stream,
                         static_cast<const bf16_t*>(x), static_cast<const bf16_t*>(wr), n_tokens,
                         n_embd, n_expert, k, normalize ? 1 : 0, ids, weights);
    } else {
      hipLaunchKernelGGL(router_simt_kernel<float>, grid, dim3(kThreads), lds, stream,
                         static_cast<const float*>(x), static_cast<const float*>(wr), n_tokens,
                         n_embd, n_expert, k, normalize ? 1 : 0, ids, weights);
    }
  }
  return hipGetLastError();
}

}  // namespace fmoe

namespace fmoe {

size_t router_prefill_scratch_bytes(int n_tokens, int n_embd, int n_expert, int k, int dtype) {
  if (dtype != DT_BF16 || n_tokens <= kDecodeMaxTokens || n_embd % kTileCols || n_expert <= 32 ||
      n_expert > kMfmaMaxExpert || k <= 0 || k > 16 || k > n_expert)
    return 0;
  return static_cast<size_t>(prefill_split(n_tokens, n_embd).n_split) * n_tokens * n_expert * sizeof(float);
}

hipError_t launch_router_prefill(const void* x, const void* wr, int n_tokens, int n_embd, int n_expert, int k,
                                 bool normalize, int dtype, float* part, int* ids, float* weights,
                                 hipStream_t stream) {
  if (!part || router_prefill_scratch_bytes(n_tokens, n_embd, n_expert, k, dtype) == 0 ||
      reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(wr) % 16)
    return hipErrorNotSupported;
  const PrefillSplit ps = prefill_split(n_tokens, n_embd);
  const bf16_t* xb = static_cast<const bf16_t*>(x);
  const bf16_t* wb = static_cast<const bf16_t*>(wr);
  if (n_expert <= 64)
    launch_router_tile<4, 4>(xb, wb, n_tokens, n_embd, n_expert, k, normalize, ps.n_split, ps.stages_per_range, ids,
                             weights, part, stream);
  else
    launch_router_tile<8, 4>(xb, wb, n_tokens, n_embd, n_expert, k, normalize, ps.n_split, ps.stages_per_range, ids,
                             weights, part, stream);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const dim3 grid((n_tokens + 4 * kPartWaves - 1) / (4 * kPartWaves));
  if (n_expert <= 64)
    hipLaunchKernelGGL(router_part_topk_kernel<4>, grid, dim3(kPartWaves * kWave), 0, stream, part, ps.n_split,
                       n_tokens, n_expert, k, normalize ? 1 : 0, ids, weights);
  else
    hipLaunchKernelGGL(router_part_topk_kernel<8>, grid, dim3(kPartWaves * kWave), 0, stream, part, ps.n_split,
                       n_tokens, n_expert, k, normalize ? 1 : 0, ids, weights);
  return hipGetLastError();
}

size_t router_decode_scratch_bytes(int n_tokens, int n_embd, int n_expert, int k, int dtype) {
  if (dtype != DT_BF16 || n_tokens <= 0 || n_tokens > kDecodeMaxTokens || n_embd % 32 || n_expert <= 0 ||
      n_expert > 256 || k <= 0 || k > 16 || k > n_expert)
    return 0;
  const int n_split = (n_embd + kSplitCols - 1) / kSplitCols;
  return static_cast<size_t>(n_split) * n_tokens * n_expert * sizeof(float);
}

int router_decode_splits(int n_embd) { return (n_embd + kSplitCols - 1) / kSplitCols; }

hipError_t launch_router_split_logits(const void* x, const void* wr, int n_tokens, int n_embd, int n_expert, int k,
                                      int dtype, float* part, int* n_split_out, hipStream_t stream) {
  if (!part || router_decode_scratch_bytes(n_tokens, n_embd, n_expert, k, dtype) == 0 ||
      reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(wr) % 16)
    return hipErrorNotSupported;
  const int n_split = router_decode_splits(n_embd);
  hipLaunchKernelGGL(router_split_logits_kernel, dim3((n_tokens + 15) / 16, (n_expert + 15) / 16, n_split),
                     dim3(kSplitWaves * kWave), 0, stream, static_cast<const bf16_t*>(x),
                     static_cast<const bf16_t*>(wr), n_tokens, n_embd, n_expert, part);
  *n_split_out = n_split;
  return hipGetLastError();
}

hipError_t launch_router_decode(const void* x, const void* wr, int n_tokens, int n_embd, int n_expert, int k,
                                bool normalize, int dtype, float* part, int* ids, float* weights, int* order,
                                int* offsets, int* err_count, hipStream_t stream) {
  int n_split = 0;
  const hipError_t e = launch_router_split_logits(x, wr, n_tokens, n_embd, n_expert, k, dtype, part, &n_split, stream);
  if (e != hipSuccess) return e;
  const int nv = (n_expert + 15) / 16;
  if (n_expert > 64 && n_tokens > 32) {
    // Many experts and tokens: one block's waves would select every token's
    // experts on one CU's 4 SIMDs (C3 T=64: 14.5 us for the fused kernel).
    // The prefill top-k (same partial layout, splits summed in the same
    // order) spreads the tokens over blocks; the one-block permutation
    // follows as its own launch.  Measured (whole block calls, cold): C3
    // T=64 123.0 -> 119.4 us; at T=16 the fused kernel is ahead (77.3 against
    // 78.8 us), its 4 waves one per SIMD.
    const dim3 grid((n_tokens + 4 * kPartWaves - 1) / (4 * kPartWaves));
    if (nv <= 8)
      hipLaunchKernelGGL(router_part_topk_kernel<8>, grid, dim3(kPartWaves * kWave), 0, stream, part, n_split,
                         n_tokens, n_expert, k, normalize ? 1 : 0, ids, weights);
    else
      hipLaunchKernelGGL(router_part_topk_kernel<16>, grid, dim3(kPartWaves * kWave), 0, stream, part, n_split,
                         n_tokens, n_expert, k, normalize ? 1 : 0, ids, weights);
    const hipError_t e2 = hipGetLastError();
    if (e2 != hipSuccess) return e2;
    return launch_permute(ids, k * n_tokens, n_expert, order, offsets, err_count, nullptr, stream);
  }
  if (n_tokens <= 4 && k * n_tokens <= kWave) {
    // one wave (see router_topk_permute_wave_kernel)
#define FMOE_TOPK_WAVE(NV)                                                                                    \
    hipLaunchKernelGGL(router_topk_permute_wave_kernel<NV>, dim3(1), dim3(kWave), 0, stream, part, n_split, \
                       n_tokens, n_expert, k, normalize ? 1 : 0, ids, weights, order, offsets, err_count)
    if (nv <= 1) FMOE_TOPK_WAVE(1);
    else if (nv <= 2) FMOE_TOPK_WAVE(2);
    else if (nv <= 4) FMOE_TOPK_WAVE(4);
    else if (nv <= 8) FMOE_TOPK_WAVE(8);
    else FMOE_TOPK_WAVE(16);
#undef FMOE_TOPK_WAVE
    return hipGetLastError();
  }
  if (nv <= 1) return launch_topk_permute<1>(part, n_split, n_tokens, n_expert, k, normalize, ids, weights, order, offsets, err_count, stream);
  if (nv <= 2) return launch_topk_permute<2>(part, n_split, n_tokens, n_expert, k, normalize, ids, weights, order, offsets, err_count, stream);
  if (nv <= 4) return launch_topk_permute<4>(part, n_split, n_tokens, n_expert, k, normalize, ids, weights, order, offsets, err_count, stream);
  if (nv <= 8) return launch_topk_permute<8>(part, n_split, n_tokens, n_expert, k, normalize, ids, weights, order, offsets, err_count, stream);
  return launch_topk_permute<16>(part, n_split, n_tokens, n_expert, k, normalize, ids, weights, order, offsets, err_count, stream);
}

}  // namespace fmoe
