// The decode step's attention half: paged KV cache copies, the projection
// epilogue (bias + RoPE), and grouped-query attention of one new token per
// sequence against the paged cache.
//
// Paged cache (components/kvcache/kvcache.mlir, oracles/kvcache.py:51-185):
// a pool [n_blocks, block_size, n_head_kv, head_dim]; sequence b's position
// j lives in physical block block_tables[b, j / block_size] at row
// j % block_size.  The reference gathers max_context_len positions per
// sequence (zero rows at and past context_lens[b]), appends the new K/V and
// runs attention_gqa without a mask (attention_block_decode.mlir:202-216,
// attention_gqa.mlir:120-137).  The attention kernels here read the pool in
// place instead of gathering: the zero rows' contribution is exact in closed
// form (score 0, value 0), so they are counted, not read.
//
// Attention is split over the context: one block per (split of kSplitLen
// positions, KV head, sequence) computes, for the G query heads sharing the
// KV head, the split's max score, sum of exp and unnormalised output; a
// combine kernel merges the splits in order with the zero rows and the new
// token and, in the paged calls, writes the new K/V rows into the pools.
// Where the streaming GEMM does not apply its own epilogue (fp32
// activations, more than 16 rows for Q/K/V), the separate bias + RoPE and
// bias + cast kernels here finish the projections.
#include "common.h"
#include "launch.h"

namespace fmoe {
namespace {

constexpr int kCopyThreads = 256;

// ------------------------------------------------------------------ cache copies
// Rows are copied as 32-bit words (a row is n_head_kv * head_dim elements,
// head_dim even, so a bf16 row is a whole number of words).

__global__ __launch_bounds__(kCopyThreads) void kv_gather_kernel(const uint32_t* __restrict__ cache, int64_t n_blocks,
                                                                 int block_size, int row_words,
                                                                 const int* __restrict__ tables, int max_blocks,
                                                                 const int* __restrict__ ctx_lens, int max_ctx,
                                                                 uint32_t* __restrict__ out) {
  const int j = blockIdx.x, b = blockIdx.y;
  const int n = min(max(ctx_lens[b], 0), max_ctx);
  const uint32_t* src = nullptr;
  if (j < n) {
    const int lb = j / block_size;
    const int pb = lb < max_blocks ? tables[static_cast<int64_t>(b) * max_blocks + lb] : -1;
    if (pb >= 0 && pb < n_blocks) src = cache + (static_cast<int64_t>(pb) * block_size + j % block_size) * row_words;
  }
  uint32_t* dst = out + (static_cast<int64_t>(b) * max_ctx + j) * row_words;
  for (int w = threadIdx.x; w < row_words; w += kCopyThreads) dst[w] = src ? src[w] : 0u;
}

// Sequence b's new row into slot (block_idx[b], pos_idx[b]) of `cache`, by
// a whole block of NT threads.  When several sequences name the same slot
// the last one wins, as in the reference's sequential loop
// (oracles/kvcache.py:134-139); slots outside the pool are skipped.
template <int NT>
__device__ void scatter_decode_row(uint32_t* __restrict__ cache, int64_t n_blocks, int block_size, int row_words,
                                   const uint32_t* __restrict__ vals, const int* __restrict__ block_idx,
                                   const int* __restrict__ pos_idx, int batch, int b) {
  const int bi = block_idx[b], p = pos_idx[b];
  bool later = false;
  for (int b2 = b + 1 + static_cast<int>(threadIdx.x); b2 < batch; b2 += NT)
    later |= block_idx[b2] == bi && pos_idx[b2] == p;
  if (__syncthreads_or(later)) return;
  if (bi < 0 || bi >= n_blocks || p < 0 || p >= block_size) return;
  uint32_t* dst = cache + (static_cast<int64_t>(bi) * block_size + p) * row_words;
  const uint32_t* src = vals + static_cast<int64_t>(b) * row_words;
  for (int w = threadIdx.x; w < row_words; w += NT) dst[w] = src[w];
}

__global__ __launch_bounds__(kCopyThreads) void kv_scatter_decode_kernel(uint32_t* __restrict__ cache,
                                                                         int64_t n_blocks, int block_size,
                                                                         int row_words,
                                                                         const uint32_t* __restrict__ vals,
                                                                         const int* __restrict__ block_idx,
                                                                         const int* __restrict__ pos_idx, int batch) {
  scatter_decode_row<kCopyThreads>(cache, n_blocks, block_size, row_words, vals, block_idx, pos_idx, batch,
                                   blockIdx.x);
}

__global__ __launch_bounds__(kCopyThreads) void kv_scatter_prefill_kernel(
    uint32_t* __restrict__ cache, int64_t n_blocks, int block_size, int row_words, const uint32_t* __restrict__ vals,
    int seq_len, const int* __restrict__ tables, int max_blocks, const int* __restrict__ start) {
  const int s = blockIdx.x, b = blockIdx.y;
  const int64_t p = static_cast<int64_t>(start[b]) + s;
  if (p < 0) return;
  const int64_t lb = p / block_size;
  if (lb >= max_blocks) return;
  const int pb = tables[static_cast<int64_t>(b) * max_blocks + lb];
  if (pb < 0 || pb >= n_blocks) return;
  uint32_t* dst = cache + (static_cast<int64_t>(pb) * block_size + p % block_size) * row_words;
  const uint32_t* src = vals + (static_cast<int64_t>(b) * seq_len + s) * row_words;
  for (int w = threadIdx.x; w < row_words; w += kCopyThreads) dst[w] = src[w];
}

// ------------------------------------------------------------------ small helpers
__global__ void iota_kernel(int* __restrict__ v, int n, int* __restrict__ pair, int pair0, int pair1) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) v[i] = i;
  if (i == 0 && pair) {
    pair[0] = pair0;
    pair[1] = pair1;
  }
}

__global__ void fill_int_kernel(int* __restrict__ v, int n, int value) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) v[i] = value;
}

__device__ __forceinline__ float load_act(const void* p, int dt, int64_t i) {
  return dt == DT_F32 ? static_cast<const float*>(p)[i] : bf16_to_f32(static_cast<const bf16_t*>(p)[i]);
}

__device__ __forceinline__ void store_act(void* p, int dt, int64_t i, float v) {
  if (dt == DT_F32)
    static_cast<float*>(p)[i] = v;
  else
    static_cast<bf16_t*>(p)[i] = f32_to_bf16(v);
}

// qkv [B, nq + 2 nkv] fp32 GEMM output -> + bias, RoPE on the q and k parts
// (pairs (2i, 2i+1), angle pos * freq_scale / freq_base^(2i/D), in double
// precision like the reference oracle), q_rot fp32 [B, nq], k_new / v_new
// [B, nkv] in act dtype (rope.mlir:38-104, oracles/position.py:6-50).
__device__ __forceinline__ float split_sum(const float* p, int nsplit, int64_t stride) {
  float v = p[0];
  for (int k = 1; k < nsplit; ++k) v += p[k * stride];
  return v;
}

__global__ __launch_bounds__(256) void qkv_rope_kernel(const float* __restrict__ qkv, int nsplit, int64_t split_stride,
                                                       const float* __restrict__ bq, const float* __restrict__ bk,
                                                       const float* __restrict__ bv,
                                                       const int64_t* __restrict__ positions, int nq, int nkv, int D,
                                                       double freq_base, double freq_scale, float* __restrict__ q_rot,
                                                       void* __restrict__ k_new, void* __restrict__ v_new, int act) {
  // grid (batch, items / 256): an item is a RoPE pair of the q or k part or
  // one element of the v part
  const int b = blockIdx.x;
  const int i = blockIdx.y * blockDim.x + threadIdx.x;
  const int pairs = (nq + nkv) / 2;
  if (i >= pairs + nkv) return;
  const int width = nq + 2 * nkv;
  const float* row = qkv + static_cast<int64_t>(b) * width;
  if (i >= pairs) {
    const int c = i - pairs;
    float v = split_sum(row + nq + nkv + c, nsplit, split_stride);
    if (bv) v += bv[c];
    store_act(v_new, act, static_cast<int64_t>(b) * nkv + c, v);
    return;
  }
  const int col = 2 * i;
  const bool is_q = col < nq;
  const int c = is_q ? col : col - nq;
  const float* bias = is_q ? bq : bk;
  float x0 = split_sum(row + col, nsplit, split_stride), x1 = split_sum(row + col + 1, nsplit, split_stride);
  if (bias) {
    x0 += bias[c];
    x1 += bias[c + 1];
  }
  float y0, y1;
  rope_pair(x0, x1, positions[b], (c % D) / 2, D, freq_base, freq_scale, y0, y1);
  if (is_q) {
    q_rot[static_cast<int64_t>(b) * nq + c] = y0;
    q_rot[static_cast<int64_t>(b) * nq + c + 1] = y1;
  } else {
    store_act(k_new, act, static_cast<int64_t>(b) * nkv + c, y0);
    store_act(k_new, act, static_cast<int64_t>(b) * nkv + c + 1, y1);
  }
}

// out[b, n] = y[b, n] (+ bias[n]) in act dtype.
// out may alias residual (element-wise, same index).
__global__ __launch_bounds__(256) void bias_cast_kernel(const float* __restrict__ y, int nsplit, int64_t split_stride,
                                                        const float* __restrict__ bias, const void* residual,
                                                        void* out, int64_t rows, int n, int act) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= rows * n) return;
  float v = split_sum(y + i, nsplit, split_stride);
  if (bias) v += bias[i % n];
  if (residual) {
    // the reference rounds the attention output, then adds
    // (transformer_layer_moe_decode.mlir:208-221)
    if (act == DT_BF16) v = bf16_to_f32(f32_to_bf16(v));
    v += load_act(residual, act, i);
  }
  store_act(out, act, i, v);
}

// ------------------------------------------------------------------ split attention
// Two bf16 (low element first) -> two floats.
__device__ __forceinline__ void unpack2(uint32_t w, float* v) {
  v[0] = __uint_as_float(w << 16);
  v[1] = __uint_as_float(w & 0xFFFF0000u);
}

__device__ __forceinline__ f32x4_t attn_mfma16(const u32x4_t a, const u32x4_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                0, 0, 0);
}

struct AttnArgs {
  const float* q;         // [B, n_head * D] fp32, RoPE applied
  const void* k_pool;     // [n_blocks, block_size, n_head_kv, D]
  const void* v_pool;
  const int* tables;      // [B, max_blocks] (this layer)
  const int* ctx_lens;    // [B] (this layer)
  int max_blocks;
  int max_ctx;
  int64_t n_blocks;
  int block_size;
  int n_head, n_head_kv;
  int n_split;
  float scale;
  float* part;            // [B, n_head, n_split, D + 2]: o[D], m, l
};

constexpr int kSplitLen = 256;
constexpr int kAttnThreads = 256;  // one thread per position of a split (rows[] fill)
static_assert(kAttnThreads == kSplitLen, "the rows[] fill gives each thread one position");
constexpr int kAttnWaves = kAttnThreads / kWave;

// Block (split s, KV head, sequence b); wave w owns the split's positions
// [64 w, 64 w + 64) in both phases, so a wave's memory traffic is two
// rounds of independent loads: all of its K rows, then (issued before the
// block-wide softmax, so that their latency overlaps it) all of its V rows.
// Scores: LP lanes per position, each lane holding DL = D/LP dimensions in
// chunks of up to 16 bytes spread so that the LP lanes of a position read
// each span of the row together; the G query heads of the KV head are
// scored from one read of K (query registers: G * DL per lane).  P.V: LPR
// lanes per row, 16 bytes each.
template <typename T, int D, int G, int LP>
__global__ __launch_bounds__(kAttnThreads) void attn_split_kernel(AttnArgs a) {
  constexpr int DL = D / LP;
  static_assert(G <= LP, "one lane per query head stores its score");
  constexpr int EPV = 16 / static_cast<int>(sizeof(T));  // elements per 16 bytes
  constexpr int CW = EPV < DL ? EPV : DL;                 // score chunk (elements)
  constexpr int NC = DL / CW;                             // score chunks per lane per position
  constexpr int kQ = kSplitLen / kAttnWaves;              // positions per wave
  constexpr int PPS = kWave / LP;                         // positions per score step
  constexpr int kSteps = kQ / PPS;                        // score steps
  constexpr int SR = 16 / NC < kSteps ? 16 / NC : kSteps;  // steps per load round (<= 16 loads)
  constexpr int VC = EPV;                                 // P.V elements per lane per row
  constexpr int LPR = D / VC;                             // lanes per row
  constexpr int PP = kWave / LPR;                         // rows per load instruction
  constexpr int NV = kQ / PP;                             // V load instructions per wave
  constexpr int VR = NV < 16 ? NV : 16;                   // per round
  static_assert(kSteps % SR == 0 && NV % VR == 0, "rounds must tile the wave's positions");
  constexpr bool kMfmaScores = sizeof(T) == 2 && (D == 64 || D == 128) && G <= 8 && kQ % 8 == 0;
  __shared__ float sc[G][kSplitLen];
  __shared__ int rows[kSplitLen];
  __shared__ float red[kAttnWaves][G][D];
  __shared__ float stat[G][2];

  const int s = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int n_b = min(max(a.ctx_lens[b], 0), a.max_ctx);
  const int j0 = s * kSplitLen;
  const int len = min(kSplitLen, n_b - j0);  // block-uniform; <= 0: no cached position here
  float* part = a.part + (static_cast<int64_t>(b) * a.n_head + kvh * G) * a.n_split * (D + 2);
  if (len <= 0) {
    for (int i = tid; i < G * (D + 2); i += kAttnThreads) {
      const int g = i / (D + 2), k = i - g * (D + 2);
      part[(static_cast<int64_t>(g) * a.n_split + s) * (D + 2) + k] = k == D ? -INFINITY : 0.f;
    }
    return;
  }
  const int64_t row_elems = static_cast<int64_t>(a.n_head_kv) * D;
  {
    const int t = tid;  // kAttnThreads == kSplitLen: one position per thread
    int r = -2;         // -2: past the split's positions; -1: table entry outside the pool (a zero row)
    if (t < len) {
      const int j = j0 + t;
      const int lb = j / a.block_size;
      const int pb = lb < a.max_blocks ? a.tables[static_cast<int64_t>(b) * a.max_blocks + lb] : -1;
      r = (pb >= 0 && pb < a.n_blocks) ? pb * a.block_size + j % a.block_size : -1;
    }
    rows[t] = r;
  }
  const T* kp = static_cast<const T*>(a.k_pool) + static_cast<int64_t>(kvh) * D;
  const T* vp = static_cast<const T*>(a.v_pool) + static_cast<int64_t>(kvh) * D;
  const int tw = wave * kQ;  // this wave's first position
  if constexpr (kMfmaScores) {
    // ---- scores on the matrix cores (v_mfma_f32_16x16x32_bf16), 8
    // positions per tile.  A row i = 2p + s holds half s of position p's K
    // row, B column j = 2h + s' half s' of query head h (heads >= G zero):
    // at step ks, lane group kg (lane >> 4) of row / column parity s takes
    // the 8 dimensions of chunk 8 ks + 4 s + kg, so the 8 lanes of a
    // position read 128 contiguous bytes per load.  score(p, h) =
    // D[2p][2h] + D[2p+1][2h+1]; the cross terms (s != s') are unused.  q is
    // split into bf16 high and low parts (two MFMAs per step): the products
    // carry q * scale to about 16 significant bits, K is exact in bf16 and
    // the sums are fp32.
    constexpr int NKS = D / 64, PT = kQ / 8;
    const int kg = lane >> 4, par = lane & 1, hh = (lane & 15) >> 1;
    u32x4_t qh[NKS], ql[NKS];
    {
      const float* qg = a.q + (static_cast<int64_t>(b) * a.n_head + kvh * G + (hh < G ? hh : 0)) * D;
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int d = (ks * 8 + par * 4 + kg) * 8 + 2 * e;
          const float x0 = hh < G ? qg[d] * a.scale : 0.f;
          const float x1 = hh < G ? qg[d + 1] * a.scale : 0.f;
          const uint32_t h = pack_bf16x2(x0, x1);
          qh[ks][e] = h;
          ql[ks][e] = pack_bf16x2(x0 - __uint_as_float(h << 16), x1 - __uint_as_float(h & 0xFFFF0000u));
        }
    }
    __syncthreads();  // rows[]
    u32x4_t kr[PT][NKS];
#pragma unroll
    for (int pt = 0; pt < PT; ++pt) {
      const int r = rows[tw + pt * 8 + hh];
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks)
        kr[pt][ks] = r >= 0 ? *reinterpret_cast<const u32x4_t*>(kp + r * row_elems + (ks * 8 + par * 4 + kg) * 8)
                            : u32x4_t{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int pt = 0; pt < PT; ++pt) {
      f32x4_t c{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        c = attn_mfma16(kr[pt][ks], qh[ks], c);
        c = attn_mfma16(kr[pt][ks], ql[ks], c);
      }
      // lane (kg, column 2h + s'): c[r] = D[4 kg + r][2h + s'], rows 4 kg + r
      // = position 2 kg + (r >> 1), half r & 1
      const float odd1 = __shfl_xor(c[1], 1, kWave), odd3 = __shfl_xor(c[3], 1, kWave);
      if (par == 0 && hh < G) {
        const int t = tw + pt * 8 + 2 * kg;
        sc[hh][t] = rows[t] == -2 ? -INFINITY : c[0] + odd1;  // a zero row scores 0
        sc[hh][t + 1] = rows[t + 1] == -2 ? -INFINITY : c[2] + odd3;
      }
    }
  } else {
  const int pi = lane / LP, sub = lane % LP;
  float q[G][DL];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int e = 0; e < CW; ++e)
        q[g][c * CW + e] =
            a.q[(static_cast<int64_t>(b) * a.n_head + kvh * G + g) * D + c * LP * CW + sub * CW + e] * a.scale;
  __syncthreads();

  // ---- scores, SR steps of 8 positions per round of loads; K stays in its
  // storage format (CWW 32-bit words per chunk) until it is used
  constexpr int CWW = CW * static_cast<int>(sizeof(T)) / 4;
#pragma unroll
  for (int r0 = 0; r0 < kSteps; r0 += SR) {
    uint32_t kr[SR][NC][CWW];
    int rr[SR];
#pragma unroll
    for (int u = 0; u < SR; ++u) {
      rr[u] = rows[tw + (r0 + u) * PPS + pi];
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const T* src = kp + rr[u] * row_elems + c * LP * CW + sub * CW;
        if (CWW == 4) {
          const u32x4_t w = rr[u] >= 0 ? *reinterpret_cast<const u32x4_t*>(src) : u32x4_t{0u, 0u, 0u, 0u};
          kr[u][c][0] = w[0], kr[u][c][1 % CWW] = w[1], kr[u][c][2 % CWW] = w[2], kr[u][c][3 % CWW] = w[3];
        } else if (CWW == 2) {
          const u32x2_t w = rr[u] >= 0 ? *reinterpret_cast<const u32x2_t*>(src) : u32x2_t{0u, 0u};
          kr[u][c][0] = w[0], kr[u][c][1 % CWW] = w[1];
        } else {
          kr[u][c][0] = rr[u] >= 0 ? *reinterpret_cast<const uint32_t*>(src) : 0u;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < SR; ++u) {
      const int t = tw + (r0 + u) * PPS + pi;
      float kv[DL];
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        if (sizeof(T) == 4) {
#pragma unroll
          for (int e = 0; e < CW; ++e) kv[c * CW + e] = __uint_as_float(kr[u][c][e % CWW]);
        } else {
#pragma unroll
          for (int e = 0; e < CWW; ++e) unpack2(kr[u][c][e], kv + c * CW + 2 * e);
        }
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < DL; ++i) acc = fmaf(q[g][i], kv[i], acc);
#pragma unroll
        for (int o = 1; o < LP; o <<= 1) acc += __shfl_xor(acc, o, kWave);
        if (sub == g) sc[g][t] = rr[u] == -2 ? -INFINITY : acc;  // a zero row scores 0
      }
    }
  }
  }

  // ---- V rows of this wave, first round issued before the softmax
  const int pr = lane / LPR, dl = lane - pr * LPR;
  u32x4_t vraw[VR];
  auto load_v = [&](int i0) {
#pragma unroll
    for (int i = 0; i < VR; ++i) {
      const int r = rows[tw + (i0 + i) * PP + pr];
      vraw[i] = r >= 0 ? *reinterpret_cast<const u32x4_t*>(vp + r * row_elems + dl * VC) : u32x4_t{0u, 0u, 0u, 0u};
    }
  };
  load_v(0);
  __syncthreads();

  // ---- per-head max and sum of exp over the split's len positions (only
  // those scores were written); probabilities in place
  for (int g = wave; g < G; g += kAttnWaves) {
    float m = -INFINITY;
    for (int t = lane; t < len; t += kWave) m = fmaxf(m, sc[g][t]);
    m = wave_max(m);
    float l = 0.f;
    for (int t = lane; t < len; t += kWave) {
      const float p = __expf(sc[g][t] - m);
      sc[g][t] = p;
      l += p;
    }
    l = wave_sum(l);
    if (lane == 0) {
      stat[g][0] = m;
      stat[g][1] = l;
    }
  }
  __syncthreads();

  // ---- P.V over this wave's positions
  float acc[G][VC];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < VC; ++e) acc[g][e] = 0.f;
#pragma unroll
  for (int i0 = 0; i0 < NV; i0 += VR) {
    if (i0 > 0) load_v(i0);
#pragma unroll
    for (int i = 0; i < VR; ++i) {
      const int t = tw + (i0 + i) * PP + pr;
      if (t < len) {
        float v[VC];
        if (sizeof(T) == 4) {
#pragma unroll
          for (int e = 0; e < VC; ++e) v[e] = __uint_as_float(vraw[i][e]);
        } else {
#pragma unroll
          for (int e = 0; e < VC / 2; ++e) unpack2(vraw[i][e], v + 2 * e);
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const float p = sc[g][t];
#pragma unroll
          for (int e = 0; e < VC; ++e) acc[g][e] = fmaf(p, v[e], acc[g][e]);
        }
      }
    }
  }
  // rows handled by different lane groups of the wave, then the waves in order
#pragma unroll
  for (int o = LPR; o < kWave; o <<= 1)
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < VC; ++e) acc[g][e] += __shfl_xor(acc[g][e], o, kWave);
  if (pr == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < VC; ++e) red[wave][g][dl * VC + e] = acc[g][e];
  }
  __syncthreads();
  for (int i = tid; i < G * D; i += kAttnThreads) {
    const int g = i / D, d = i - g * D;
    float o = red[0][g][d];
#pragma unroll
    for (int w = 1; w < kAttnWaves; ++w) o += red[w][g][d];
    float* pg = part + (static_cast<int64_t>(g) * a.n_split + s) * (D + 2);
    pg[d] = o;
    if (d == 0) {
      pg[D] = stat[g][0];
      pg[D + 1] = stat[g][1];
    }
  }
}

// One block per (query head, sequence) merges the context splits with the
// zero rows of the gather (max_ctx - min(ctx_len, max_ctx) keys of score 0
// and value 0) and the new token, whose K/V (RoPE applied) are k_new/v_new.
// Wave 0 reduces the per-split statistics with one split per lane and
// leaves the split weights exp(m_s - M) in LDS; then thread d adds
// dimension d over the splits, kCombineUnroll loads at a time.
constexpr int kCombineThreads = 128;  // >= head_dim
constexpr int kCombineChunk = 1024;   // splits whose weights are held in LDS at once
constexpr int kCombineUnroll = 16;
constexpr int kCombinePre = 16;       // splits (4096 positions) prefetched into registers

// Blocks x = n_head and n_head + 1 (launched only with a scatter) write
// k_new / v_new into the pools: the split kernel has read them by then.
__global__ __launch_bounds__(kCombineThreads) void attn_combine_kernel(AttnArgs a, int D,
                                                                       const void* __restrict__ k_new,
                                                                       const void* __restrict__ v_new, int act,
                                                                       void* __restrict__ out, KvScatterDecode sc) {
  __shared__ float wts[kCombineChunk];
  __shared__ float stat[3];  // M, 1 / l, exp(s_new - M) / l
  const int h = blockIdx.x, b = blockIdx.y;
  if (h >= a.n_head) {  // block-uniform
    const bool v = h > a.n_head;
    scatter_decode_row<kCombineThreads>(static_cast<uint32_t*>(v ? sc.v_cache : sc.k_cache), sc.n_blocks,
                                        sc.block_size, sc.row_bytes / 4,
                                        static_cast<const uint32_t*>(v ? v_new : k_new), sc.block_idx, sc.pos_idx,
                                        static_cast<int>(gridDim.y), b);
    return;
  }
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int kvh = h / (a.n_head / a.n_head_kv);
  const int n_b = min(max(a.ctx_lens[b], 0), a.max_ctx);
  const int n_zero = a.max_ctx - n_b;
  const int n_used = (n_b + kSplitLen - 1) / kSplitLen;
  const float* qh = a.q + (static_cast<int64_t>(b) * a.n_head + h) * D;
  const int64_t kv0 = (static_cast<int64_t>(b) * a.n_head_kv + kvh) * D;
  const float* part = a.part + (static_cast<int64_t>(b) * a.n_head + h) * a.n_split * (D + 2);
  // The first kCombinePre splits' outputs and v_new are loaded before the
  // statistics, so their latency overlaps wave 0's reductions.
  const int n_pre = min(n_used, kCombinePre);
  float pv[kCombinePre];
#pragma unroll
  for (int u = 0; u < kCombinePre; ++u)
    pv[u] = tid < D && u < n_pre ? part[static_cast<int64_t>(u) * (D + 2) + tid] : 0.f;
  const float vn = tid < D ? load_act(v_new, act, kv0 + tid) : 0.f;
  if (tid < kWave) {
    float dot = 0.f;
    for (int d = lane; d < D; d += kWave) dot = fmaf(qh[d] * a.scale, load_act(k_new, act, kv0 + d), dot);
    const float s_new = wave_sum(dot);
    const float m0 = lane < n_used ? part[static_cast<int64_t>(lane) * (D + 2) + D] : -INFINITY;
    float M = fmaxf(fmaxf(s_new, n_zero > 0 ? 0.f : -INFINITY), m0);
    for (int s = lane + kWave; s < n_used; s += kWave) M = fmaxf(M, part[static_cast<int64_t>(s) * (D + 2) + D]);
    M = wave_max(M);
    float l = 0.f;
    for (int s = lane; s < n_used; s += kWave) {
      const float* ps = part + static_cast<int64_t>(s) * (D + 2);
      l = fmaf(ps[D + 1], __expf(ps[D] - M), l);
    }
    l = wave_sum(l) + __expf(s_new - M) + (n_zero > 0 ? static_cast<float>(n_zero) * __expf(-M) : 0.f);
    const float inv = 1.f / l;
    // the first chunk's split weights exp(m_s - M) / l
    for (int s = lane; s < min(n_used, kCombineChunk); s += kWave)
      wts[s] = __expf((s == lane ? m0 : part[static_cast<int64_t>(s) * (D + 2) + D]) - M) * inv;
    if (lane == 0) {
      stat[0] = M;
      stat[1] = inv;
      stat[2] = __expf(s_new - M) / l;
    }
  }
  __syncthreads();
  const float M = stat[0], inv = stat[1];
  float o = stat[2] * vn;
  // splits in order: the prefetched ones, then the rest of each chunk
#pragma unroll
  for (int u = 0; u < kCombinePre; ++u)
    if (u < n_pre) o = fmaf(pv[u], wts[u], o);
  for (int c0 = 0; c0 < n_used; c0 += kCombineChunk) {
    const int cn = min(kCombineChunk, n_used - c0);
    if (c0 > 0) {
      __syncthreads();
      for (int s = tid; s < cn; s += kCombineThreads)
        wts[s] = __expf(part[static_cast<int64_t>(c0 + s) * (D + 2) + D] - M) * inv;
      __syncthreads();
    }
    if (tid < D) {
      for (int s0 = c0 == 0 ? n_pre : 0; s0 < cn; s0 += kCombineUnroll) {
        float v[kCombineUnroll];
#pragma unroll
        for (int u = 0; u < kCombineUnroll; ++u)
          v[u] = s0 + u < cn ? part[static_cast<int64_t>(c0 + s0 + u) * (D + 2) + tid] : 0.f;
#pragma unroll
        for (int u = 0; u < kCombineUnroll; ++u)
          if (s0 + u < cn) o = fmaf(v[u], wts[s0 + u], o);
      }
    }
  }
  if (tid < D) store_act(out, act, (static_cast<int64_t>(b) * a.n_head + h) * D + tid, o);
}

// Lanes per position in the score phase.  For head_dim 128 (bf16, 4 query
// heads per KV head) 8 lanes beat 16 (61.5 against 77.9 us at 16 x 4096
// positions, 72.5 us with 16 lanes forced to 4 waves per SIMD), although
// 16 lanes halve the query registers.
constexpr int kLanesPerPos64 = 8;
constexpr int kLanesPerPos128 = 8;

template <typename T, int D, int LP>
hipError_t launch_split_g(const AttnArgs& a, int G, int B, hipStream_t s) {
  const dim3 grid(a.n_split, a.n_head_kv, B);
  switch (G) {
    case 1: hipLaunchKernelGGL((attn_split_kernel<T, D, 1, LP>), grid, dim3(kAttnThreads), 0, s, a); break;
    case 2: hipLaunchKernelGGL((attn_split_kernel<T, D, 2, LP>), grid, dim3(kAttnThreads), 0, s, a); break;
    case 4: hipLaunchKernelGGL((attn_split_kernel<T, D, 4, LP>), grid, dim3(kAttnThreads), 0, s, a); break;
    case 8: hipLaunchKernelGGL((attn_split_kernel<T, D, 8, LP>), grid, dim3(kAttnThreads), 0, s, a); break;
    default: return hipErrorNotSupported;
  }
  return hipGetLastError();
}

template <typename T>
hipError_t launch_split_d(const AttnArgs& a, int D, int G, int B, hipStream_t s) {
  switch (D) {
    case 16: return launch_split_g<T, 16, 8>(a, G, B, s);
    case 32: return launch_split_g<T, 32, 8>(a, G, B, s);
    case 64: return launch_split_g<T, 64, kLanesPerPos64>(a, G, B, s);
    case 128: return launch_split_g<T, 128, kLanesPerPos128>(a, G, B, s);
    default: return hipErrorNotSupported;
  }
}

}  // namespace

bool attn_decode_supported(int head_dim, int group) {
  return (head_dim == 16 || head_dim == 32 || head_dim == 64 || head_dim == 128) &&
         (group == 1 || group == 2 || group == 4 || group == 8);
}

int attn_decode_splits(int max_ctx) { return (max_ctx + kSplitLen - 1) / kSplitLen; }

hipError_t launch_attn_decode(const float* q_rot, const void* k_pool, const void* v_pool, int64_t n_blocks,
                              int block_size, const int* tables, int max_blocks, const int* ctx_lens, int max_ctx,
                              const void* k_new, const void* v_new, int batch, int n_head, int n_head_kv,
                              int head_dim, int dtype, float scale, float* part, void* out, hipStream_t s,
                              const KvScatterDecode* scatter) {
  if (!attn_decode_supported(head_dim, n_head / n_head_kv) || n_head % n_head_kv) return hipErrorNotSupported;
  if (scatter && (scatter->row_bytes % 4 || !scatter->k_cache || !scatter->v_cache || !scatter->block_idx ||
                  !scatter->pos_idx))
    return hipErrorInvalidValue;
  if (batch == 0) return hipSuccess;
  AttnArgs a;
  a.q = q_rot;
  a.k_pool = k_pool;
  a.v_pool = v_pool;
  a.tables = tables;
  a.ctx_lens = ctx_lens;
  a.max_blocks = max_blocks;
  a.max_ctx = max_ctx;
  a.n_blocks = n_blocks;
  a.block_size = block_size;
  a.n_head = n_head;
  a.n_head_kv = n_head_kv;
  a.n_split = attn_decode_splits(max_ctx);
  a.scale = scale;
  a.part = part;
  const int G = n_head / n_head_kv;
  if (a.n_split > 0) {
    const hipError_t e = dtype == DT_F32 ? launch_split_d<float>(a, head_dim, G, batch, s)
                                         : launch_split_d<bf16_t>(a, head_dim, G, batch, s);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(attn_combine_kernel, dim3(n_head + (scatter ? 2 : 0), batch), dim3(kCombineThreads), 0, s, a,
                     head_dim, k_new, v_new, dtype, out, scatter ? *scatter : KvScatterDecode{});
  return hipGetLastError();
}

hipError_t launch_qkv_rope(const float* qkv, int nsplit, int64_t split_stride, const float* bq, const float* bk,
                           const float* bv, const int64_t* positions, int batch, int nq, int nkv, int head_dim,
                           double freq_base, double freq_scale, float* q_rot, void* k_new, void* v_new, int act,
                           hipStream_t s) {
  if (batch == 0) return hipSuccess;
  const int items = (nq + nkv) / 2 + nkv;
  hipLaunchKernelGGL(qkv_rope_kernel, dim3(batch, (items + 255) / 256), dim3(256), 0, s, qkv, nsplit, split_stride, bq,
                     bk, bv, positions,
                     nq, nkv, head_dim, freq_base, freq_scale, q_rot, k_new, v_new, act);
  return hipGetLastError();
}

hipError_t launch_bias_cast(const float* y, int nsplit, int64_t split_stride, const float* bias, const void* residual,
                            void* out, int64_t rows, int n, int act, hipStream_t s) {
  const int64_t total = rows * n;
  if (total == 0) return hipSuccess;
  hipLaunchKernelGGL(bias_cast_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0, s, y, nsplit,
                     split_stride, bias, residual, out, rows, n, act);
  return hipGetLastError();
}

hipError_t launch_iota(int* v, int n, int* pair, int pair0, int pair1, hipStream_t s) {
  const int blocks = n > 0 ? (n + 255) / 256 : 1;
  hipLaunchKernelGGL(iota_kernel, dim3(blocks), dim3(256), 0, s, v, n, pair, pair0, pair1);
  return hipGetLastError();
}

hipError_t launch_fill_int(int* v, int n, int value, hipStream_t s) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(fill_int_kernel, dim3((n + 255) / 256), dim3(256), 0, s, v, n, value);
  return hipGetLastError();
}

hipError_t launch_kv_gather(const void* cache, int64_t n_blocks, int block_size, int row_bytes, const int* tables,
                            int max_blocks, const int* ctx_lens, int max_ctx, int batch, void* out, hipStream_t s) {
  if (batch == 0 || max_ctx == 0 || row_bytes == 0) return hipSuccess;
  hipLaunchKernelGGL(kv_gather_kernel, dim3(max_ctx, batch), dim3(kCopyThreads), 0, s,
                     static_cast<const uint32_t*>(cache), n_blocks, block_size, row_bytes / 4, tables, max_blocks,
                     ctx_lens, max_ctx, static_cast<uint32_t*>(out));
  return hipGetLastError();
}

hipError_t launch_kv_scatter_decode(void* cache, int64_t n_blocks, int block_size, int row_bytes, const void* vals,
                                    const int* block_idx, const int* pos_idx, int batch, hipStream_t s) {
  if (batch == 0 || row_bytes == 0) return hipSuccess;
  hipLaunchKernelGGL(kv_scatter_decode_kernel, dim3(batch), dim3(kCopyThreads), 0, s, static_cast<uint32_t*>(cache),
                     n_blocks, block_size, row_bytes / 4, static_cast<const uint32_t*>(vals), block_idx, pos_idx,
                     batch);
  return hipGetLastError();
}

hipError_t launch_kv_scatter_prefill(void* cache, int64_t n_blocks, int block_size, int row_bytes, const void* vals,
                                     int seq_len, const int* tables, int max_blocks, const int* start, int batch,
                                     hipStream_t s) {
  if (batch == 0 || seq_len == 0 || row_bytes == 0) return hipSuccess;
  hipLaunchKernelGGL(kv_scatter_prefill_kernel, dim3(seq_len, batch), dim3(kCopyThreads), 0, s,
                     static_cast<uint32_t*>(cache), n_blocks, block_size, row_bytes / 4,
                     static_cast<const uint32_t*>(vals), seq_len, tables, max_blocks, start);
  return hipGetLastError();
}

}  // namespace fmoe
