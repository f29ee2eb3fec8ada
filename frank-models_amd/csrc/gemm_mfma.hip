// MFMA grouped GEMMs for gfx950: bf16 activations x (bf16 | fp8-e4m3)
// expert weights in the WF_MFMA16 packed layout, fp32 accumulation.
//
// These are mul_mat_id's per-assignment mat-vecs (components/moe/
// mul_mat_id.mlir:55-94, oracles/moe.py:37-45) with the assignments of one
// expert batched into a GEMM over the expert-sorted rows of the permutation.
// The gate and up projections share one kernel (two weight sets, the SwiGLU
// of components/activation/swiglu.mlir:37-47 in the epilogue); the down
// projection's epilogue applies the routing weight
// (moe_ffn_block.mlir:162-177) and writes each assignment's row.
//
// Operand roles are swapped with respect to "rows x columns": the MFMA's A
// operand is a 16-row weight block (16 outputs x 32 inputs), its B operand
// is 16 assignment rows x 32 inputs.  The accumulator then gives each lane 4
// consecutive output columns of one assignment row, so epilogue stores are
// 8-byte (bf16) or 16-byte (fp32) vectors.
//
// Two kernels:
//   tiled   128 rows x 256 weight rows per 256-thread block (2x2 waves, each
//           64 rows x 128 weight rows), 64 inputs per stage, LDS double
//           buffer (96 KiB), global loads of stage k+1 in flight while stage
//           k computes.  Block order is XCD-aware: consecutive tiles that
//           share weight rows run on the same XCD (same L2).
//   stream  decode-sized batches: every weight block is read exactly once
//           straight into MFMA registers (no LDS), 16 assignment rows per
//           pass, 8 input steps of loads in flight per wave (16 for the
//           one-tile bf16 gate/up kernel); one-weight projections of at most
//           16 rows stream through a ring in LDS instead (gemm_stream_lds_kernel).
//           For decode batches of at most 4 tokens the gate/up kernel can run
//           the router's top-k and grouping in its own blocks (RoutePrologue),
//           one launch fewer.
// And, for decode batches of at most 16 assignments, the down projection
// fused with the slot-ordered combine (down_combine_small_kernel).
#include "common.h"
#include "launch.h"
#include "router_topk.h"

#include <map>
#include <mutex>
#include <utility>

namespace fmoe {
namespace {

// 16 e4m3fn codes (two 32-input steps of one lane) -> two bf16x8 fragments.
__device__ __forceinline__ void f8x16_to_bf16(const u32x4_t q, u32x4_t& s0, u32x4_t& s1) {
  s0 = f8x8_to_bf16x8(q.x, q.y);
  s1 = f8x8_to_bf16x8(q.z, q.w);
}

__device__ __forceinline__ f32x4_t mfma16(const u32x4_t a, const u32x4_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// Source row of assignment p (see AMode).
__device__ __forceinline__ int64_t a_source_row(const GroupedGemmArgs& g, int p) {
  if (g.a_mode == A_GATHER_TOKEN) return g.order[p] % g.n_tokens;
  if (g.a_mode == A_GATHER_FLAT) return g.order[p];
  return p;
}

// Fused projection epilogues (one expert, rows in order, bf16 output):
// columns [n, n+4) of row p.  EPI_LINEAR rounds acc + bias to bf16 before
// adding the residual (the reference adds the rounded attention output,
// transformer_layer_moe_decode.mlir:208-221); the residual may alias out
// (each element is read and written by the same lane).  EPI_QKV_ROPE: the
// column groups of 4 lie inside one of the q | k | v parts (nq, nkv
// multiples of 4) and hold two RoPE pairs of one head (head_dim even).
// CS: the pairs' (cos, sin) come precomputed in cs0 / cs1 (rope_cos_sin of
// the same position and pair), else they are computed here.
template <int EPI, bool CS = false>
__device__ __forceinline__ void store4_proj(const GroupedGemmArgs& g, int p, int64_t n, float v0, float v1,
                                            float v2, float v3, float2 cs0 = float2{}, float2 cs1 = float2{}) {
  const ProjEpilogue& e = g.pe;
  if (EPI == EPI_LINEAR) {
    if (e.bias) v0 += e.bias[n], v1 += e.bias[n + 1], v2 += e.bias[n + 2], v3 += e.bias[n + 3];
    const int64_t i = static_cast<int64_t>(p) * g.N + n;
    u32x2_t pk{pack_bf16x2(v0, v1), pack_bf16x2(v2, v3)};
    if (e.residual) {
      const u32x2_t r = *reinterpret_cast<const u32x2_t*>(static_cast<const bf16_t*>(e.residual) + i);
      pk = u32x2_t{pack_bf16x2(__uint_as_float(pk[0] << 16) + __uint_as_float(r[0] << 16),
                               __uint_as_float(pk[0] & 0xFFFF0000u) + __uint_as_float(r[0] & 0xFFFF0000u)),
                   pack_bf16x2(__uint_as_float(pk[1] << 16) + __uint_as_float(r[1] << 16),
                               __uint_as_float(pk[1] & 0xFFFF0000u) + __uint_as_float(r[1] & 0xFFFF0000u))};
    }
    *reinterpret_cast<u32x2_t*>(static_cast<bf16_t*>(e.out) + i) = pk;
  } else {
    const int nq = e.nq, nkv = e.nkv;
    if (n >= nq + nkv) {  // v: bias only
      const int64_t c = n - nq - nkv;
      if (e.bias_v) v0 += e.bias_v[c], v1 += e.bias_v[c + 1], v2 += e.bias_v[c + 2], v3 += e.bias_v[c + 3];
      *reinterpret_cast<u32x2_t*>(static_cast<bf16_t*>(e.v_out) + static_cast<int64_t>(p) * nkv + c) =
          u32x2_t{pack_bf16x2(v0, v1), pack_bf16x2(v2, v3)};
      return;
    }
    const bool is_q = n < nq;
    const int64_t c = is_q ? n : n - nq;
    const float* b = is_q ? e.bias : e.bias_k;
    if (b) v0 += b[c], v1 += b[c + 1], v2 += b[c + 2], v3 += b[c + 3];
    float y0, y1, y2, y3;
    if (CS) {
      rope_apply(v0, v1, cs0, y0, y1);
      rope_apply(v2, v3, cs1, y2, y3);
    } else {
      const int64_t pos = e.positions[p];
      const int i0 = static_cast<int>(c % e.head_dim) / 2;
      rope_pair(v0, v1, pos, i0, e.head_dim, e.freq_base, e.freq_scale, y0, y1);
      rope_pair(v2, v3, pos, i0 + 1, e.head_dim, e.freq_base, e.freq_scale, y2, y3);
    }
    if (is_q)
      *reinterpret_cast<float4*>(e.q_out + static_cast<int64_t>(p) * nq + c) = float4{y0, y1, y2, y3};
    else
      *reinterpret_cast<u32x2_t*>(static_cast<bf16_t*>(e.k_out) + static_cast<int64_t>(p) * nkv + c) =
          u32x2_t{pack_bf16x2(y0, y1), pack_bf16x2(y2, y3)};
  }
}

// Writes 4 consecutive columns [n, n+4) of row p's result.
template <int EPI>
__device__ __forceinline__ void store4(const GroupedGemmArgs& g, int p, int64_t n, float v0, float v1,
                                       float v2, float v3) {
  if (EPI == EPI_LINEAR || EPI == EPI_QKV_ROPE) {
    store4_proj<EPI>(g, p, n, v0, v1, v2, v3);
    return;
  }
  if (EPI == EPI_SWIGLU || g.out_dtype == DT_BF16) {
    int64_t row = p;
    if (EPI != EPI_SWIGLU && g.order) row = g.order[p];
    if (EPI == EPI_SCATTER_WEIGHTED) {
      const float w = g.route_w[row];
      v0 *= w, v1 *= w, v2 *= w, v3 *= w;
    }
    u32x2_t pk{pack_bf16x2(v0, v1), pack_bf16x2(v2, v3)};
    *reinterpret_cast<u32x2_t*>(static_cast<bf16_t*>(g.out) + row * g.ldo + n) = pk;
  } else {
    const int64_t row = g.order ? g.order[p] : p;
    if (EPI == EPI_SCATTER_WEIGHTED) {
      const float w = g.route_w[row];
      v0 *= w, v1 *= w, v2 *= w, v3 *= w;
    }
    *reinterpret_cast<float4*>(static_cast<float*>(g.out) + row * g.ldo + n) = float4{v0, v1, v2, v3};
  }
}

// ======================================================================= tiled
constexpr int kThreads = 256;
constexpr int kBM = 128;  // assignment rows per tile
constexpr int kBK = 64;   // inputs per stage
constexpr int kGroupN = 4;  // column tiles swept together per row-tile sweep

template <int NSETS>
struct Tiled {
  static constexpr int kBNSet = NSETS == 2 ? 128 : 256;  // weight rows per set per tile
  static constexpr int kWaveN = kBNSet / 2;              // per wave per set
  static constexpr int kNSub = kWaveN / 16;              // 16-row weight blocks per wave per set
  static constexpr int kMSub = 4;                        // 64 rows per wave
  static constexpr int kNBStage = NSETS * kBNSet / 16;   // weight row blocks per stage (16)
  static constexpr int kABytes = kBM * kBK * 2;          // 16 KiB
  static constexpr int kBBytes = kNBStage * 2 * 1024;    // 32 KiB (two 32-input blocks per row block)
};

// Logical tile of a hardware block id: hardware dispatches block b to XCD
// b % 8; logical ids are handed out so that each XCD gets a contiguous range,
// and within it kGroupN column tiles are swept across all row tiles
// (weight rows of a column tile are then re-read from the XCD's L2 by the
// row tiles of the same expert running beside each other).
__device__ __forceinline__ bool logical_tile(int n_row_tiles, int n_col_tiles, int* row_tile, int* col_tile) {
  const int total = n_row_tiles * n_col_tiles;
  const int per_xcd = (total + 7) / 8;
  const int b = blockIdx.x;
  const int logical = (b % 8) * per_xcd + b / 8;
  if (logical >= total) return false;
  const int group_span = kGroupN * n_row_tiles;
  const int group = logical / group_span;
  const int within = logical - group * group_span;
  const int cols_in_group = min(kGroupN, n_col_tiles - group * kGroupN);
  *row_tile = within / cols_in_group;
  *col_tile = group * kGroupN + within % cols_in_group;
  return true;
}

template <int EPI, int NSETS, bool F8>
__global__ __launch_bounds__(kThreads, 1) void gemm_tiled_kernel(GroupedGemmArgs g, int n_row_tiles,
                                                                  int n_col_tiles) {
  using C = Tiled<NSETS>;
  extern __shared__ __attribute__((aligned(1024))) unsigned char lds[];
  unsigned char* a_s = lds;                   // [2][kBM][kBK] bf16, 16-byte chunks XOR-swizzled
  unsigned char* b_s = lds + 2 * C::kABytes;  // [2][kNBStage][2][64 lanes][16 B]

  int row_tile, col_tile;
  if (!logical_tile(n_row_tiles, n_col_tiles, &row_tile, &col_tile)) return;
  TileInfo ti;
  if (!find_tile(g.offsets, g.n_expert, kBM, row_tile, &ti)) return;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1;  // rows wm*64 .. +64
  const int wn = wave & 1;   // weight rows wn*kWaveN .. per set
  const int64_t N = g.N, K = g.K;
  const int64_t n0 = static_cast<int64_t>(col_tile) * C::kBNSet;
  const int64_t nblocks = N / 16;  // row blocks per expert
  const int KT = static_cast<int>(K / kBK);

  // ---- A rows this thread stages: rows (tid >> 3) + 32 j, 16-byte chunk tid & 7.
  const int a_chunk = tid & 7;
  const bf16_t* a_src[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = (tid >> 3) + 32 * j;
    const int p = ti.row0 + (r < ti.rows ? r : 0);
    a_src[j] = static_cast<const bf16_t*>(g.a) + a_source_row(g, p) * g.lda + a_chunk * 8;
  }

  // ---- weight blocks this thread stages, per weight set.
  // bf16: 2 input blocks per row block per stage; chunk c = tid + 256 j covers
  //   stage block c >> 6 = 2 * (row block) + input block, lane c & 63, so
  //   thread tid stages row blocks (tid >> 7) + 2 jj of each set (jj < kRB / 2)
  //   at input block (tid >> 6) & 1.
  // fp8: 1 packed block (64 inputs) per row block per stage; thread tid stages
  //   row blocks (tid >> 6) + 4 jj of each set (jj < kRB / 4).
  constexpr int kRB = C::kBNSet / 16;               // row blocks per set per stage
  constexpr int kJ = F8 ? kRB / 4 : kRB / 2;        // loads per set per stage
  const int64_t kblocks = F8 ? K / 64 : K / 32;     // packed blocks per row block
  const int rb_first = F8 ? (tid >> 6) : (tid >> 7);
  const int rb_step = F8 ? 4 : 2;
  const int kb_sel = F8 ? 0 : ((tid >> 6) & 1);
  const int64_t b_stride = static_cast<int64_t>(rb_step) * kblocks * 1024;  // bytes between jj
  const unsigned char* b_base[NSETS];
#pragma unroll
  for (int set = 0; set < NSETS; ++set) {
    const unsigned char* w = static_cast<const unsigned char*>(set == 0 ? g.w0 : g.w1);
    b_base[set] = w + ((static_cast<int64_t>(ti.expert) * nblocks + n0 / 16 + rb_first) * kblocks + kb_sel) * 1024 +
                  lane * 16;
  }
  // Row blocks past N (partial last column tile) are staged as zeros.
  const int64_t rb_limit = nblocks - n0 / 16 - rb_first;  // jj*rb_step < rb_limit is in range

  u32x4_t a_reg[4];
  u32x4_t b_reg[NSETS * kJ];

  auto load_stage = [&](int kt) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < 4; ++j) a_reg[j] = *reinterpret_cast<const u32x4_t*>(a_src[j] + kt * kBK);
    const int64_t adv = static_cast<int64_t>(kt) * (F8 ? 1024 : 2048);
#pragma unroll
    for (int set = 0; set < NSETS; ++set)
#pragma unroll
      for (int jj = 0; jj < kJ; ++jj)
        b_reg[set * kJ + jj] = (jj * rb_step < rb_limit)
                                   ? *reinterpret_cast<const u32x4_t*>(b_base[set] + jj * b_stride + adv)
                                   : u32x4_t{0u, 0u, 0u, 0u};
  };
  auto store_stage = [&](int st) __attribute__((always_inline)) {
    unsigned char* as = a_s + st * C::kABytes;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = (tid >> 3) + 32 * j;
      *reinterpret_cast<u32x4_t*>(as + r * 128 + ((a_chunk ^ (r & 7)) << 4)) = a_reg[j];
    }
    unsigned char* bs = b_s + st * C::kBBytes;
#pragma unroll
    for (int set = 0; set < NSETS; ++set) {
#pragma unroll
      for (int jj = 0; jj < kJ; ++jj) {
        const int rb = set * kRB + rb_first + jj * rb_step;  // stage row block
        if (F8) {
          u32x4_t s0, s1;
          f8x16_to_bf16(b_reg[set * kJ + jj], s0, s1);
          *reinterpret_cast<u32x4_t*>(bs + (rb * 2 + 0) * 1024 + lane * 16) = s0;
          *reinterpret_cast<u32x4_t*>(bs + (rb * 2 + 1) * 1024 + lane * 16) = s1;
        } else {
          *reinterpret_cast<u32x4_t*>(bs + (rb * 2 + kb_sel) * 1024 + lane * 16) = b_reg[set * kJ + jj];
        }
      }
    }
  };

  f32x4_t acc[NSETS][C::kNSub][C::kMSub];
#pragma unroll
  for (int s = 0; s < NSETS; ++s)
#pragma unroll
    for (int i = 0; i < C::kNSub; ++i)
#pragma unroll
      for (int m = 0; m < C::kMSub; ++m) acc[s][i][m] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  load_stage(0);
  store_stage(0);
  __syncthreads();

  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    // Prefetch the next stage (the last iteration re-reads the final stage
    // into the idle buffer: branch-free, so the staging registers stay in
    // registers).
    load_stage(kt + 1 < KT ? kt + 1 : kt);
    const unsigned char* as = a_s + cur * C::kABytes;
    const unsigned char* bs = b_s + cur * C::kBBytes;
#pragma unroll
    for (int s = 0; s < 2; ++s) {  // two 32-input steps per stage
      u32x4_t tok[C::kMSub];
#pragma unroll
      for (int m = 0; m < C::kMSub; ++m) {
        const int r = wm * 64 + m * 16 + (lane & 15);
        const int ch = s * 4 + (lane >> 4);
        tok[m] = *reinterpret_cast<const u32x4_t*>(as + r * 128 + ((ch ^ (r & 7)) << 4));
      }
#pragma unroll
      for (int set = 0; set < NSETS; ++set) {
#pragma unroll
        for (int i = 0; i < C::kNSub; ++i) {
          const int rb = set * (C::kBNSet / 16) + wn * C::kNSub + i;
          const u32x4_t w = *reinterpret_cast<const u32x4_t*>(bs + (rb * 2 + s) * 1024 + lane * 16);
#pragma unroll
          for (int m = 0; m < C::kMSub; ++m) acc[set][i][m] = mfma16(w, tok[m], acc[set][i][m]);
        }
      }
    }
    store_stage(cur ^ 1);
    __syncthreads();
  }

  // ---- epilogue: lane holds row (lane & 15) of each 16-row group, columns 4*(lane>>4) .. +4.
  const int64_t e = ti.expert;
#pragma unroll
  for (int i = 0; i < C::kNSub; ++i) {
    const int64_t n = n0 + wn * C::kWaveN + i * 16 + 4 * (lane >> 4);
    if (n >= N) continue;
    float4 sc0{1.f, 1.f, 1.f, 1.f}, sc1{1.f, 1.f, 1.f, 1.f};
    if (F8) {
      sc0 = *reinterpret_cast<const float4*>(g.s0 + e * N + n);
      if (NSETS == 2) sc1 = *reinterpret_cast<const float4*>(g.s1 + e * N + n);
    }
#pragma unroll
    for (int m = 0; m < C::kMSub; ++m) {
      const int r = wm * 64 + m * 16 + (lane & 15);
      if (r >= ti.rows) continue;
      const int p = ti.row0 + r;
      const f32x4_t a0 = acc[0][i][m];
      if (EPI == EPI_SWIGLU) {
        const f32x4_t a1 = acc[NSETS - 1][i][m];
        store4<EPI>(g, p, n, silu_mul(a0[0] * sc0.x, a1[0] * sc1.x), silu_mul(a0[1] * sc0.y, a1[1] * sc1.y),
                    silu_mul(a0[2] * sc0.z, a1[2] * sc1.z), silu_mul(a0[3] * sc0.w, a1[3] * sc1.w));
      } else {
        store4<EPI>(g, p, n, a0[0] * sc0.x, a0[1] * sc0.y, a0[2] * sc0.z, a0[3] * sc0.w);
      }
    }
  }
}

// ======================================================================= stream
// Weight blocks are read exactly once per launch (a pass covers up to 64 of
// an expert's rows), so they are loaded non-temporally: they do not push the
// token rows and outputs out of the caches.
__device__ __forceinline__ u32x4_t stream_load(const u32x4_t* p) { return __builtin_nontemporal_load(p); }

constexpr int kStreamRows = 16;     // weight rows per set per block
constexpr int kStreamUnroll = 8;    // 32-input steps per iteration
constexpr int kStreamWaves = kThreads / kWave;

// Decode-sized grouped GEMM: block = (expert, 16 weight rows per set); its
// 4 waves split the input axis in four and their partial sums are added in
// wave order through LDS, so even a handful of active experts keeps many
// waves streaming.  Each wave streams its weight blocks from HBM straight
// into MFMA registers (U 1 KiB blocks per set in flight, below) and
// applies each fragment to up to kStreamTiles 16-row tiles of the expert's
// token rows, so an expert's weights are read once for up to
// 16 * kStreamTiles rows.  An expert has at most n_tokens rows (top-k picks
// distinct experts), so the launcher sizes kStreamTiles from n_tokens and
// decode batches keep the one-tile register footprint.
// Waves per SIMD the register allocation must allow: without a target the
// multi-tile gate/up kernels put their accumulators in AGPRs and fit only 2
// waves per SIMD (measured: 3 is 2-5% faster at 64 tokens); 1-set kernels
// keep the occupancy they reach anyway (6 for one tile spills).
// The RoPE epilogue's double-precision angles need more registers; its
// projection has one or two blocks per CU anyway.
// U: 32-input steps per trip (kStreamUnroll, or 16 for the one-tile bf16
// gate/up kernel, whose wave then loads its whole share of a 2048-input axis
// in one trip at 2 waves per SIMD).
template <int EPI, int NSETS, int kStreamTiles, int U>
constexpr int stream_waves_per_eu() {
  return EPI == EPI_QKV_ROPE ? 2 : U > kStreamUnroll ? 2 : NSETS == 2 ? 3 : kStreamTiles == 1 ? 5 : 4;
}

// RNV > 0 (one-tile gate/up kernels of decode batches of at most 4 tokens,
// GroupedGemmArgs::rp): the block computes the routing itself from the
// router's split partial logits.  Wave 0 runs the router's top-k
// (wave_topk4_splits, RNV experts per row lane), marks the selected experts
// in LDS, and block row a = blockIdx.x / col_tiles takes the a-th selected
// expert in ascending order (found with wave ballots), with its rows in the
// stable order: the flat ids f of that expert ascending, row r reading token
// f % n_tokens, as the permutation would order them.  Blocks past the
// selected experts exit.  Block 0 also stores ids, weights, order, offsets
// and the invalid-id count for the down projection and the caller.
template <int EPI, int NSETS, bool F8, int kStreamTiles, int U = kStreamUnroll, int RNV = 0>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(stream_waves_per_eu<EPI, NSETS, kStreamTiles, U>())))
void gemm_stream_kernel(GroupedGemmArgs g, int col_tiles) {
  static_assert(RNV == 0 || (EPI == EPI_SWIGLU && kStreamTiles == 1), "routing in the one-tile gate/up kernel only");
  __shared__ f32x4_t partial[kStreamWaves - 1][kStreamTiles][NSETS][kWave];
  __shared__ float r_lg[RNV > 0 ? 4 * (16 * RNV + 1) : 1];
  __shared__ int r_idl[RNV > 0 ? kWave : 1];
  __shared__ int r_flag[RNV > 0 ? 256 : 1];
  __shared__ int r_tok[RNV > 0 ? 16 : 1];
  __shared__ int r_meta[RNV > 0 ? 3 : 1];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int ct = blockIdx.x - (blockIdx.x / col_tiles) * col_tiles;
  int e, row_begin, count;
  if constexpr (RNV > 0) {
    const RoutePrologue& rp = g.rp;
    const int T = g.n_tokens, E = g.n_expert, n = rp.k * T;
    const bool pub = blockIdx.x == 0;
    if (wave == 0)
      wave_topk4_splits<RNV>(rp.part, rp.n_split, T, E, rp.k, rp.normalize != 0, r_lg, pub ? rp.ids : nullptr,
                             pub ? rp.weights : nullptr, r_idl);
    for (int i = tid; i < E; i += kThreads) r_flag[i] = 0;
    __syncthreads();
    if (wave == 0) {
      // ids outside [0, E) (the top-k's sentinel when probabilities are NaN)
      // mark nothing and take no rows
      if (lane < n && r_idl[lane] >= 0 && r_idl[lane] < E) r_flag[r_idl[lane]] = 1;
      if (pub) {
        wave_permute(r_idl, n, E, rp.order, rp.offsets);
        if (lane == 0) rp.err_count[0] = 0;
      }
    }
    __syncthreads();
    if (wave == 0) {
      const int a = blockIdx.x / col_tiles;
      const uint64_t lt = lane == 0 ? 0ull : (~0ull >> (kWave - lane));
      int sel = -1, below = 0;
      for (int c0 = 0; c0 < E; c0 += kWave) {
        const int c = c0 + lane;
        const bool f = c < E && r_flag[c] != 0;
        const uint64_t m = __ballot(f);
        const uint64_t hit = __ballot(f && below + __popcll(m & lt) == a);
        if (hit && sel < 0) sel = c0 + __builtin_ctzll(hit);
        below += __popcll(m);
      }
      const int fe = lane < n ? r_idl[lane] : 0x7FFFFFFF;
      const uint64_t mine = __ballot(lane < n && fe == sel);
      const uint64_t lower = __ballot(lane < n && fe < sel);
      // at most n_tokens rows (distinct experts per token), within the one tile
      const int rank = __popcll(mine & lt);
      if (lane < n && fe == sel && rank < 16) r_tok[rank] = lane % T;
      if (lane == 0) {
        r_meta[0] = sel;
        r_meta[1] = __popcll(lower);
        r_meta[2] = sel >= 0 ? min(__popcll(mine), 16) : 0;
      }
    }
    __syncthreads();
    e = r_meta[0];
    row_begin = r_meta[1];
    count = r_meta[2];
  } else {
    e = blockIdx.x / col_tiles;
    row_begin = g.offsets ? g.offsets[e] : 0;
    count = g.offsets ? g.offsets[e + 1] - row_begin : g.n_assign;
  }
  if (count == 0) return;  // block-uniform
  const int64_t N = g.N, K = g.K;
  const int64_t n_base = static_cast<int64_t>(ct) * kStreamRows;
  const int64_t nblocks = N / 16;
  const int64_t nb = n_base / 16;
  const int64_t kblocks = F8 ? K / 64 : K / 32;
  // This wave's share of the input axis, in 32-input steps (whole fp8
  // blocks of two steps for fp8 weights).
  // With a K split (gridDim.y > 1, one-set fp32 scatter only) block row
  // blockIdx.y takes its share first and writes partial sums split_stride
  // elements apart.
  const int ksteps = static_cast<int>(K / 32);
  const int unit = F8 ? 2 : 1;
  const int units = ksteps / unit;
  const int kz = blockIdx.y, nz = gridDim.y;
  const int u0 = kz * units / nz, u1 = (kz + 1) * units / nz;
  const int ks_begin = (u0 + wave * (u1 - u0) / kStreamWaves) * unit;
  const int ks_end = (u0 + (wave + 1) * (u1 - u0) / kStreamWaves) * unit;
  if (kz > 0) g.out = static_cast<float*>(g.out) + kz * g.split_stride;
  const unsigned char* wsrc[NSETS];
#pragma unroll
  for (int s = 0; s < NSETS; ++s) {
    const unsigned char* base = static_cast<const unsigned char*>(s == 0 ? g.w0 : g.w1);
    wsrc[s] = base + ((static_cast<int64_t>(e) * nblocks + nb) * kblocks) * 1024 + lane * 16;
  }
  const int kq = (lane >> 4) * 8;  // this lane's 8 inputs within a 32-input step
  const u32x4_t zero{0u, 0u, 0u, 0u};

  for (int m0 = 0; m0 < count; m0 += 16 * kStreamTiles) {
    const int nt = min(kStreamTiles, (count - m0 + 15) / 16);  // block-uniform
    const bf16_t* arow[kStreamTiles];
    bool r_ok[kStreamTiles];
#pragma unroll
    for (int mt = 0; mt < kStreamTiles; ++mt) {
      const int r = m0 + mt * 16 + (lane & 15);
      r_ok[mt] = r < count;
      const int64_t src = RNV > 0 ? r_tok[r_ok[mt] ? r : 0] : a_source_row(g, row_begin + (r_ok[mt] ? r : 0));
      arow[mt] = static_cast<const bf16_t*>(g.a) + src * g.lda + kq;
    }
    f32x4_t acc[kStreamTiles][NSETS];
#pragma unroll
    for (int mt = 0; mt < kStreamTiles; ++mt)
#pragma unroll
      for (int s = 0; s < NSETS; ++s) acc[mt][s] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    // U steps per trip, all loads first; a short last trip is
    // predicated per step (wave-uniform), so it keeps its loads in flight too.
    for (int ks = ks_begin; ks < ks_end; ks += U) {
      u32x4_t wv[NSETS][U];
#pragma unroll
      for (int s = 0; s < NSETS; ++s) {
        if (F8) {
          // all loads, then all conversions (a conversion waits for its load)
          u32x4_t q[U / 2];
#pragma unroll
          for (int u = 0; u < U; u += 2)
            q[u / 2] = ks + u < ks_end ? stream_load(reinterpret_cast<const u32x4_t*>(
                                             wsrc[s] + static_cast<int64_t>((ks + u) / 2) * 1024))
                                       : zero;
#pragma unroll
          for (int u = 0; u < U; u += 2) f8x16_to_bf16(q[u / 2], wv[s][u], wv[s][u + 1]);
        } else {
#pragma unroll
          for (int u = 0; u < U; ++u)
            wv[s][u] = ks + u < ks_end
                           ? stream_load(reinterpret_cast<const u32x4_t*>(wsrc[s] + static_cast<int64_t>(ks + u) * 1024))
                           : zero;
        }
      }
#pragma unroll
      for (int mt = 0; mt < kStreamTiles; ++mt) {
        if (mt < nt) {
          u32x4_t tok[U];
#pragma unroll
          for (int u = 0; u < U; ++u)
            tok[u] = (r_ok[mt] && ks + u < ks_end) ? *reinterpret_cast<const u32x4_t*>(arow[mt] + (ks + u) * 32) : zero;
#pragma unroll
          for (int u = 0; u < U; ++u)
            if (ks + u < ks_end)
#pragma unroll
              for (int s = 0; s < NSETS; ++s) acc[mt][s] = mfma16(wv[s][u], tok[u], acc[mt][s]);
        }
      }
    }

    // Partial sums of waves 1..3 -> LDS; wave 0 adds them in wave order.
    if (wave > 0) {
#pragma unroll
      for (int mt = 0; mt < kStreamTiles; ++mt)
#pragma unroll
        for (int s = 0; s < NSETS; ++s)
          if (mt < nt) partial[wave - 1][mt][s][lane] = acc[mt][s];
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
      for (int w = 1; w < kStreamWaves; ++w)
#pragma unroll
        for (int mt = 0; mt < kStreamTiles; ++mt)
#pragma unroll
          for (int s = 0; s < NSETS; ++s)
            if (mt < nt) acc[mt][s] += partial[w - 1][mt][s][lane];
      const int64_t n = n_base + 4 * (lane >> 4);
      float4 sc0{1.f, 1.f, 1.f, 1.f}, sc1{1.f, 1.f, 1.f, 1.f};
      if (F8) {
        sc0 = *reinterpret_cast<const float4*>(g.s0 + static_cast<int64_t>(e) * N + n);
        if (NSETS == 2) sc1 = *reinterpret_cast<const float4*>(g.s1 + static_cast<int64_t>(e) * N + n);
      }
#pragma unroll
      for (int mt = 0; mt < kStreamTiles; ++mt) {
        if (mt < nt && r_ok[mt]) {
          const int p = row_begin + m0 + mt * 16 + (lane & 15);
          const f32x4_t a0 = acc[mt][0];
          if (EPI == EPI_SWIGLU) {
            const f32x4_t a1 = acc[mt][NSETS - 1];
            store4<EPI>(g, p, n, silu_mul(a0[0] * sc0.x, a1[0] * sc1.x), silu_mul(a0[1] * sc0.y, a1[1] * sc1.y),
                        silu_mul(a0[2] * sc0.z, a1[2] * sc1.z), silu_mul(a0[3] * sc0.w, a1[3] * sc1.w));
          } else {
            store4<EPI>(g, p, n, a0[0] * sc0.x, a0[1] * sc0.y, a0[2] * sc0.z, a0[3] * sc0.w);
          }
        }
      }
    }
    __syncthreads();  // partial[] is rewritten by the next pass
  }
}

// ===================================================== stream through LDS
// One-weight projections of at most 16 rows (the decode attention's Q/K/V
// and output projections): a column slab per block and four K quarters per
// wave, as gemm_stream_kernel, but each wave keeps D input steps of loads in
// flight by loading them straight into a ring of its own in LDS
// (global_load_lds, no staging registers): per step the 1 KiB weight block
// and the 1 KiB token fragment block, in the lane order the MFMA reads them.
// gemm_stream_kernel holds one trip of 8 steps per wave in registers and
// waits for it before loading the next, so a slab of a 4096-input weight
// (4 trips per wave) costs four round trips to HBM; here the wave waits only
// for the oldest step.  The arithmetic is gemm_stream_kernel's (the same
// quarters, MFMA chains, wave-order sum and epilogue), so the results are
// bit for bit the same.  Token rows past the batch load row 0 (their output
// rows are not stored).
// Cache policy of the weight loads: non-temporal (each weight byte is read
// once per launch), as gemm_stream_kernel's, so the weights do not push the
// token rows and the next kernel's data out of the caches.
constexpr int kNonTemporal = 2;
// The Q/K/V kernel's block has two more waves: they compute the RoPE
// (cos, sin) of each (row, pair) of the block's 16 columns into LDS while
// the four streaming waves wait on their loads, so the epilogue only
// rotates.  The angles are rope_cos_sin's, so the results are unchanged.
constexpr int kRopeWaves = 2;
constexpr int kRopeItems = kStreamRows * kStreamRows / 2;  // rows x pairs
static_assert(kRopeItems == kRopeWaves * kWave, "one (row, pair) per angle lane");

template <int EPI>
constexpr int stream_lds_threads() {
  return kThreads + (EPI == EPI_QKV_ROPE ? kRopeWaves * kWave : 0);
}

template <int D, int EPI>
constexpr int stream_lds_bytes() {
  return kStreamWaves * D * 2048 + (kStreamWaves - 1) * kWave * 16 + (EPI == EPI_QKV_ROPE ? kRopeItems * 8 : 0);
}

template <int EPI, int D>
__global__ __launch_bounds__(kThreads + kRopeWaves * kWave) void gemm_stream_lds_kernel(GroupedGemmArgs g) {
  static_assert(EPI == EPI_LINEAR || EPI == EPI_QKV_ROPE, "fused one-weight projection epilogues");
  static_assert((D & (D - 1)) == 0 && 2 * D <= 62, "ring slots: a power of two, loads within the vmcnt range");
  extern __shared__ __attribute__((aligned(1024))) unsigned char lds[];
  f32x4_t* partial = reinterpret_cast<f32x4_t*>(lds + kStreamWaves * D * 2048);  // [kStreamWaves - 1][kWave]
  float2* rope_cs = reinterpret_cast<float2*>(lds + kStreamWaves * D * 2048 + (kStreamWaves - 1) * kWave * 16);
  const int ct = blockIdx.x;
  const int count = g.n_assign;  // <= 16 rows, in order (one expert, no grouping arrays)
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar loop control
  const int64_t N = g.N;
  const int r = lane & 15;
  f32x4_t acc{0.f, 0.f, 0.f, 0.f};
  if (EPI == EPI_QKV_ROPE && wave >= kStreamWaves) {
    // item = row * 8 + pair: columns 2 pair, 2 pair + 1 of the block, in the
    // q or k part (v columns take no rotation)
    const ProjEpilogue& e = g.pe;
    const int item = tid - kThreads;
    const int rr = item >> 3;
    const int64_t n = static_cast<int64_t>(ct) * kStreamRows + 2 * (item & 7);
    if (rr < count && n < static_cast<int64_t>(e.nq) + e.nkv) {
      const int64_t c = n < e.nq ? n : n - e.nq;
      rope_cs[item] = rope_cos_sin(e.positions[rr], static_cast<int>(c % e.head_dim) / 2, e.head_dim, e.freq_base,
                                   e.freq_scale);
    }
  } else {
    const int ksteps = static_cast<int>(g.K / 32);
    const int ks_begin = wave * ksteps / kStreamWaves;
    const int n = (wave + 1) * ksteps / kStreamWaves - ks_begin;
    const unsigned char* wsrc =
        static_cast<const unsigned char*>(g.w0) + (static_cast<int64_t>(ct) * ksteps + ks_begin) * 1024 + lane * 16;
    const unsigned char* tsrc = reinterpret_cast<const unsigned char*>(
        static_cast<const bf16_t*>(g.a) + static_cast<int64_t>(r < count ? r : 0) * g.lda + (lane >> 4) * 8 +
        static_cast<int64_t>(ks_begin) * 32);
    unsigned char* ring = lds + wave * D * 2048;
    auto issue = [&](int i) __attribute__((always_inline)) {
      unsigned char* slot = ring + (i & (D - 1)) * 2048;
      __builtin_amdgcn_global_load_lds(wsrc + static_cast<int64_t>(i) * 1024, slot, 16, 0, kNonTemporal);
      __builtin_amdgcn_global_load_lds(tsrc + static_cast<int64_t>(i) * 64, slot + 1024, 16, 0, 0);
    };
    const int pre = n < D ? n : D;
    for (int i = 0; i < pre; ++i) issue(i);
    for (int i = 0; i < n; ++i) {
      // step i's two loads are done once at most 2 (D - 1) younger ones are
      // in flight (loads complete in order); near the end, all of them
      if (i + D <= n)
        __builtin_amdgcn_s_waitcnt(wait_vm(2 * D - 2, false));
      else
        __builtin_amdgcn_s_waitcnt(wait_vm(0, false));
      __builtin_amdgcn_sched_barrier(0);
      asm volatile("" ::: "memory");
      const unsigned char* slot = ring + (i & (D - 1)) * 2048;
      const u32x4_t w = *reinterpret_cast<const u32x4_t*>(slot + lane * 16);
      const u32x4_t t = *reinterpret_cast<const u32x4_t*>(slot + 1024 + lane * 16);
      acc = mfma16(w, t, acc);
      // the slot is refilled only after its reads have returned (the MFMA
      // above waits for them)
      __builtin_amdgcn_sched_barrier(0);
      if (i + D < n) issue(i + D);
    }
  }

  // Partial sums of waves 1..3 -> LDS; wave 0 adds them in wave order.
  if (wave > 0 && wave < kStreamWaves) partial[(wave - 1) * kWave + lane] = acc;
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int w = 1; w < kStreamWaves; ++w) acc += partial[(w - 1) * kWave + lane];
    const int64_t col = static_cast<int64_t>(ct) * kStreamRows + 4 * (lane >> 4);
    if (r < count && col < N) {
      if (EPI == EPI_QKV_ROPE) {
        const int pr = r * 8 + 2 * (lane >> 4);  // the lane's two pairs
        store4_proj<EPI, true>(g, r, col, acc[0], acc[1], acc[2], acc[3], rope_cs[pr], rope_cs[pr + 1]);
      } else {
        store4<EPI>(g, r, col, acc[0], acc[1], acc[2], acc[3]);
      }
    }
  }
}

// ============================================================ down + combine
// Decode batches whose n_assign = n_tokens * k assignments fit one 16-row
// MFMA tile (n_assign <= 16): the down projection and the slot-ordered
// combine (moe_ffn_block.mlir:158-206) in one launch.  Block = 16 output
// columns; its 16 waves take (active expert, K quarter) items, each the
// arithmetic of one wave of gemm_stream_kernel (same quarters, same steps,
// same MFMA sequence: the B tile holds all assignment rows, those of other
// experts zeroed).  Then, through LDS, each assignment's quarters are added
// in order, scaled and weighted as gemm_stream_kernel's epilogue does, and
// the slots of each token are summed in slot order (plus the residual) as
// combine_kernel does, with one rounding to bf16: the result is the
// two-launch path's, bit for bit.  Every weight byte of the active experts'
// 16-row slabs is read once; a block streams n_active slabs, so the
// launcher takes this path only while that stays small.
constexpr int kFcThreads = 1024;
constexpr int kFcWaves = kFcThreads / kWave;
constexpr int kFcRows = 16;                 // assignment rows (one MFMA tile)
constexpr int kFcItems = 4 * kFcRows;       // (active expert, K quarter) items, at most
constexpr int kFcUnroll = 12;               // 32-input steps per trip (a K quarter of 1408 inputs in one)
// Weight bytes one block may stream, for a grid that fills the 256 CUs; a
// smaller grid (n_embd / 16 blocks) takes proportionally less.  Measured
// (whole block calls, cold, medians against the two launches): C2 T=1 127
// against 136 us (917 KiB per block, 256 blocks), C5 T=1 80.2 against 84.8
// us (458 KiB, 256), C3 T=1 38.8 against 41.1 us (196 KiB, 128), C4 T=1
// 39.9 against 41.2 us (270 KiB, 128), C3 T=2 44.3 against 45.0 us (393 KiB,
// 128); C4 T=2 (540 KiB, 128) 51.7 against 49.3 us, hence the scaling.
constexpr int64_t kFcMaxBlockBytes = 1 << 20;

template <bool F8>
__global__ __launch_bounds__(kFcThreads) void down_combine_small_kernel(GroupedGemmArgs g, const bf16_t* residual,
                                                                        bf16_t* out, int n_tokens, int k) {
  __shared__ f32x4_t part[kFcItems][kWave];
  __shared__ float ys[kFcRows][kStreamRows];  // weighted y of flat assignment f, the block's columns
  __shared__ int act_e[kFcRows], act_off[kFcRows], act_cnt[kFcRows], row_act[kFcRows], n_act_s;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int64_t N = g.N, K = g.K;
  const int64_t nblocks = N / 16, nb = blockIdx.x;
  const int64_t n_base = nb * kStreamRows;

  // Active experts in ascending order (wave ballots over the offsets); rows
  // of no expert (none, for valid ids) keep row_act = -1.
  if (tid < kFcRows) {
    row_act[tid] = -1;
    for (int c = 0; c < kStreamRows; ++c) ys[tid][c] = 0.f;
  }
  if (wave == 0) {
    const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (kWave - lane));
    int n = 0;
    for (int e0 = 0; e0 < g.n_expert; e0 += kWave) {
      const int e = e0 + lane;
      const int o = e < g.n_expert ? g.offsets[e] : 0;
      const int c = e < g.n_expert ? g.offsets[e + 1] - o : 0;
      const bool has = c > 0 && o >= 0 && o + c <= g.n_assign;
      const uint64_t m = __ballot(has);
      const int idx = n + __popcll(m & lt_mask);
      if (has && idx < kFcRows) {
        act_e[idx] = e;
        act_off[idx] = o;
        act_cnt[idx] = c;
      }
      n += __popcll(m);
    }
    if (lane == 0) n_act_s = min(n, kFcRows);
  }
  __syncthreads();
  const int n_act = n_act_s;
  if (tid < n_act)
    for (int r = act_off[tid]; r < act_off[tid] + act_cnt[tid]; ++r) row_act[r] = tid;

  const int64_t kblocks = F8 ? K / 64 : K / 32;
  const int ksteps = static_cast<int>(K / 32);
  const int unit = F8 ? 2 : 1;
  const int units = ksteps / unit;
  const int kq = (lane >> 4) * 8;
  const int j = lane & 15;  // this lane's B row: assignment row j
  const u32x4_t zero{0u, 0u, 0u, 0u};
  for (int it = wave; it < 4 * n_act; it += kFcWaves) {
    const int a = it >> 2, q = it & 3;
    const int e = act_e[a];
    const int ks_begin = (q * units / kStreamWaves) * unit;
    const int ks_end = ((q + 1) * units / kStreamWaves) * unit;
    const bool mine = j >= act_off[a] && j < act_off[a] + act_cnt[a];
    const bf16_t* arow = static_cast<const bf16_t*>(g.a) + a_source_row(g, mine ? j : act_off[a]) * g.lda + kq;
    const unsigned char* wsrc =
        static_cast<const unsigned char*>(g.w0) + ((static_cast<int64_t>(e) * nblocks + nb) * kblocks) * 1024 + lane * 16;
    f32x4_t acc{0.f, 0.f, 0.f, 0.f};
    for (int ks = ks_begin; ks < ks_end; ks += kFcUnroll) {
      u32x4_t wv[kFcUnroll];
      if (F8) {
        u32x4_t qv[kFcUnroll / 2];
#pragma unroll
        for (int u = 0; u < kFcUnroll; u += 2)
          qv[u / 2] = ks + u < ks_end
                          ? stream_load(reinterpret_cast<const u32x4_t*>(wsrc + static_cast<int64_t>((ks + u) / 2) * 1024))
                          : zero;
#pragma unroll
        for (int u = 0; u < kFcUnroll; u += 2) f8x16_to_bf16(qv[u / 2], wv[u], wv[u + 1]);
      } else {
#pragma unroll
        for (int u = 0; u < kFcUnroll; ++u)
          wv[u] = ks + u < ks_end
                      ? stream_load(reinterpret_cast<const u32x4_t*>(wsrc + static_cast<int64_t>(ks + u) * 1024))
                      : zero;
      }
      u32x4_t tok[kFcUnroll];
#pragma unroll
      for (int u = 0; u < kFcUnroll; ++u)
        tok[u] = (mine && ks + u < ks_end) ? *reinterpret_cast<const u32x4_t*>(arow + (ks + u) * 32) : zero;
#pragma unroll
      for (int u = 0; u < kFcUnroll; ++u)
        if (ks + u < ks_end) acc = mfma16(wv[u], tok[u], acc);
    }
    part[it][lane] = acc;
  }
  __syncthreads();

  // Lane L of wave 0: assignment row L % 16, columns 4 (L / 16) .. + 3.
  if (wave == 0) {
    const int a = row_act[j];
    if (a >= 0) {
      f32x4_t acc = part[4 * a][lane];
#pragma unroll
      for (int q = 1; q < 4; ++q) acc += part[4 * a + q][lane];
      const int c = 4 * (lane >> 4);
      const int64_t n = n_base + c;
      float4 sc{1.f, 1.f, 1.f, 1.f};
      if (F8) sc = *reinterpret_cast<const float4*>(g.s0 + static_cast<int64_t>(act_e[a]) * N + n);
      const int f = g.order[j];
      if (f >= 0 && f < g.n_assign) {
        const float w = g.route_w[f];
        float v0 = acc[0] * sc.x, v1 = acc[1] * sc.y, v2 = acc[2] * sc.z, v3 = acc[3] * sc.w;
        v0 *= w, v1 *= w, v2 *= w, v3 *= w;
        ys[f][c] = v0, ys[f][c + 1] = v1, ys[f][c + 2] = v2, ys[f][c + 3] = v3;
      }
    }
  }
  __syncthreads();
  // out[t, 4 columns]: slots in order, then the residual, one rounding
  if (tid < n_tokens * 4) {
    const int t = tid >> 2, c = 4 * (tid & 3);
    float acc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] = ys[t][c + i];
    for (int sl = 1; sl < k; ++sl)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] = acc[i] + ys[sl * n_tokens + t][c + i];
    const int64_t o = static_cast<int64_t>(t) * N + n_base + c;
    if (residual) {
      const u32x2_t r = *reinterpret_cast<const u32x2_t*>(residual + o);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t h = r[i / 2];
        const float pv = __uint_as_float((i & 1) ? (h & 0xFFFF0000u) : (h << 16));
        acc[i] = pv + acc[i];
      }
    }
    *reinterpret_cast<u32x2_t*>(out + o) = u32x2_t{pack_bf16x2(acc[0], acc[1]), pack_bf16x2(acc[2], acc[3])};
  }
}

// The grouping of assignment rows: order + offsets, or (streaming kernel
// only, identity_ok) neither, for one expert whose rows are read in order.
bool grouping_ok(const GroupedGemmArgs& g, bool identity_ok) {
  if (g.order && g.offsets) return true;
  return identity_ok && !g.order && !g.offsets && g.n_expert == 1 && g.a_mode == A_DIRECT;
}

bool mfma_common_ok(const GroupedGemmArgs& g) {
  if (g.a_kb_rows || g.out_kb_rows) return false;  // K-blocked operands: 256-tile kernel only
  if (g.act_dtype != DT_BF16) return false;
  if (g.w_dtype != DT_BF16 && g.w_dtype != DT_F8) return false;
  if (g.w_format != WF_MFMA16) return false;
  if (g.epi == EPI_SWIGLU && g.out_dtype != DT_BF16) return false;
  if (g.epi == EPI_SWIGLU && !g.w1) return false;
  if (g.N % 16 || g.lda % 8 || g.ldo % 4) return false;
  if (reinterpret_cast<uintptr_t>(g.a) % 16 || reinterpret_cast<uintptr_t>(g.out) % 16) return false;
  if (g.w_dtype == DT_F8 && (!g.s0 || (g.epi == EPI_SWIGLU && !g.s1))) return false;
  return true;
}

template <bool F8>
hipError_t launch_tiled_t(const GroupedGemmArgs& g, hipStream_t s) {
  const int row_tiles = max_row_tiles(g.n_assign, g.n_expert, kBM);
  if (g.epi == EPI_SWIGLU) {
    using C = Tiled<2>;
    const int col_tiles = static_cast<int>((g.N + C::kBNSet - 1) / C::kBNSet);
    const size_t lds = 2 * (C::kABytes + C::kBBytes);
    const int64_t total = static_cast<int64_t>(row_tiles) * col_tiles;
    const unsigned blocks = static_cast<unsigned>((total + 7) / 8 * 8);
    hipLaunchKernelGGL((gemm_tiled_kernel<EPI_SWIGLU, 2, F8>), dim3(blocks), dim3(kThreads), lds, s, g,
                       row_tiles, col_tiles);
  } else {
    using C = Tiled<1>;
    const int col_tiles = static_cast<int>((g.N + C::kBNSet - 1) / C::kBNSet);
    const size_t lds = 2 * (C::kABytes + C::kBBytes);
    const int64_t total = static_cast<int64_t>(row_tiles) * col_tiles;
    const unsigned blocks = static_cast<unsigned>((total + 7) / 8 * 8);
    if (g.epi == EPI_SCATTER_WEIGHTED)
      hipLaunchKernelGGL((gemm_tiled_kernel<EPI_SCATTER_WEIGHTED, 1, F8>), dim3(blocks), dim3(kThreads), lds,
                         s, g, row_tiles, col_tiles);
    else
      hipLaunchKernelGGL((gemm_tiled_kernel<EPI_SCATTER, 1, F8>), dim3(blocks), dim3(kThreads), lds, s, g,
                         row_tiles, col_tiles);
  }
  return hipGetLastError();
}

template <bool F8, int TILES>
void launch_stream_tiles(const GroupedGemmArgs& g, hipStream_t s, dim3 grid, int col_tiles) {
  grid.y = g.ksplit > 1 ? g.ksplit : 1;
  // The one-tile bf16 gate/up kernel loads 16 steps per trip (2 waves per
  // SIMD) unless its blocks with rows (estimated: column tiles x experts
  // that can have rows) would just overflow one round of 2 blocks per CU
  // that 3 blocks per CU still hold.  Measured (whole block calls, cold):
  // C2 T=16 gate/up 287 -> 278 us, C2 T=1 78 -> 75.5 us, C3 T=1 16.6 ->
  // 15.7 us; C4 T=1 (528 blocks) 18.1 -> 19.5 us.  One-set (down) kernels
  // were slower with it (C4 T=16 51 -> 61 us), and so was the fp8-weight
  // gate/up kernel (C5 T=16 144 -> 156 us, T=1 42.5 -> 47.8 us).
  const int64_t active = static_cast<int64_t>(col_tiles) * (g.n_assign < g.n_expert ? g.n_assign : g.n_expert);
  if (g.epi == EPI_SWIGLU && TILES == 1 && !F8 && !(active > 2 * 256 && active <= 3 * 256)) {
    hipLaunchKernelGGL((gemm_stream_kernel<EPI_SWIGLU, 2, F8, TILES, 16>), grid, dim3(kThreads), 0, s, g, col_tiles);
    return;
  }
  if (g.epi == EPI_SWIGLU)
    hipLaunchKernelGGL((gemm_stream_kernel<EPI_SWIGLU, 2, F8, TILES>), grid, dim3(kThreads), 0, s, g, col_tiles);
  else if (g.epi == EPI_LINEAR)
    hipLaunchKernelGGL((gemm_stream_kernel<EPI_LINEAR, 1, F8, TILES>), grid, dim3(kThreads), 0, s, g, col_tiles);
  else if (g.epi == EPI_QKV_ROPE)
    hipLaunchKernelGGL((gemm_stream_kernel<EPI_QKV_ROPE, 1, F8, TILES>), grid, dim3(kThreads), 0, s, g, col_tiles);
  else if (g.epi == EPI_SCATTER_WEIGHTED)
    hipLaunchKernelGGL((gemm_stream_kernel<EPI_SCATTER_WEIGHTED, 1, F8, TILES>), grid, dim3(kThreads), 0, s, g,
                       col_tiles);
  else
    hipLaunchKernelGGL((gemm_stream_kernel<EPI_SCATTER, 1, F8, TILES>), grid, dim3(kThreads), 0, s, g, col_tiles);
}

// The one-tile gate/up kernel with the routing in its blocks
// (GroupedGemmArgs::rp): one block row per selected expert (at most
// k * n_tokens of them), the trip length chosen as launch_stream_tiles does.
// Every block pays the top-k (about 3 us) before its first weight load, so
// the launch is taken only while its grid fits one round of resident blocks
// (measured, cold calls: C4 T=1, 528 blocks in one round, 38.6 -> 37.1 us;
// C4 T=4, 2112 blocks in about four rounds, 79.4 -> 85.2 us).
template <bool F8, int RNV, int U>
const void* routed_kernel() {
  return reinterpret_cast<const void*>(gemm_stream_kernel<EPI_SWIGLU, 2, F8, 1, U, RNV>);
}

template <bool F8, int RNV>
const void* routed_kernel_for(unsigned blocks) {
  if constexpr (!F8) {
    if (!(blocks > 2 * 256 && blocks <= 3 * 256)) return routed_kernel<F8, RNV, 16>();
  }
  return routed_kernel<F8, RNV, kStreamUnroll>();
}

template <bool F8>
const void* routed_kernel_nv(int nv, unsigned blocks) {
  if (nv == 1) return routed_kernel_for<F8, 1>(blocks);
  if (nv == 4) return routed_kernel_for<F8, 4>(blocks);
  if (nv == 8) return routed_kernel_for<F8, 8>(blocks);
  return nullptr;
}

// Blocks of `kernel` one round of the current device holds (occupancy x
// CUs), cached per device.
int round_blocks(const void* kernel) {
  static std::mutex mu;
  static std::map<std::pair<int, const void*>, int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  std::lock_guard<std::mutex> lk(mu);
  const auto key = std::make_pair(dev, kernel);
  const auto it = cache.find(key);
  if (it != cache.end()) return it->second;
  int per_cu = 0, cus = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kThreads, 0) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  return cache[key] = per_cu * cus;
}

// The routed launch's kernel, or nullptr when the arguments do not qualify
// or its grid would not fit one round.
const void* routed_launch(const GroupedGemmArgs& g, unsigned* grid_out) {
  const RoutePrologue& rp = g.rp;
  const int rows = g.max_rows_per_expert > 0 ? g.max_rows_per_expert : g.n_assign;
  if (!rp.part || g.epi != EPI_SWIGLU || rows > 16 || g.ksplit > 1 || g.n_tokens < 1 || g.n_tokens > 4 ||
      rp.k < 1 || rp.k * g.n_tokens > kWave || g.n_expert > 256 || g.n_expert > 16 * rp.nv || rp.n_split < 1 ||
      !rp.ids || !rp.weights || !rp.order || !rp.offsets || !rp.err_count || !gemm_stream_supported(g))
    return nullptr;
  const int col_tiles = static_cast<int>((g.N + kStreamRows - 1) / kStreamRows);
  const int n_rows = g.n_expert < rp.k * g.n_tokens ? g.n_expert : rp.k * g.n_tokens;
  const unsigned blocks = static_cast<unsigned>(col_tiles * n_rows);
  const void* k = g.w_dtype == DT_F8 ? routed_kernel_nv<true>(rp.nv, blocks) : routed_kernel_nv<false>(rp.nv, blocks);
  if (!k || static_cast<int64_t>(blocks) > round_blocks(k)) return nullptr;
  *grid_out = blocks;
  return k;
}

template <bool F8>
hipError_t launch_stream_routed(const GroupedGemmArgs& g, hipStream_t s, int col_tiles) {
  unsigned blocks = 0;
  const void* k = routed_launch(g, &blocks);
  if (!k) return hipErrorNotSupported;
  GroupedGemmArgs a = g;
  void* args[] = {&a, &col_tiles};
  return hipLaunchKernel(k, dim3(blocks), dim3(kThreads), args, 0, s);
}

template <bool F8>
hipError_t launch_stream_t(const GroupedGemmArgs& g, hipStream_t s) {
  const int col_tiles = static_cast<int>((g.N + kStreamRows - 1) / kStreamRows);
  if (g.rp.part) return launch_stream_routed<F8>(g, s, col_tiles);
  const dim3 grid(static_cast<unsigned>(col_tiles * g.n_expert));
  // Rows one pass must cover to read each expert's weights once.
  const int rows = g.max_rows_per_expert > 0 ? g.max_rows_per_expert : g.n_assign;
  if (!F8 && (g.epi == EPI_LINEAR || g.epi == EPI_QKV_ROPE) && g.n_expert == 1 && !g.offsets && !g.order &&
      g.n_assign <= 16 && g.ksplit <= 1) {
    // 8 ring steps per wave (67 KiB of LDS per block, two blocks per CU): measured
    // against 16 (one block per CU) on the Mixtral attention shape, Q/K/V
    // 19.0 against 22.3 us and the output projection 11.4 against 12.4 us at
    // 16 rows, and ahead at 1 and 4 rows too.
    constexpr int kDepth = 8;
    static const bool configured = [] {
      (void)hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_stream_lds_kernel<EPI_LINEAR, kDepth>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, stream_lds_bytes<kDepth, EPI_LINEAR>());
      (void)hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_stream_lds_kernel<EPI_QKV_ROPE, kDepth>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, stream_lds_bytes<kDepth, EPI_QKV_ROPE>());
      (void)hipGetLastError();
      return true;
    }();
    (void)configured;
    const dim3 lgrid(static_cast<unsigned>(col_tiles));
    if (g.epi == EPI_LINEAR)
      hipLaunchKernelGGL((gemm_stream_lds_kernel<EPI_LINEAR, kDepth>), lgrid,
                         dim3(stream_lds_threads<EPI_LINEAR>()), (stream_lds_bytes<kDepth, EPI_LINEAR>()), s, g);
    else
      hipLaunchKernelGGL((gemm_stream_lds_kernel<EPI_QKV_ROPE, kDepth>), lgrid,
                         dim3(stream_lds_threads<EPI_QKV_ROPE>()), (stream_lds_bytes<kDepth, EPI_QKV_ROPE>()), s, g);
    return hipGetLastError();
  }
  if (rows <= 16)
    launch_stream_tiles<F8, 1>(g, s, grid, col_tiles);
  else if (rows <= 32)
    launch_stream_tiles<F8, 2>(g, s, grid, col_tiles);
  else
    launch_stream_tiles<F8, 4>(g, s, grid, col_tiles);
  return hipGetLastError();
}

}  // namespace

bool gemm_tiled_supported(const GroupedGemmArgs& g) {
  return gemm_tiled256_supported(g) ||
         (g.epi <= EPI_SCATTER_WEIGHTED && mfma_common_ok(g) && grouping_ok(g, false) && g.K % kBK == 0 && g.K > 0);
}

// The fused projection epilogues: one expert read in row order, no K split,
// bf16 outputs stored 8 bytes (4 columns) at a time.
bool proj_epilogue_ok(const GroupedGemmArgs& g) {
  const ProjEpilogue& e = g.pe;
  if (g.ksplit > 1 || g.n_expert != 1 || g.order || g.offsets || g.a_mode != A_DIRECT) return false;
  auto al8 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 8 == 0; };
  if (g.epi == EPI_LINEAR) return e.out && al8(e.out) && al8(e.residual);
  return e.positions && e.q_out && e.k_out && e.v_out && reinterpret_cast<uintptr_t>(e.q_out) % 16 == 0 &&
         al8(e.k_out) && al8(e.v_out) && e.nq > 0 && e.nkv > 0 && e.nq % 4 == 0 && e.nkv % 4 == 0 &&
         e.head_dim > 0 && e.head_dim % 4 == 0 && e.nq % e.head_dim == 0 && e.nkv % e.head_dim == 0 &&
         g.N == static_cast<int64_t>(e.nq) + 2 * e.nkv;
}

bool gemm_stream_routed_ok(const GroupedGemmArgs& g) {
  unsigned blocks = 0;
  return routed_launch(g, &blocks) != nullptr;
}

bool gemm_stream_supported(const GroupedGemmArgs& g) {
  if ((g.epi == EPI_LINEAR || g.epi == EPI_QKV_ROPE) && !proj_epilogue_ok(g)) return false;
  if (g.epi > EPI_QKV_ROPE || g.epi < 0) return false;
  const bool split_ok = g.ksplit <= 1 || (g.epi == EPI_SCATTER && g.out_dtype == DT_F32 && g.split_stride > 0 &&
                                          g.ksplit <= 64);
  return mfma_common_ok(g) && grouping_ok(g, true) && g.K > 0 && g.K % (g.w_dtype == DT_F8 ? 64 : 32) == 0 &&
         split_ok;
}

int resolve_tiled_variant(const GroupedGemmArgs& g, int variant) {
  const bool large_ok = gemm_tiled256_supported(g);
  const bool small_ok = g.epi <= EPI_SCATTER_WEIGHTED && mfma_common_ok(g) && grouping_ok(g, false) &&
                        g.K % kBK == 0 && g.K > 0 && g.ksplit == 1;
  // The 256-tile kernel skips the MFMAs of empty row groups, so it wins at
  // every batch the tiled path serves (measured from ~64 rows per expert);
  // the 128-row kernel covers what it does not support.
  if (variant == TILED_AUTO) variant = large_ok ? TILED_256 : TILED_128;
  if (variant == TILED_256 && large_ok) return TILED_256;
  if (small_ok) return TILED_128;
  return large_ok ? TILED_256 : -1;
}

hipError_t launch_gemm_tiled(const GroupedGemmArgs& g, hipStream_t s, int variant) {
  const int v = resolve_tiled_variant(g, variant);
  if (v == TILED_256) return launch_gemm_tiled256(g, s);
  if (v != TILED_128) return hipErrorNotSupported;
  if (g.n_assign == 0 || g.N == 0) return hipSuccess;
  // 96 KiB of dynamic LDS per block (gfx950 has 160 KiB per CU); set once per process.
  static const bool configured = [] {
    const int b2 = 2 * (Tiled<2>::kABytes + Tiled<2>::kBBytes);
    const int b1 = 2 * (Tiled<1>::kABytes + Tiled<1>::kBBytes);
    const void* k2[] = {reinterpret_cast<const void*>(gemm_tiled_kernel<EPI_SWIGLU, 2, false>),
                        reinterpret_cast<const void*>(gemm_tiled_kernel<EPI_SWIGLU, 2, true>)};
    const void* k1[] = {reinterpret_cast<const void*>(gemm_tiled_kernel<EPI_SCATTER_WEIGHTED, 1, false>),
                        reinterpret_cast<const void*>(gemm_tiled_kernel<EPI_SCATTER_WEIGHTED, 1, true>),
                        reinterpret_cast<const void*>(gemm_tiled_kernel<EPI_SCATTER, 1, false>),
                        reinterpret_cast<const void*>(gemm_tiled_kernel<EPI_SCATTER, 1, true>)};
    for (const void* k : k2) (void)hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, b2);
    for (const void* k : k1) (void)hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, b1);
    (void)hipGetLastError();
    return true;
  }();
  (void)configured;
  return g.w_dtype == DT_F8 ? launch_tiled_t<true>(g, s) : launch_tiled_t<false>(g, s);
}

hipError_t launch_gemm_stream(const GroupedGemmArgs& g, hipStream_t s) {
  if (!gemm_stream_supported(g)) return hipErrorNotSupported;
  if (g.n_assign == 0 || g.N == 0) return hipSuccess;
  return g.w_dtype == DT_F8 ? launch_stream_t<true>(g, s) : launch_stream_t<false>(g, s);
}

hipError_t launch_down_combine_small(const GroupedGemmArgs& d, const void* residual, void* out, int out_dtype,
                                     int n_tokens, int k, hipStream_t s) {
  GroupedGemmArgs g = d;
  g.ksplit = 1;
  if (g.epi != EPI_SCATTER_WEIGHTED || g.out_dtype != DT_F32 || out_dtype != DT_BF16 || !g.order || !g.offsets ||
      !g.route_w || !gemm_stream_supported(g) || g.a_mode != A_DIRECT)
    return hipErrorNotSupported;
  if (n_tokens <= 0 || k <= 0 || g.n_assign != n_tokens * k || g.n_assign > kFcRows) return hipErrorNotSupported;
  if (g.N % 4 || reinterpret_cast<uintptr_t>(out) % 8 || reinterpret_cast<uintptr_t>(residual) % 8)
    return hipErrorNotSupported;
  const int64_t slabs = g.n_assign < g.n_expert ? g.n_assign : g.n_expert;
  const int64_t block_bytes = slabs * kStreamRows * g.K * (g.w_dtype == DT_F8 ? 1 : 2);
  const int64_t blocks = g.N / kStreamRows;
  if (block_bytes * 256 > kFcMaxBlockBytes * (blocks < 256 ? blocks : 256)) return hipErrorNotSupported;
  const dim3 grid(static_cast<unsigned>(blocks));
  if (g.w_dtype == DT_F8)
    hipLaunchKernelGGL(down_combine_small_kernel<true>, grid, dim3(kFcThreads), 0, s, g,
                       static_cast<const bf16_t*>(residual), static_cast<bf16_t*>(out), n_tokens, k);
  else
    hipLaunchKernelGGL(down_combine_small_kernel<false>, grid, dim3(kFcThreads), 0, s, g,
                       static_cast<const bf16_t*>(residual), static_cast<bf16_t*>(out), n_tokens, k);
  return hipGetLastError();
}

}  // namespace fmoe
