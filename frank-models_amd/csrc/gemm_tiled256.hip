// Large-tile MFMA grouped GEMM for gfx950 (bf16 activations x bf16 expert
// weights in the WF_MFMA16 packed layout, fp32 accumulation).  This is the
// prefill kernel of the MoE FFN block: mul_mat_id's per-assignment mat-vecs
// (components/moe/mul_mat_id.mlir:55-94) batched per expert, the gate/up pair
// fused with SwiGLU (components/activation/swiglu.mlir:37-47), the down
// projection with the routing weight (moe_ffn_block.mlir:162-177).
//
// Tile: 256 assignment rows x 256 weight rows (gate/up: 128 + 128) per
// 512-thread block; 4x2 waves, each 64 x 128 = 4 x 8 v_mfma_f32_16x16x32_bf16
// tiles, 128 fp32 accumulators per lane.  Per 32-input stage a wave reads 12
// fragments (12 KiB) from LDS for 32 MFMAs.  A wave's four 16-row groups are
// interleaved (wm, wm+4, wm+8, wm+12), and a wave skips the reads and MFMAs
// of groups past the expert's last row, so the last (partial) row tile of an
// expert costs in proportion to its rows.
//
// Pipeline (bf16 weights): a 5-deep LDS ring of 32-input stages (32 KiB
// each: 256 token rows x 64 B + 16 weight blocks x 1 KiB), filled straight
// from global memory (global_load_lds_dwordx4, no staging registers).  The
// two waves of each SIMD take turns: one multiplies two stages while the
// other reads its next fragments and issues the loads of a stage two to
// three stages ahead (k_body).  Tiles of at most 64 rows take a loop of
// their own (thin_k_loop); fp8 weights take k_loop_f8.
//
// Tile order: each XCD works through a contiguous range of the tiles
// (sched_tile), or, for GEMMs of 16 or more column tiles, through a list
// dealt before the launch (tile_table.h) by the permutation or by a
// one-block kernel (tile_table_kernel).
//
// LDS layouts: weight blocks are copied as packed (lane-ordered 1 KiB blocks,
// conflict-free 16-byte reads); token rows are 64 B with the 16-byte chunk
// index XORed by ((row >> 1) & 3) so the 8 lanes of an LDS read phase hit 8
// distinct bank groups.
#include "common.h"
#include "launch.h"
#include "permute_block.h"
#include "tile_table.h"

namespace fmoe {
namespace {

constexpr int kThreads = 512;
constexpr int kBM = 256;
constexpr int kBN = 256;   // weight rows per tile over all sets
constexpr int kBK = 32;    // inputs per stage
constexpr int kRing = 5;   // bf16: stages in the LDS ring
constexpr int kAStage = kBM * kBK * 2;       // 16 KiB
constexpr int kBStage = (kBN / 16) * 1024;   // 16 KiB
constexpr int kStage = kAStage + kBStage;    // 32 KiB
constexpr int kLds = kRing * kStage;         // 160 KiB
// fp8 weights: 64-input stages (A as two 32-input halves in the bf16 layout,
// then 16 fp8 weight blocks of 16 rows x 64 inputs), 3-deep ring.
constexpr int kStagesF8 = 3;
constexpr int kStageF8 = 2 * kAStage + kBStage;  // 48 KiB
constexpr int kLdsF8 = kStagesF8 * kStageF8;     // 144 KiB
constexpr int kGroupN = 4;                   // column tiles swept together
constexpr bool kThin = true;                 // tiles of <= 64 rows take the thin loop (bf16)

__device__ __forceinline__ f32x4_t mfma16(const u32x4_t a, const u32x4_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

typedef __attribute__((ext_vector_type(8))) int i32x8_t;

// v_mfma_f32_16x16x128_f8f6f4 on e4m3 x e4m3 (format codes 0, 0; scale
// operands 0 select the unscaled form).  Each operand is a lane's 32 codes:
// the 16 bytes it read from each of two consecutive 64-input stages.  Lane
// l of either operand holds row l % 16; the instruction pairs byte b of
// operand-0 lane (i + 16 g) with byte b of operand-1 lane (j + 16 g), so any
// input order works as long as weights and activations share it.
__device__ __forceinline__ f32x4_t mfma_f8x2(const u32x4_t a0, const u32x4_t a1, const u32x4_t b0,
                                             const u32x4_t b1, f32x4_t c) {
  const i32x8_t a = {static_cast<int>(a0[0]), static_cast<int>(a0[1]), static_cast<int>(a0[2]),
                     static_cast<int>(a0[3]), static_cast<int>(a1[0]), static_cast<int>(a1[1]),
                     static_cast<int>(a1[2]), static_cast<int>(a1[3])};
  const i32x8_t b = {static_cast<int>(b0[0]), static_cast<int>(b0[1]), static_cast<int>(b0[2]),
                     static_cast<int>(b0[3]), static_cast<int>(b1[0]), static_cast<int>(b1[1]),
                     static_cast<int>(b1[2]), static_cast<int>(b1[3])};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

// s_waitcnt immediates (gfx9 encoding: vmcnt bits 3:0 and 15:14, expcnt 6:4,
// lgkmcnt 11:8; a field at its maximum does not wait).  Issued through the
// builtin so the compiler's own wait insertion accounts for them.
constexpr int kWaitLgkm0 = 0xC07F;                  // lgkmcnt(0)
constexpr int kWaitVm0 = 0x0F70;                    // vmcnt(0)

// First K stage of piece s of a tile split ksplit ways: equal pieces rounded
// down to even stages, except that a two-way split may put its boundary at
// first64 / 64 of the stages (gemm_tiled256_split_first64).
__host__ __device__ __forceinline__ int split_boundary(int kblocks, int ksplit, int s, int first64 = 32) {
  if (s >= ksplit) return kblocks;
  if (ksplit == 2 && s == 1) return (kblocks * first64 / 64) & ~1;
  return (s * kblocks / ksplit) & ~1;
}

__device__ __forceinline__ int64_t source_row(const GroupedGemmArgs& g, int p) {
  if (g.a_mode == A_GATHER_TOKEN) return g.order[p] % g.n_tokens;
  if (g.a_mode == A_GATHER_FLAT) return g.order[p];
  return p;
}

// Hardware block b runs on XCD b % 8.  Logical tiles are dealt so that each
// XCD owns a contiguous range, swept kGroupN column tiles at a time over all
// row tiles: the row tiles of one expert that share a column tile's weights
// run side by side on one XCD and share its L2.
// With a K split, the split index is the slowest-varying part of the
// logical id.
__device__ __forceinline__ bool logical_tile(int n_row_tiles, int n_col_tiles, int ksplit, int* row_tile,
                                             int* col_tile, int* split) {
  const int per_split = n_row_tiles * n_col_tiles;
  const int total = per_split * ksplit;
  const int per_xcd = (total + 7) / 8;
  const int b = blockIdx.x;
  int logical = (b % 8) * per_xcd + b / 8;
  if (logical >= total) return false;
  *split = logical / per_split;
  logical -= *split * per_split;
  const int group_span = kGroupN * n_row_tiles;
  const int group = logical / group_span;
  const int within = logical - group * group_span;
  const int cols_in_group = min(kGroupN, n_col_tiles - group * kGroupN);
  *row_tile = within / cols_in_group;
  *col_tile = group * kGroupN + within % cols_in_group;
  return true;
}

// ---- The same order over the actual row tiles (up to kSchedExperts
// experts): ceil(count / 256) per expert, counted from the offsets, so the
// XCDs split the real tiles evenly.  The grid is sized for the upper bound
// (every expert with a partial tile); with a skewed routing (Qwen3-like,
// 128 experts with Zipf counts: 355 real of 384 bounded row tiles at 8192
// tokens) the bound-sized ranges left whole XCDs short of work.  (Cutting
// the ranges at equal estimated cost, partial tiles weighted by their
// MFMA share, measured slower than equal counts: a partial tile streams
// its whole weight slab.)
constexpr int kSchedChunks = 4;                 // experts per lane
constexpr int kSchedExperts = 64 * kSchedChunks;

// v of expert e (wave-uniform e), from the lane and chunk that hold it.
__device__ __forceinline__ int sched_get(const int (&v)[kSchedChunks], int e) {
  const int c = e / kWave;
  int x = v[0];
#pragma unroll
  for (int i = 1; i < kSchedChunks; ++i)
    if (c == i) x = v[i];
  return __builtin_amdgcn_readfirstlane(__shfl(x, e % kWave, kWave));
}

// The actual row tiles: R, and per lane and chunk c (expert 64 c + lane)
// its first row, rows and the row tiles before it.
struct SchedTables {
  int off[kSchedChunks], cnt[kSchedChunks], tp[kSchedChunks];
  int R;
};

__device__ __forceinline__ void sched_tables(const GroupedGemmArgs& g, SchedTables& t) {
  const int lane = threadIdx.x & (kWave - 1);
  const int E = g.n_expert;
  const int nch = (E + kWave - 1) / kWave;
  t.R = 0;
#pragma unroll
  for (int c = 0; c < kSchedChunks; ++c) {
    t.off[c] = t.cnt[c] = t.tp[c] = 0;
    if (c < nch) {
      const int e = c * kWave + lane;
      t.off[c] = e < E ? g.offsets[e] : 0;
      t.cnt[c] = e < E ? g.offsets[e + 1] - t.off[c] : 0;
      const int nt = (t.cnt[c] + kBM - 1) / kBM;
      const int incl = wave_inclusive_scan(nt);
      t.tp[c] = t.R + incl - nt;
      t.R += __shfl(incl, kWave - 1, kWave);
    }
  }
  t.R = __builtin_amdgcn_readfirstlane(t.R);
}

// Logical tile L (< R * n_col * ksplit) -> its rows, column tile and split.
__device__ __forceinline__ void sched_decode(const GroupedGemmArgs& g, const SchedTables& t, int n_col, int L,
                                             TileInfo* ti, int* col_tile, int* split) {
  const int lane = threadIdx.x & (kWave - 1);
  const int E = g.n_expert;
  const int nch = (E + kWave - 1) / kWave;
  const int tiles_split = t.R * n_col;
  const int sp = L / tiles_split;
  const int l = L - sp * tiles_split;
  const int group_span = kGroupN * t.R;
  const int grp = l / group_span;
  const int within = l - grp * group_span;
  const int cig = min(kGroupN, n_col - grp * kGroupN);
  const int r = within / cig;
  // the expert of row tile r: the last one whose tiles start at or before r
  // (an expert with no rows shares its start with the next one)
  int n = 0;
#pragma unroll
  for (int c = 0; c < kSchedChunks; ++c)
    if (c < nch) n += __popcll(__ballot(c * kWave + lane < E && t.tp[c] <= r));
  const int e = n - 1;
  const int local = r - sched_get(t.tp, e);
  ti->expert = __builtin_amdgcn_readfirstlane(e);
  ti->row0 = __builtin_amdgcn_readfirstlane(sched_get(t.off, e) + local * kBM);
  ti->rows = __builtin_amdgcn_readfirstlane(min(kBM, sched_get(t.cnt, e) - local * kBM));
  *col_tile = __builtin_amdgcn_readfirstlane(grp * kGroupN + within % cig);
  *split = __builtin_amdgcn_readfirstlane(sp);
}

// XCD x's range [lo, hi) of the logical order: ceil(total / 8) tiles each.
__device__ __forceinline__ void sched_range(const GroupedGemmArgs& g, const SchedTables& t, int n_col, int* lo,
                                            int* hi) {
  const int total = t.R * n_col * g.ksplit;
  const int per = (total + 7) / 8;
  const int x = static_cast<int>(blockIdx.x % 8);
  *lo = min(x * per, total);
  *hi = min(*lo + per, total);
}

// This block's tile (one tile per block): false when the block has none.
__device__ __forceinline__ bool sched_tile(const GroupedGemmArgs& g, int n_col, TileInfo* ti, int* col_tile,
                                           int* split) {
  SchedTables t;
  sched_tables(g, t);
  int lo, hi;
  sched_range(g, t, n_col, &lo, &hi);
  const int L = lo + static_cast<int>(blockIdx.x / 8);
  if (L >= hi) return false;
  sched_decode(g, t, n_col, L, ti, col_tile, split);
  return true;
}

// ---- Per-launch tile schedule (the block's prefill GEMMs), dealt longest
// first over the XCDs (tile_table.h).  The permutation builds it beside its
// scatter when the caller asks (GroupedGemmArgs::tile_table_ready); this
// one-block kernel builds it otherwise.
// GEMMs with fewer column tiles keep the in-kernel ranges: one with a table
// the permutation built, and one with a table this launcher builds first.
constexpr int kTableMinCols = 16;
constexpr int kTableMinColsOwn = 32;
static_assert(kBM == ttab::kBM, "the table deals this kernel's tiles");

__global__ __launch_bounds__(perm::kThreads) void tile_table_kernel(const int* __restrict__ offsets, int n_expert,
                                                                     TileTableReq r) {
  __shared__ int rows[ttab::kMaxExperts];
  for (int e = threadIdx.x; e < n_expert; e += perm::kThreads) rows[e] = offsets[e + 1] - offsets[e];
  __syncthreads();
  ttab::build(rows, n_expert, r, reinterpret_cast<int4*>(r.table));
}

// The epilogue, staged through LDS so that every global store writes whole
// contiguous output rows (16 bytes per lane, 256 B - 1 KiB per row) instead
// of 16 rows x 32-64 B.  The lane holds assignment row (lane & 15) of each
// 16-row group and outputs 4*(lane >> 4) .. +4 of each 16-output fragment.
// Two passes of 128 tile rows (groups m = 2P, 2P+1 of every wave): write the
// finished values to LDS (row pitch = row bytes + 16), barrier, then the
// block stores them row by row.  SwiGLU rows go to h in expert-sorted order
// (row p); the scatter epilogues write row order[p], times the routing
// weight for EPI_SCATTER_WEIGHTED, and K-split partials (fp32 or bf16) at
// split * split_stride.  The scatter epilogues first load the tile's
// order[p] (loaded before the K loop) and routing weights once into an LDS
// table behind the staging rows, so each pass waits on no global load.  fp32 outputs take the weight
// as they are read back, bf16 outputs before rounding (the same fp32
// product either way).  fp8 weights: the per-output-channel scale
// multiplies the fp32 dot product.
// What the scatter epilogues read from global memory per row of the tile:
// the destination order[p] of row `threadIdx.x`, loaded before the
// prologue's stage loads (its round trip overlaps theirs), and the routing
// weight route_w[order[p]], loaded after the K loop (waiting for order
// before it would wait for the stage loads issued after it).
struct EpiRows {
  int o = 0;
  float w = 1.f;
  bool have_w = false;
};

template <int EPI>
__device__ __forceinline__ void epi_rows_first(const GroupedGemmArgs& g, const TileInfo& ti, EpiRows& er) {
  if constexpr (EPI != EPI_SWIGLU) {
    if (static_cast<int>(threadIdx.x) < ti.rows) er.o = g.order[ti.row0 + threadIdx.x];
  }
}

template <int EPI>
__device__ __forceinline__ void epi_rows_second(const GroupedGemmArgs& g, const TileInfo& ti, EpiRows& er) {
  if constexpr (EPI == EPI_SCATTER_WEIGHTED) {
    if (static_cast<int>(threadIdx.x) < ti.rows) er.w = g.route_w[er.o];
    er.have_w = true;
  }
}

template <int EPI, int NSETS, bool F8, bool A8, bool OUT_F32>
__device__ __forceinline__ void epilogue(const GroupedGemmArgs& g, const TileInfo& ti, int split, int64_t n0,
                                         int wm, int wn, int lane, unsigned char* lds, const f32x4_t (&acc)[8][4],
                                         const EpiRows& er) {
  constexpr int kFrags = NSETS == 2 ? 4 : 8;       // output fragments per wave
  constexpr int kEsz = OUT_F32 ? 4 : 2;
  constexpr int kRowBytes = (NSETS == 2 ? kBN / 2 : kBN) * kEsz;
  constexpr int kPitch = kRowBytes + 16;
  constexpr int kChunks = kRowBytes / 16;          // 16-byte chunks per row
  const int64_t N = g.N;
  const int colw = (NSETS == 2 ? wn * 64 : wn * 128) + 4 * (lane >> 4);
  constexpr bool kScatter = EPI != EPI_SWIGLU;
  constexpr bool kWeighted = EPI == EPI_SCATTER_WEIGHTED;
  int* t_order = reinterpret_cast<int*>(lds + 128 * kPitch);           // [256]
  float* t_w = reinterpret_cast<float*>(lds + 128 * kPitch + 1024);    // [256]
  if constexpr (kScatter) {
    const int t = static_cast<int>(threadIdx.x);
    float w = er.w;
    if (kWeighted && !er.have_w && t < ti.rows) w = g.route_w[er.o];
    lds_barrier();  // the ring is no longer read
    if (t < kBM) {
      t_order[t] = er.o;
      if (kWeighted) t_w[t] = w;
    }
  }
  // fp8 activations: each A row's dequantisation scale (rows past the tile: 1)
  float as[4] = {1.f, 1.f, 1.f, 1.f};
  if constexpr (A8) {
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const int r = (wm + 4 * m) * 16 + (lane & 15);
      if (r < ti.rows) as[m] = g.a_scale[ti.row0 + r];
    }
  }
  f32x4_t sc0[kFrags], sc1[kFrags];
#pragma unroll
  for (int n = 0; n < kFrags; ++n) {
    sc0[n] = sc1[n] = f32x4_t{1.f, 1.f, 1.f, 1.f};
    if constexpr (F8) {
      const int64_t col = n0 + colw + n * 16;
      if (col < N) {
        sc0[n] = *reinterpret_cast<const f32x4_t*>(g.s0 + ti.expert * N + col);
        if (NSETS == 2) sc1[n] = *reinterpret_cast<const f32x4_t*>(g.s1 + ti.expert * N + col);
      }
    }
  }
#pragma unroll
  for (int pass = 0; pass < 2; ++pass) {
    lds_barrier();  // the ring (or the last pass's rows) is no longer read
#pragma unroll
    for (int mm = 0; mm < 2; ++mm) {
      const int m = 2 * pass + mm;
      const int rl = (wm + 4 * mm) * 16 + (lane & 15);  // row within the pass
      const float w = kWeighted && !OUT_F32 ? t_w[pass * 128 + rl] : 1.f;
      unsigned char* dst = lds + rl * kPitch + colw * kEsz;
#pragma unroll
      for (int n = 0; n < kFrags; ++n) {
        const f32x4_t a0 = acc[n][m] * sc0[n] * as[m];
        f32x4_t v;
        if constexpr (EPI == EPI_SWIGLU) {
          const f32x4_t a1 = acc[n + 4][m] * sc1[n] * as[m];
          v = f32x4_t{silu_mul(a0[0], a1[0]), silu_mul(a0[1], a1[1]), silu_mul(a0[2], a1[2]), silu_mul(a0[3], a1[3])};
        } else {
          v = a0 * w;
        }
        if constexpr (OUT_F32)
          *reinterpret_cast<f32x4_t*>(dst + n * 16 * 4) = v;
        else
          *reinterpret_cast<u32x2_t*>(dst + n * 16 * 2) = u32x2_t{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
      }
    }
    lds_barrier();
#pragma unroll
    for (int i = 0; i < 128 * kChunks / kThreads; ++i) {
      const int id = i * kThreads + static_cast<int>(threadIdx.x);
      const int rl = id / kChunks, ch = id % kChunks;
      const int r = pass * 128 + rl;
      const int64_t col = n0 + ch * (16 / kEsz);
      if constexpr (A8 && EPI == EPI_SWIGLU) {
        // The next GEMM's per-row activation scale: max|h| of this tile's
        // columns of row r (its 16 chunks sit on one 16-lane DPP row).
        float m = 0.f;
        if (r < ti.rows && col < N) m = absmax_bf16x8(*reinterpret_cast<const u32x4_t*>(lds + rl * kPitch + ch * 16));
        m = row16_max(m);
        if (ch == 0 && r < ti.rows && g.row_amax) atomicMax(g.row_amax + ti.row0 + r, __float_as_uint(m));
      }
      if (r >= ti.rows || col >= N) continue;
      u32x4_t v = *reinterpret_cast<const u32x4_t*>(lds + rl * kPitch + ch * 16);
      if constexpr (kWeighted && OUT_F32)
        v = __builtin_bit_cast(u32x4_t, __builtin_bit_cast(f32x4_t, v) * t_w[r]);
      const int64_t row = kScatter ? static_cast<int64_t>(t_order[r]) : static_cast<int64_t>(ti.row0 + r);
      const int64_t elem = !kScatter && g.out_kb_rows ? kb_offset(row, col, g.out_kb_rows)
                                                      : split * g.split_stride + row * g.ldo + col;
      unsigned char* out = static_cast<unsigned char*>(g.out) + elem * kEsz;
      *reinterpret_cast<u32x4_t*>(out) = v;
    }
  }
}

// Everything one wave needs to stage and read tiles: computed once per block.
struct WaveCtx {
  unsigned char* lds;
  const unsigned char* a_base;
  uint32_t a_off[4];           // byte offsets of the staged token rows: this wave's share (0, 1), wave ^ 4's (2, 3)
  const unsigned char* b_base[4];  // staged weight row blocks, same order
  uint32_t b_lane;
  uint32_t a_kstride;          // bytes between the 32-input blocks of an A row (64, or 64 * rows K-blocked)
  uint32_t a_plane;            // two-term e4m3 activations: bytes from the hi to the lo codes
  int a_lane;                  // LDS byte offset of this lane's A fragment in a 16-row group
  int wave, wm, wn;
  int KT;                      // stages of 32 inputs in this block's K range
};

// Fragment m of a wave covers 16-row group wm + 4 m of the tile, so the
// groups of a partial tile are spread over all four SIMDs.
template <int NM, int NSETS>
__device__ __forceinline__ void read_frags(const WaveCtx& c, int buf, u32x4_t* fa, u32x4_t* fb) {
  const unsigned char* st = c.lds + buf * kStage;
#pragma unroll
  for (int m = 0; m < NM; ++m)
    fa[m] = *reinterpret_cast<const u32x4_t*>(st + (c.wm + 4 * m) * 16 * 64 + c.a_lane);
#pragma unroll
  for (int n = 0; n < 8; ++n) {
    const int rb = NSETS == 2 ? ((n >> 2) * 8 + c.wn * 4 + (n & 3)) : (c.wn * 8 + n);
    fb[n] = *reinterpret_cast<const u32x4_t*>(st + kAStage + rb * 1024 + c.b_lane);
  }
}

// One group's loads of a whole stage: this wave's share and wave ^ 4's.
template <int NSETS>
__device__ __forceinline__ void issue_full_stage(const WaveCtx& c, int kt, int buf) {
  unsigned char* st = c.lds + buf * kStage;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int share = j < 2 ? c.wave : (c.wave ^ 4);
    __builtin_amdgcn_global_load_lds(c.a_base + (c.a_off[j] + static_cast<uint32_t>(kt) * c.a_kstride),
                                     st + (share * 2 + (j & 1)) * 1024, 16, 0, 0);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int share = j < 2 ? c.wave : (c.wave ^ 4);
    __builtin_amdgcn_global_load_lds(c.b_base[j] + (static_cast<uint32_t>(kt) * 1024 + c.b_lane),
                                     st + kAStage + (share * 2 + (j & 1)) * 1024, 16, 0, 0);
  }
}

// The K loop, ping-pong between two wave groups: G0 = waves 0-3 and G1 =
// waves 4-7, one wave of each per SIMD.  Barriers cut time into slots.  In
// every slot one group multiplies two 32-input stages (64 MFMAs per wave,
// operands already in registers) while the other reads its next fragments
// from LDS and loads a later stage, and the groups swap at each barrier, so
// each SIMD's matrix core is fed by one wave while the other wave's LDS
// traffic and barrier wait overlap it.  The ring holds kRing = 5 stages;
// super-step j = stages 2j, 2j+1.
//   Slot 2j:   G0 multiplies j; G1 reads j's fragments and loads stage 2j+4.
//   Slot 2j+1: G1 multiplies j; G0 reads j+1's fragments and loads stage 2j+5.
// Each stage is loaded whole by one group (8 loads per thread).  G1 ends its
// memory slot 2j with stage 2j+2 complete (only stage 2j+4 in flight), G0
// ends its compute slot 2j with stage 2j+3 complete, so stages 2j+2 and
// 2j+3 are visible from the barrier that ends slot 2j, before G0 reads them
// in slot 2j+1.  At slot 2j the live stages are 2j..2j+4, five distinct
// buffers; the buffer G1 refills held stage 2j-1 (last read in slot 2j-2),
// the one G0 refills in slot 2j+1 held stage 2j (last read in slot 2j).
// Stages past the end are not loaded; the waits then drain everything.
// The MFMAs of one super-step (two stages) for one wave: bf16 operands run
// one 16x16x32 MFMA per stage and fragment pair; fp8 activations (A8) run
// one 16x16x128 MFMA per fragment pair over both 64-input stages.
template <int NM, bool A8>
__device__ __forceinline__ void multiply2(f32x4_t (&acc)[8][4], const u32x4_t (&fa)[2][4], const u32x4_t (&fb)[2][8]) {
  if constexpr (A8) {
#pragma unroll
    for (int n = 0; n < 8; ++n)
#pragma unroll
      for (int m = 0; m < NM; ++m) acc[n][m] = mfma_f8x2(fb[0][n], fb[1][n], fa[0][m], fa[1][m], acc[n][m]);
  } else {
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int n = 0; n < 8; ++n)
#pragma unroll
        for (int m = 0; m < NM; ++m) acc[n][m] = mfma16(fb[h][n], fa[h][m], acc[n][m]);
  }
}

// The loop's prologue loads: this group's stages (1 - G and 3 - G) that lie
// in [s_lo, s_hi), each into the buffer of its own index.
template <int NSETS>
__device__ __forceinline__ void k_issue_range(const WaveCtx& c, int s_lo, int s_hi) {
  const int G = c.wave >> 2;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int st = 2 * i + 1 - G;
    if (st >= s_lo && st < s_hi && st < c.KT) issue_full_stage<NSETS>(c, st, st);
  }
}

// The K loop after its prologue loads were issued (k_issue_range over
// stages 0..3).  With more than two stages the last load a group issued is
// its stage 3 - G, so vmcnt(8) leaves its first stage complete.
template <int NM, int NSETS, int G, bool A8>
__device__ __forceinline__ void k_body(const WaveCtx& c, f32x4_t (&acc)[8][4]) {
  constexpr int R = kRing;
  const int KT = c.KT;  // even
  const int JT = KT >> 1;
  u32x4_t fa[2][4], fb[2][8];
  const bool two = KT > 2;
  if (two)
    __builtin_amdgcn_s_waitcnt(wait_vm(8, false));
  else
    __builtin_amdgcn_s_waitcnt(kWaitVm0);
  asm volatile("s_barrier" ::: "memory");
  if constexpr (G == 0) {
    if constexpr (NM > 0) {
      read_frags<NM, NSETS>(c, 0, fa[0], fb[0]);
      read_frags<NM, NSETS>(c, 1, fa[1], fb[1]);
    }
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
  }
  asm volatile("s_barrier" ::: "memory");

  int b0 = 0;  // buffer of stage 2j
  for (int j = 0; j < JT; ++j) {
    const int b1 = b0 + 1 >= R ? b0 + 1 - R : b0 + 1;
    const int b2 = b0 + 2 >= R ? b0 + 2 - R : b0 + 2;
    const int b3 = b0 + 3 >= R ? b0 + 3 - R : b0 + 3;
    const int b4 = b0 + 4 >= R ? b0 + 4 - R : b0 + 4;
    if constexpr (G == 0) {
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_setprio(1);
      multiply2<NM, A8>(acc, fa, fb);
      __builtin_amdgcn_s_setprio(0);
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_waitcnt(kWaitVm0);
      asm volatile("s_barrier" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (NM > 0) {
        if (j + 1 < JT) {
          read_frags<NM, NSETS>(c, b2, fa[0], fb[0]);
          read_frags<NM, NSETS>(c, b3, fa[1], fb[1]);
        }
      }
      if (2 * j + 5 < KT) issue_full_stage<NSETS>(c, 2 * j + 5, b0);
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
      asm volatile("s_barrier" ::: "memory");
    } else {
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (NM > 0) {
        read_frags<NM, NSETS>(c, b0, fa[0], fb[0]);
        read_frags<NM, NSETS>(c, b1, fa[1], fb[1]);
      }
      if (2 * j + 4 < KT) {
        issue_full_stage<NSETS>(c, 2 * j + 4, b4);
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(wait_vm(8, true));
      } else {
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(wait_vm(0, true));
      }
      asm volatile("s_barrier" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_setprio(1);
      multiply2<NM, A8>(acc, fa, fb);
      __builtin_amdgcn_s_setprio(0);
      __builtin_amdgcn_sched_barrier(0);
      asm volatile("s_barrier" ::: "memory");
    }
    b0 = b2;
  }
  __builtin_amdgcn_s_waitcnt(kWaitVm0);
}

// ---------------------------------------------------------------- fp8 weights
// Stage kt (64 inputs) in buffer buf: A halves h = 0, 1 (inputs 32 h .. +32)
// at h * kAStage in the bf16 layout, the 16 fp8 weight blocks after them.
// One of the 6 global->LDS loads of an fp8 stage (d = 0..3: A half d >> 1,
// row set d & 1; d = 4, 5: weight blocks).
// With two-term e4m3 activations (X2) the A halves are the stage's 64-input
// piece of the hi codes (h = 0) and of the lo codes (h = 1).
template <bool X2>
__device__ __forceinline__ void issue_one_f8(const WaveCtx& c, int kt, int buf, int d) {
  unsigned char* st = c.lds + buf * kStageF8;
  if (d < 4) {
    const int h = d >> 1, j = d & 1;
    const uint32_t src = X2 ? h * c.a_plane + c.a_off[j] + static_cast<uint32_t>(kt) * c.a_kstride
                            : c.a_off[j] + static_cast<uint32_t>(2 * kt + h) * c.a_kstride;
    __builtin_amdgcn_global_load_lds(c.a_base + src, st + h * kAStage + (c.wave * 2 + j) * 1024, 16, 0, 0);
  } else {
    const int j = d - 4;
    __builtin_amdgcn_global_load_lds(c.b_base[j] + (static_cast<uint32_t>(kt) * 1024 + c.b_lane),
                                     st + 2 * kAStage + (c.wave * 2 + j) * 1024, 16, 0, 0);
  }
}

__device__ __forceinline__ u32x4_t read_a_frag(const WaveCtx& c, const unsigned char* half_base, int m) {
  return *reinterpret_cast<const u32x4_t*>(half_base + (c.wm + 4 * m) * 16 * 64 + c.a_lane);
}

// Weight fragment n of a stage, still fp8: lane bytes 0-7 feed the first
// 32-input half, bytes 8-15 the second.
template <int NSETS>
__device__ __forceinline__ u32x4_t read_b_frag(const WaveCtx& c, const unsigned char* b_base, int n) {
  const int rb = NSETS == 2 ? ((n >> 2) * 8 + c.wn * 4 + (n & 3)) : (c.wn * 8 + n);
  return *reinterpret_cast<const u32x4_t*>(b_base + rb * 1024 + c.b_lane);
}

template <int H>
__device__ __forceinline__ u32x4_t convert_frag(const u32x4_t q) {
  return f8x8_to_bf16x8(q[2 * H], q[2 * H + 1]);
}

// This wave's 6 loads of fp8 stage kt (its share) into buffer buf.
template <bool X2>
__device__ __forceinline__ void issue_share_f8(const WaveCtx& c, int kt, int buf) {
#pragma unroll
  for (int d = 0; d < 6; ++d) issue_one_f8<X2>(c, kt, buf, d);
}

// A fragments of both 32-input halves and the 8 raw fp8 weight fragments of
// the stage in buffer buf.
template <int NM, int NSETS>
__device__ __forceinline__ void read_stage_f8(const WaveCtx& c, int buf, u32x4_t (&fa)[2][4], u32x4_t (&fq)[8]) {
  const unsigned char* st = c.lds + buf * kStageF8;
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int m = 0; m < NM; ++m) fa[h][m] = read_a_frag(c, st + h * kAStage, m);
#pragma unroll
  for (int n = 0; n < 8; ++n) fq[n] = read_b_frag<NSETS>(c, st + 2 * kAStage, n);
}

// The 64 MFMAs of one fp8 stage, half by half; weight fragment n+1's codes
// are converted to bf16 while fragment n's MFMAs run.  Two-term e4m3
// activations (X2): one 16x16x128 fp8 MFMA per fragment pair, its first
// operand the weight codes twice, its second the hi and the lo codes, so
// the 128 products are w * hi and w * lo over the stage's 64 inputs.
template <int NM, bool X2>
__device__ __forceinline__ void multiply_f8(f32x4_t (&acc)[8][4], const u32x4_t (&fa)[2][4], const u32x4_t (&fq)[8]) {
  if constexpr (X2) {
#pragma unroll
    for (int n = 0; n < 8; ++n)
#pragma unroll
      for (int m = 0; m < NM; ++m) acc[n][m] = mfma_f8x2(fq[n], fq[n], fa[0][m], fa[1][m], acc[n][m]);
  } else if constexpr (NM > 0) {
    u32x4_t cur = convert_frag<0>(fq[0]);
#pragma unroll
    for (int n = 0; n < 8; ++n) {
      const u32x4_t nxt = n < 7 ? convert_frag<0>(fq[n + 1]) : convert_frag<1>(fq[0]);
#pragma unroll
      for (int m = 0; m < NM; ++m) acc[n][m] = mfma16(cur, fa[0][m], acc[n][m]);
      cur = nxt;
    }
#pragma unroll
    for (int n = 0; n < 8; ++n) {
      const u32x4_t nxt = n < 7 ? convert_frag<1>(fq[n + 1]) : cur;
#pragma unroll
      for (int m = 0; m < NM; ++m) acc[n][m] = mfma16(cur, fa[1][m], acc[n][m]);
      cur = nxt;
    }
  }
}

// K loop for fp8 weights: the bf16 loop's ping-pong between wave groups G0
// (waves 0-3) and G1 (waves 4-7), one 64-input stage per slot, a 3-deep ring
// (R = kStagesF8), and each wave loading its own share (6 loads) of a stage.
//   Slot 2k:   G0 multiplies stage k; G1 reads stage k and loads stage k+2.
//   Slot 2k+1: G1 multiplies stage k; G0 reads stage k+1 and loads stage k+3.
// Every memory slot ends with lgkmcnt(0) and vmcnt(6): only the share just
// issued may be in flight, so G1 has stage k+1 and G0 stage k+2 complete,
// each ahead of the barrier before its first reader.  The buffer a load
// refills held stage k-1 (G1, last read in slot 2k-2) or stage k (G0, last
// read in slot 2k); the other buffers hold stages being read or still
// landing.  Loads past the last stage are not issued (those slots wait for
// everything instead); the prologue re-reads the last stage into buffers
// that are never read when K has fewer stages than the ring.
template <int NM, int NSETS, int G, bool X2>
__device__ __forceinline__ void k_loop_f8(const WaveCtx& c, f32x4_t (&acc)[8][4]) {
  constexpr int R = kStagesF8;
  const int KT = c.KT;
  u32x4_t fa[2][4], fq[8];
#pragma unroll
  for (int s = 0; s < (G == 0 ? R : R - 1); ++s) issue_share_f8<X2>(c, s < KT ? s : KT - 1, s);
  __builtin_amdgcn_s_waitcnt(wait_vm(6 * (G == 0 ? R - 1 : R - 2), false));
  asm volatile("s_barrier" ::: "memory");
  if constexpr (G == 0) {
    if constexpr (NM > 0) read_stage_f8<NM, NSETS>(c, 0, fa, fq);
    __builtin_amdgcn_s_waitcnt(wait_vm(6 * (R - 2), true));
  }
  asm volatile("s_barrier" ::: "memory");

  int rd = G == 0 ? 1 : 0;      // buffer of the stage this group reads next
  int wr = G == 0 ? 0 : R - 1;  // buffer its next load refills
  for (int kt = 0; kt < KT; ++kt) {
    if constexpr (G == 0) {
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_setprio(1);
      multiply_f8<NM, X2>(acc, fa, fq);
      __builtin_amdgcn_s_setprio(0);
      __builtin_amdgcn_sched_barrier(0);
      asm volatile("s_barrier" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (NM > 0)
        if (kt + 1 < KT) read_stage_f8<NM, NSETS>(c, rd, fa, fq);
      if (kt + R < KT) {
        issue_share_f8<X2>(c, kt + R, wr);
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(wait_vm(6 * (R - 2), true));
      } else {
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(wait_vm(0, true));
      }
      asm volatile("s_barrier" ::: "memory");
    } else {
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (NM > 0) read_stage_f8<NM, NSETS>(c, rd, fa, fq);
      if (kt + R - 1 < KT) {
        issue_share_f8<X2>(c, kt + R - 1, wr);
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(wait_vm(6 * (R - 2), true));
      } else {
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(wait_vm(0, true));
      }
      asm volatile("s_barrier" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_setprio(1);
      multiply_f8<NM, X2>(acc, fa, fq);
      __builtin_amdgcn_s_setprio(0);
      __builtin_amdgcn_sched_barrier(0);
      asm volatile("s_barrier" ::: "memory");
    }
    rd = rd + 1 == R ? 0 : rd + 1;
    wr = wr + 1 == R ? 0 : wr + 1;
  }
  __builtin_amdgcn_s_waitcnt(kWaitVm0);
}

// Byte offset (from the A base) of this lane's 16-byte piece of 16-row
// group `group` of the tile in the stage that starts at A piece kb_first:
// row group * 16 + (lane >> 2), physical chunk lane & 3, which holds logical
// chunk (lane & 3) ^ ((lane >> 3) & 3).  Rows past the tile re-read its
// first row.
__device__ __forceinline__ uint32_t a_group_offset(const GroupedGemmArgs& g, const TileInfo& ti, int group, int lane,
                                                   int64_t kb_first) {
  const int r = group * 16 + (lane >> 2);
  const int p = ti.row0 + (r < ti.rows ? r : 0);
  const int ch = (lane & 3) ^ ((lane >> 3) & 3);
  return g.a_kb_rows ? static_cast<uint32_t>((kb_first * g.a_kb_rows + p) * 64 + ch * 16)
                     : static_cast<uint32_t>(source_row(g, p) * g.lda * 2 + ch * 16 + kb_first * 64);
}

// Stage sources of tile (ti, col_tile, split) for this wave.  A stage is
// staged in 8 shares; share w holds token rows (w*2 + j)*16 + (lane >> 2),
// 16-byte physical chunk (lane & 3), which holds logical chunk
// (lane & 3) ^ ((lane >> 3) & 3), and weight row blocks w*2 + j.  Each wave
// keeps the addresses of its own share (j = 0, 1) and of share wave ^ 4
// (j = 2, 3): the bf16 loop has one group load a whole stage, the fp8 loop
// has every wave load its own share.  Rows past the tile re-read its first
// row.  Byte offsets from the A base fit 32 bits (checked on the host).  A
// K-blocked A operand keeps each 32-input block of the tile's rows in one
// contiguous run.
template <int NSETS, bool F8, bool A8>
__device__ __forceinline__ WaveCtx tile_ctx(const GroupedGemmArgs& g, const TileInfo& ti, int col_tile, int split,
                                            unsigned char* lds, int lane, int wave) {
  const int64_t N = g.N, K = g.K;
  const int64_t n0 = static_cast<int64_t>(col_tile) * (kBN / NSETS);
  const int64_t nblocks = N / 16;
  constexpr int kStageInputs = F8 ? 64 : 32;  // one packed weight block
  const int64_t kblocks = K / kStageInputs;
  // This block's share of K: stages [k_first, k_first + KT), piece s covering
  // [b(s), b(s+1)) with b = split_boundary, a multiple of two stages (the bf16
  // loop runs two stages per trip).
  const int k_first = split_boundary(static_cast<int>(kblocks), g.ksplit, split, g.ksplit_first64);
  const int KT = split_boundary(static_cast<int>(kblocks), g.ksplit, split + 1, g.ksplit_first64) - k_first;
  WaveCtx c;
  c.lds = lds;
  c.a_base = static_cast<const unsigned char*>(g.a);
  const bool a_kb = g.a_kb_rows > 0;
  c.a_kstride = a_kb ? static_cast<uint32_t>(g.a_kb_rows * 64) : 64u;
  c.a_plane = static_cast<uint32_t>(g.a_lo_plane);
  // first A piece of this block's K range (bf16 pieces hold 32 inputs, fp8 pieces 64)
  const int64_t kb_first = static_cast<int64_t>(k_first) * (A8 ? 1 : kStageInputs / 32);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int share = j < 2 ? wave : (wave ^ 4);
    c.a_off[j] = a_group_offset(g, ti, share * 2 + (j & 1), lane, kb_first);
  }
  // Weight blocks (wave-uniform addresses).  The packed buffer has a
  // 256-row tail, so row blocks past N stay in bounds (their columns are
  // never stored).
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int rb = (j < 2 ? wave : (wave ^ 4)) * 2 + (j & 1);
    const int set = NSETS == 2 ? rb >> 3 : 0;
    const int64_t nb = n0 / 16 + (NSETS == 2 ? (rb & 7) : rb);
    const unsigned char* w = static_cast<const unsigned char*>(set == 0 ? g.w0 : g.w1);
    c.b_base[j] = w + ((static_cast<int64_t>(ti.expert) * nblocks + nb) * kblocks + k_first) * 1024;
  }
  c.b_lane = lane * 16;
  // A fragment: row (lane & 15) of a 16-row group, logical chunk lane >> 4
  // (the XOR swizzle depends only on the row within the group).
  c.a_lane = (lane & 15) * 64 + ((((lane >> 4) ^ (((lane & 15) >> 1) & 3))) << 4);
  c.wave = wave;
  c.wm = wave >> 1;  // 16-row groups wm, wm+4, wm+8, wm+12
  c.wn = wave & 1;   // weight rows of each set: wn half
  c.KT = KT;
  return c;
}

// ---- Thin tiles (bf16, at most 64 rows: one 16-row group per wave pair).
// Such a tile is bound by how many weight bytes are in flight, not by its
// few MFMAs, so it runs its own loop: 20 KiB stages (the 4 KiB of token
// rows it has, then the 16 weight blocks) in an 8-deep ring with 6 stages
// in flight, against 2-3 of the 32 KiB stages in the main loop.  Waves 0-3
// load token group `wave` and every wave its two weight blocks; one barrier
// per stage (a buffer is refilled two stages after its last read).
constexpr int kThinRows = 64;
constexpr int kThinStage = 20 * 1024;
constexpr int kThinRing = kLds / kThinStage;  // 8
constexpr int kThinAhead = kThinRing - 2;     // stages in flight

__device__ __forceinline__ void thin_issue(const WaveCtx& c, uint32_t a_off_thin, int kt, int buf) {
  unsigned char* st = c.lds + buf * kThinStage;
  if (c.wave < 4)
    __builtin_amdgcn_global_load_lds(c.a_base + (a_off_thin + static_cast<uint32_t>(kt) * c.a_kstride),
                                     st + c.wave * 1024, 16, 0, 0);
#pragma unroll
  for (int j = 0; j < 2; ++j)
    __builtin_amdgcn_global_load_lds(c.b_base[j] + (static_cast<uint32_t>(kt) * 1024 + c.b_lane),
                                     st + 4096 + (c.wave * 2 + j) * 1024, 16, 0, 0);
}

template <int NSETS>
__device__ __forceinline__ void thin_k_loop(const WaveCtx& c, uint32_t a_off_thin, int rows, f32x4_t (&acc)[8][4]) {
  const int KT = c.KT;
  const bool active = c.wm * 16 < rows;  // this wave pair's row group holds rows
  for (int kt = 0; kt < kThinAhead && kt < KT; ++kt) thin_issue(c, a_off_thin, kt, kt);
  for (int kt = 0; kt < KT; ++kt) {
    // Refill the buffer read two stages ago, then wait for stage kt (loads
    // per stage: 3 for waves 0-3, 2 for the others).
    if (kt + kThinAhead < KT) {
      thin_issue(c, a_off_thin, kt + kThinAhead, (kt + kThinAhead) % kThinRing);
      if (c.wave < 4)
        __builtin_amdgcn_s_waitcnt(wait_vm(3 * kThinAhead, false));
      else
        __builtin_amdgcn_s_waitcnt(wait_vm(2 * kThinAhead, false));
    } else {
      __builtin_amdgcn_s_waitcnt(kWaitVm0);
    }
    asm volatile("s_barrier" ::: "memory");
    if (active) {
      const unsigned char* st = c.lds + (kt % kThinRing) * kThinStage;
      const u32x4_t fa = *reinterpret_cast<const u32x4_t*>(st + c.wm * 1024 + c.a_lane);
      u32x4_t fb[8];
#pragma unroll
      for (int n = 0; n < 8; ++n) {
        const int rb = NSETS == 2 ? ((n >> 2) * 8 + c.wn * 4 + (n & 3)) : (c.wn * 8 + n);
        fb[n] = *reinterpret_cast<const u32x4_t*>(st + 4096 + rb * 1024 + c.b_lane);
      }
#pragma unroll
      for (int n = 0; n < 8; ++n) acc[n][0] = mfma16(fb[n], fa, acc[n][0]);
    }
  }
  __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
}

// The bf16 / fp8-activation K loop of a tile with `rows` rows, after its
// prologue loads.  Active 16-row groups of this wave: groups wm, wm+4, wm+8,
// wm+12 below ceil(rows / 16).  Wave-uniform, so each wave runs one
// specialisation; the two ping-pong groups run mirrored loops.
template <int NSETS, bool A8>
__device__ __forceinline__ void run_k_body(const WaveCtx& c, f32x4_t (&acc)[8][4], int rows) {
  const int groups = (rows + 15) >> 4;
  const int nm = groups > c.wm ? min(4, (groups - c.wm + 3) >> 2) : 0;
  if (c.wave < 4) {
    switch (nm) {
      case 4: k_body<4, NSETS, 0, A8>(c, acc); break;
      case 3: k_body<3, NSETS, 0, A8>(c, acc); break;
      case 2: k_body<2, NSETS, 0, A8>(c, acc); break;
      case 1: k_body<1, NSETS, 0, A8>(c, acc); break;
      default: k_body<0, NSETS, 0, A8>(c, acc); break;
    }
  } else {
    switch (nm) {
      case 4: k_body<4, NSETS, 1, A8>(c, acc); break;
      case 3: k_body<3, NSETS, 1, A8>(c, acc); break;
      case 2: k_body<2, NSETS, 1, A8>(c, acc); break;
      case 1: k_body<1, NSETS, 1, A8>(c, acc); break;
      default: k_body<0, NSETS, 1, A8>(c, acc); break;
    }
  }
}

// F8: e4m3 weights.  A8 (with F8): e4m3 activations too, K-blocked in
// 64-input pieces, on the bf16 loop's ring with 64-input stages.  One tile
// per block.
// X2 (with F8 and A8): two-term e4m3 activations on the fp8 weight loop.
template <int EPI, int NSETS, bool F8, bool A8, bool X2 = false>
__global__ __launch_bounds__(kThreads, 1) void gemm_tiled256_kernel(GroupedGemmArgs g, int n_row_tiles,
                                                                     int n_col_tiles) {
  static_assert(!X2 || (F8 && A8), "two-term activations: e4m3 weights and activations");
  extern __shared__ __attribute__((aligned(1024))) unsigned char lds[];

  int col_tile, split;
  TileInfo ti;
  int4 ent = make_int4(-2, 0, 0, 0);
  if (g.tile_table) {
    const int4* tab = reinterpret_cast<const int4*>(g.tile_table);
    ent = tab[1 + blockIdx.x];
    if (ent.x == ttab::kTakeFromPool) {
      // the next tile of the shared pool, or none once it is empty (one
      // device-scope atomic per block past its XCD's own tiles), passed to
      // the block through the first word of the LDS ring before any stage
      // is loaded into it
      int* claim = reinterpret_cast<int*>(lds);
      if (threadIdx.x == 0) *claim = atomicAdd(const_cast<int*>(&tab[0].y), 1);
      __syncthreads();
      const int j = *claim;
      __syncthreads();
      ent = j < tab[0].x ? tab[1 + gridDim.x + j] : make_int4(-1, 0, 0, 0);
    }
  }
  if (ent.x >= 0) {
    ti.expert = __builtin_amdgcn_readfirstlane(ent.x);
    ti.row0 = __builtin_amdgcn_readfirstlane(ent.y);
    ti.rows = __builtin_amdgcn_readfirstlane(ent.z);
    col_tile = __builtin_amdgcn_readfirstlane(ent.w & 0xFFFF);
    split = __builtin_amdgcn_readfirstlane(ent.w >> 16);
  } else if (ent.x == -1) {
    return;
  } else if (g.n_expert <= kSchedExperts && static_cast<int64_t>(n_row_tiles) * n_col_tiles * g.ksplit < INT32_MAX) {
    if (!sched_tile(g, n_col_tiles, &ti, &col_tile, &split)) return;
  } else {
    int row_tile;
    if (!logical_tile(n_row_tiles, n_col_tiles, g.ksplit, &row_tile, &col_tile, &split)) return;
    if (!find_tile(g.offsets, g.n_expert, kBM, row_tile, &ti)) return;
  }

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const WaveCtx c = tile_ctx<NSETS, F8, A8>(g, ti, col_tile, split, lds, lane, wave);
  const int64_t n0 = static_cast<int64_t>(col_tile) * (kBN / NSETS);

  f32x4_t acc[8][4];
#pragma unroll
  for (int n = 0; n < 8; ++n)
#pragma unroll
    for (int m = 0; m < 4; ++m) acc[n][m] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  EpiRows er;
  epi_rows_first<EPI>(g, ti, er);
  if constexpr (F8 && (!A8 || X2)) {
    const int groups = (ti.rows + 15) >> 4;
    const int nm = groups > c.wm ? min(4, (groups - c.wm + 3) >> 2) : 0;
    if (wave < 4) {
      switch (nm) {
        case 4: k_loop_f8<4, NSETS, 0, X2>(c, acc); break;
        case 3: k_loop_f8<3, NSETS, 0, X2>(c, acc); break;
        case 2: k_loop_f8<2, NSETS, 0, X2>(c, acc); break;
        case 1: k_loop_f8<1, NSETS, 0, X2>(c, acc); break;
        default: k_loop_f8<0, NSETS, 0, X2>(c, acc); break;
      }
    } else {
      switch (nm) {
        case 4: k_loop_f8<4, NSETS, 1, X2>(c, acc); break;
        case 3: k_loop_f8<3, NSETS, 1, X2>(c, acc); break;
        case 2: k_loop_f8<2, NSETS, 1, X2>(c, acc); break;
        case 1: k_loop_f8<1, NSETS, 1, X2>(c, acc); break;
        default: k_loop_f8<0, NSETS, 1, X2>(c, acc); break;
      }
    }
  } else {
    if (!A8 && kThin && ti.rows <= kThinRows) {
      const int64_t kb_first = split_boundary(static_cast<int>(g.K / 32), g.ksplit, split, g.ksplit_first64);
      thin_k_loop<NSETS>(c, a_group_offset(g, ti, wave & 3, lane, kb_first), ti.rows, acc);
    } else {
      k_issue_range<NSETS>(c, 0, 4);
      run_k_body<NSETS, A8>(c, acc, ti.rows);
    }
  }
  epi_rows_second<EPI>(g, ti, er);

  if constexpr (EPI == EPI_SWIGLU)
    epilogue<EPI, NSETS, F8, A8, false>(g, ti, split, n0, c.wm, c.wn, lane, lds, acc, er);
  else if (g.out_dtype == DT_F32)
    epilogue<EPI, NSETS, F8, A8, true>(g, ti, split, n0, c.wm, c.wn, lane, lds, acc, er);
  else
    epilogue<EPI, NSETS, F8, A8, false>(g, ti, split, n0, c.wm, c.wn, lane, lds, acc, er);
}

template <int EPI, int NSETS, bool F8, bool A8, bool X2 = false>
hipError_t launch_t(const GroupedGemmArgs& g_in, hipStream_t s) {
  // A table pointer on a GEMM the table does not cover is ignored, and so is
  // one this launcher would have to build itself for a narrow GEMM (its
  // kernel costs about as much as the table gains there).
  GroupedGemmArgs g = g_in;
  g.ksplit_first64 = gemm_tiled256_split_first64(g);
  if (g.tile_table && gemm_tiled256_table_bytes(g) == 0) g.tile_table = nullptr;
  constexpr int lds_bytes = F8 && (!A8 || X2) ? kLdsF8 : kLds;
  static const bool configured = [] {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_tiled256_kernel<EPI, NSETS, F8, A8, X2>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, lds_bytes);
    (void)hipGetLastError();
    return true;
  }();
  (void)configured;
  const int row_tiles = max_row_tiles(g.n_assign, g.n_expert, kBM);
  const int col_tiles = static_cast<int>((g.N + kBN / NSETS - 1) / (kBN / NSETS));
  const int64_t total = static_cast<int64_t>(row_tiles) * col_tiles * g.ksplit;
  unsigned blocks = static_cast<unsigned>((total + 7) / 8 * 8);
  if (g.tile_table && !g.tile_table_ready && col_tiles < kTableMinColsOwn) g.tile_table = nullptr;
  if (g.tile_table) {
    TileTableReq r;
    gemm_tiled256_table_request(g, &r);
    if (!g.tile_table_ready)
      hipLaunchKernelGGL(tile_table_kernel, dim3(1), dim3(perm::kThreads), 0, s, g.offsets, g.n_expert, r);
    blocks = static_cast<unsigned>(8 * (r.bpx + r.steal));
  }
  hipLaunchKernelGGL((gemm_tiled256_kernel<EPI, NSETS, F8, A8, X2>), dim3(blocks), dim3(kThreads), lds_bytes, s, g,
                     row_tiles, col_tiles);
  return hipGetLastError();
}

}  // namespace

int gemm_tiled256_ksplit(const GroupedGemmArgs& g) {
  // Split K in two when the tiles would fill the 256 CUs fewer than ~4 times
  // (the down projection at Mixtral shapes: 4096 outputs, 14336 inputs) and
  // the caller provided room for the partials (fp32 or bf16).
  if (g.epi != EPI_SCATTER_WEIGHTED || g.split_stride == 0) return 1;
  const int row_tiles = max_row_tiles(g.n_assign, g.n_expert, kBM);
  const int64_t tiles = static_cast<int64_t>(row_tiles) * ((g.N + kBN - 1) / kBN);
  // (Three splits were measured too: the extra fp32 partial traffic and
  // per-tile fixed costs outweigh the shorter last round.)
  if (tiles < 1024 && g.K % (4 * kBK) == 0 && g.K >= 2048) return 2;
  return 1;
}

bool gemm_tiled256_table_request(const GroupedGemmArgs& g, TileTableReq* r) {
  const int nsets = g.epi == EPI_SWIGLU ? 2 : 1;
  const int col_tiles = static_cast<int>((g.N + kBN / nsets - 1) / (kBN / nsets));
  const int ksplit = gemm_tiled256_ksplit(g);
  const int64_t chunks = ttab::n_chunks(col_tiles, ksplit, g.n_expert);
  // Measured: with many column tiles (Mixtral's gate/up, 112) the table
  // deals the work better (gate/up 1.47-1.48 -> 1.45 ms at T=4096); with
  // Qwen3's 6 and 8 it was 4-13% slower and the equal-count ranges in the
  // kernel are kept.
  if (col_tiles < kTableMinCols || g.n_assign <= 0) return false;
  if (g.n_expert <= 0 || g.n_expert > kSchedExperts || g.n_expert > ttab::kMaxExperts || chunks > ttab::kChunks ||
      col_tiles >= (1 << 16))
    return false;
  const int row_tiles = max_row_tiles(g.n_assign, g.n_expert, kBM);
  if (r) {
    r->table = g.tile_table;
    r->n_col = col_tiles;
    r->ksplit = ksplit;
    r->bpx = ttab::blocks_per_xcd(row_tiles, col_tiles, ksplit);
    // The shared pool (tile_table.h) for the down projection only.  The
    // XCDs run the same tiles 3-4% apart (per-block stamps at C2 T=4096:
    // full gate/up tiles 88.5-94.6 us, down 155-163 us by XCD); taking the
    // tail of each XCD's list from a pool measured, per call over 6 x 30
    // calls: down 730.6 -> 720.3 us at C2 T=4096 and 714.9 -> 694.9 us at
    // C5 T=4096; on the gate/up projection, whose tiles share more of their
    // stages in L2, no gain (1464.5 -> 1472.6 us at C2).
    r->steal = g.epi == EPI_SWIGLU ? 0 : ttab::steal_per_xcd(r->bpx);
    r->kblocks = static_cast<int>(g.K / (g.w_dtype == DT_F8 ? 64 : 32));
    r->ksplit_first64 = gemm_tiled256_split_first64(g);
  }
  return true;
}

// The two pieces of a K-split tile are dealt as separate blocks.  When the
// launch runs many rounds of blocks per CU (at least 4.5: Mixtral's down
// projection at 4096 tokens, 35 row tiles x 16 columns x 2 pieces over 256
// CUs), a short first piece (12/64 of K) and a long second one leave short
// blocks to fill the last round: measured C2 T=4096 down 731 -> 711 us, C5
// T=4096 707 -> 700 us (e4m3 activations 372 -> 359 us), medians of three
// interleaved rounds.  A list-scheduling replay of the measured tile costs
// gave the same optimum (8.9% -> 4.1% idle CU time).  With fewer rounds the
// split is there to fill the CUs, and equal pieces keep the longest block
// short (C2 T=512: 170 us against 229 us with 12/64).
int gemm_tiled256_split_first64(const GroupedGemmArgs& g) {
  if (gemm_tiled256_ksplit(g) != 2) return 32;
  const int row_tiles = max_row_tiles(g.n_assign, g.n_expert, kBM);
  const int64_t blocks = static_cast<int64_t>(row_tiles) * ((g.N + kBN - 1) / kBN) * 2;
  return blocks * 2 >= 9 * 256 ? 12 : 32;
}

size_t gemm_tiled256_table_bytes(const GroupedGemmArgs& g) {
  TileTableReq r;
  if (!gemm_tiled256_table_request(g, &r)) return 0;
  return (1 + static_cast<size_t>(8) * (r.bpx + r.steal) + static_cast<size_t>(4) * r.steal) * 16;
}

bool gemm_tiled256_supported(const GroupedGemmArgs& g) {
  const bool a8 = g.act_dtype == DT_F8;
  if ((g.act_dtype != DT_BF16 && !a8) || (g.w_dtype != DT_BF16 && g.w_dtype != DT_F8) || g.w_format != WF_MFMA16)
    return false;
  // fp8 activations: fp8 weights, K-blocked A with per-row scales, an even
  // number of 64-input stages per split
  if (a8 && (g.w_dtype != DT_F8 || !g.a_kb_rows || !g.a_scale || g.K % 128 || g.K / 128 < 2 * g.ksplit))
    return false;
  // two-term activations: the lo codes a whole plane (K * a_kb_rows bytes or
  // more) after the hi codes, 16-byte aligned, both within 32-bit offsets
  if (g.a_lo_plane && (!a8 || g.a_lo_plane < g.K * g.a_kb_rows || g.a_lo_plane % 16 ||
                       g.a_lo_plane + g.K * g.a_kb_rows >= (int64_t(1) << 32)))
    return false;
  if (!g.order || !g.offsets || g.epi > EPI_SCATTER_WEIGHTED) return false;
  // bf16: an even number of 32-input stages per split; fp8: whole 64-input
  // blocks; at least two stages per split.
  if (g.K <= 0 || g.K % (2 * kBK) || g.K / (2 * kBK) < 2 * g.ksplit || g.N % 16 || g.lda % 8 || g.ldo % 4)
    return false;
  // the epilogue stores 16-byte chunks: 8 bf16 or 4 fp32 outputs
  const bool out_f32 = g.epi != EPI_SWIGLU && g.out_dtype == DT_F32;
  if ((!out_f32 && (g.ldo % 8 || g.split_stride % 8)) || (out_f32 && g.split_stride % 4)) return false;
  if (g.w_dtype == DT_F8 && (!g.s0 || (g.epi == EPI_SWIGLU && !g.s1))) return false;
  // 32-bit byte offsets of A rows
  const int64_t a_rows = g.a_mode == A_GATHER_TOKEN ? g.n_tokens : g.n_assign;
  if (a_rows * g.lda * 2 >= (int64_t(1) << 32)) return false;
  // K-blocked A: expert-sorted rows (A_DIRECT), all of them inside the blocks
  if (g.a_kb_rows && (g.a_mode != A_DIRECT || g.a_kb_rows < g.n_assign || g.K % 32 ||
                      g.K * g.a_kb_rows * 2 >= (int64_t(1) << 32)))
    return false;
  // K-blocked SwiGLU output: whole 32-column blocks, rows p < out_kb_rows
  if (g.out_kb_rows && (g.epi != EPI_SWIGLU || g.out_kb_rows < g.n_assign || g.N % 32)) return false;
  if (g.epi == EPI_SWIGLU && (g.out_dtype != DT_BF16 || !g.w1)) return false;
  if (reinterpret_cast<uintptr_t>(g.a) % 16 || reinterpret_cast<uintptr_t>(g.out) % 16) return false;
  return true;
}

hipError_t launch_gemm_tiled256(const GroupedGemmArgs& g, hipStream_t s) {
  if (!gemm_tiled256_supported(g)) return hipErrorNotSupported;
  if (g.n_assign == 0 || g.N == 0) return hipSuccess;
  const bool f8 = g.w_dtype == DT_F8;
  if (g.act_dtype == DT_F8 && g.a_lo_plane) {
    if (g.epi == EPI_SWIGLU) return launch_t<EPI_SWIGLU, 2, true, true, true>(g, s);
    if (g.epi == EPI_SCATTER_WEIGHTED) return launch_t<EPI_SCATTER_WEIGHTED, 1, true, true, true>(g, s);
    return launch_t<EPI_SCATTER, 1, true, true, true>(g, s);
  }
  if (g.act_dtype == DT_F8) {
    if (g.epi == EPI_SWIGLU) return launch_t<EPI_SWIGLU, 2, true, true>(g, s);
    if (g.epi == EPI_SCATTER_WEIGHTED) return launch_t<EPI_SCATTER_WEIGHTED, 1, true, true>(g, s);
    return launch_t<EPI_SCATTER, 1, true, true>(g, s);
  }
  if (g.epi == EPI_SWIGLU)
    return f8 ? launch_t<EPI_SWIGLU, 2, true, false>(g, s) : launch_t<EPI_SWIGLU, 2, false, false>(g, s);
  if (g.epi == EPI_SCATTER_WEIGHTED)
    return f8 ? launch_t<EPI_SCATTER_WEIGHTED, 1, true, false>(g, s)
              : launch_t<EPI_SCATTER_WEIGHTED, 1, false, false>(g, s);
  return f8 ? launch_t<EPI_SCATTER, 1, true, false>(g, s) : launch_t<EPI_SCATTER, 1, false, false>(g, s);
}

}  // namespace fmoe
