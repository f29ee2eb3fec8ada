// Host-side launchers of the gfx950 kernels (internal to libfmoe.so).
#pragma once

#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>

namespace fmoe {

// Element types; values match fmoe_dtype in include/fmoe.h.
enum DType { DT_F32 = 0, DT_BF16 = 1, DT_F8 = 2 };

inline size_t dtype_bytes(int dt) { return dt == DT_F32 ? 4 : dt == DT_BF16 ? 2 : 1; }

// Packed expert-weight layouts.  The layout is a function of (n_out, n_in,
// dtype) only, so producer and consumers agree without carrying a tag.
//
// WF_ROWMAJOR: per expert [n_out][n_in], n_in contiguous.
// WF_MFMA16:   per expert, blocks of 16 output rows x KB inputs (KB = 32 for
//   bf16, 64 for fp8), blocks ordered [row block][input block], each block
//   1 KiB = 64 lanes x 16 bytes in the operand order of
//   v_mfma_f32_16x16x32_bf16: lane l holds rows (l % 16) and inputs
//   8*(l / 16) .. +8 of a 32-input step.  fp8 lanes hold two such steps
//   (inputs q and 32+q at bytes q%8 and 8+q%8).  A wave loads one block with
//   one fully coalesced 16-byte-per-lane load, ready for the MFMA.
enum WFormat { WF_ROWMAJOR = 0, WF_MFMA16 = 1 };

__host__ __device__ inline int packed_format(int64_t n_out, int64_t n_in, int dtype) {
  if (dtype == DT_BF16 && n_out % 16 == 0 && n_in % 32 == 0) return WF_MFMA16;
  if (dtype == DT_F8 && n_out % 16 == 0 && n_in % 64 == 0) return WF_MFMA16;
  return WF_ROWMAJOR;
}

// Packed buffers end with a tail of kPackedTailRows rows x n_in inputs (at
// the widest element size) that tiled kernels may read past the last expert
// instead of guarding partial column tiles; its contents are never used.
constexpr int64_t kPackedTailRows = 256;

// Element offset of weight (e, n, k) in a packed buffer of n_out = N, n_in = K.
__host__ __device__ inline int64_t packed_offset(int fmt, int dtype, int64_t e, int64_t n, int64_t k,
                                                 int64_t N, int64_t K) {
  if (fmt == WF_ROWMAJOR) return (e * N + n) * K + k;
  if (dtype == DT_BF16) {
    const int64_t blk = (e * (N / 16) + n / 16) * (K / 32) + k / 32;
    const int64_t lane = (n % 16) + 16 * ((k % 32) / 8);
    return blk * 512 + lane * 8 + k % 8;
  }
  const int64_t blk = (e * (N / 16) + n / 16) * (K / 64) + k / 64;
  const int64_t kk = k % 64;
  const int64_t q = kk % 32;
  const int64_t lane = (n % 16) + 16 * (q / 8);
  return blk * 1024 + lane * 16 + (kk / 32) * 8 + q % 8;
}

// How a grouped GEMM finds row p's A operand.
enum AMode {
  A_GATHER_TOKEN = 0,  // row order[p] % n_tokens of `a` (x rows, per token)
  A_GATHER_FLAT = 1,   // row order[p] of `a` (flat slot-major assignment rows)
  A_DIRECT = 2         // row p of `a` (rows already in expert-sorted order)
};

// What a grouped GEMM does with its fp32 accumulators.
enum Epilogue {
  EPI_SWIGLU = 0,            // out[p, n] = g * silu(u) from the two weight sets
  EPI_SCATTER = 1,           // out[order[p], n] = acc
  EPI_SCATTER_WEIGHTED = 2,  // out[order[p], n] = acc * route_w[order[p]]
  // One-expert projections on the streaming kernel (bf16 activations, no K
  // split), with the fields of ProjEpilogue:
  EPI_LINEAR = 3,            // out[p, n] = bf16(acc + bias[n]) (+ residual[p, n])
  EPI_QKV_ROPE = 4           // bias, then RoPE on the q and k columns -> q_out / k_out / v_out
};

// The epilogue of a fused projection (EPI_LINEAR / EPI_QKV_ROPE).
struct ProjEpilogue {
  int kind = EPI_LINEAR;
  const float* bias = nullptr;      // EPI_LINEAR: [N]; EPI_QKV_ROPE: q bias [nq] (or null)
  const float* bias_k = nullptr;    // EPI_QKV_ROPE: [nkv] (or null)
  const float* bias_v = nullptr;    // EPI_QKV_ROPE: [nkv] (or null)
  const void* residual = nullptr;   // EPI_LINEAR: [rows, N] bf16 added after rounding; may alias out
  void* out = nullptr;              // EPI_LINEAR: [rows, N] bf16
  const int64_t* positions = nullptr;  // EPI_QKV_ROPE: [rows]
  int nq = 0, nkv = 0, head_dim = 0;   // EPI_QKV_ROPE: N = nq + 2 nkv, columns q | k | v
  double freq_base = 10000.0, freq_scale = 1.0;
  float* q_out = nullptr;           // [rows, nq] fp32
  void* k_out = nullptr;            // [rows, nkv] bf16, RoPE applied
  void* v_out = nullptr;            // [rows, nkv] bf16
};

// Routing computed inside the streaming gate/up GEMM of decode batches of
// at most 4 tokens (launch_router_split_logits wrote the partial logits):
// every block sums the n_split partials, runs the router's softmax + top-k
// (the same code as router_topk_permute_wave_kernel, so the same ids and
// weights) and takes the expert of its block row; block 0 also stores ids,
// weights, the grouping (order, offsets) and the invalid-id count (0) for
// the launches that follow, which no block of the GEMM reads.  nv: experts
// per row lane of the top-k (n_expert <= 16 nv; 1, 4 or 8).
struct RoutePrologue {
  const float* part = nullptr;  // [n_split][n_tokens][n_expert]; nullptr: no routing here
  int n_split = 0;
  int k = 0;
  int normalize = 0;
  int nv = 0;
  int* ids = nullptr;           // [k][n_tokens]
  float* weights = nullptr;     // [k][n_tokens]
  int* order = nullptr;         // [k * n_tokens]
  int* offsets = nullptr;       // [n_expert + 1]
  int* err_count = nullptr;
};

struct GroupedGemmArgs {
  const void* a = nullptr;      // A operand base, act_dtype
  int64_t lda = 0;              // elements between A rows
  int a_mode = A_DIRECT;
  const int* order = nullptr;   // [n_assign] expert-sorted flat assignment ids
  const int* offsets = nullptr; // [n_expert + 1]
  // The streaming kernel also takes order == offsets == nullptr for one
  // expert and the identity grouping (rows 0..n_assign-1 in order).
  int n_tokens = 0;
  int n_assign = 0;             // k * n_tokens
  int n_expert = 0;
  const void* w0 = nullptr;     // packed weights [E][N][K] (gate, or the only set)
  const void* w1 = nullptr;     // packed up weights for EPI_SWIGLU
  const float* s0 = nullptr;    // [E][N] scales for fp8 weights
  const float* s1 = nullptr;
  int64_t N = 0, K = 0;
  void* out = nullptr;
  int64_t ldo = 0;              // elements between output rows
  int epi = EPI_SCATTER;
  const float* route_w = nullptr;  // [n_assign] routing weight per flat assignment
  int act_dtype = DT_F32;       // A operand type
  int w_dtype = DT_F32;
  int w_format = WF_ROWMAJOR;   // packed_format(N, K, w_dtype)
  int out_dtype = DT_F32;
  // Split of K over ksplit partial products written to out + s * split_stride
  // (s < ksplit).  The 256-tile kernel splits on its own (launchers report
  // the split they used); the streaming kernel splits when the caller sets
  // ksplit (one weight set, fp32 scatter output).
  int ksplit = 1;
  int64_t split_stride = 0;
  // 256-tile kernel with ksplit == 2: the first piece covers this many 64ths
  // of the K stages (set by its launcher).
  int ksplit_first64 = 32;
  // Upper bound on any expert's row count when the caller knows one (the
  // block: n_tokens, since top-k picks distinct experts per token); 0 =
  // unknown.  A tuning hint: kernels are correct for any count.
  int max_rows_per_expert = 0;
  // K-blocked operands (256-tile kernel only): with a_kb_rows > 0 the A
  // operand (A_DIRECT) is stored as 64-byte row pieces, piece j of row r at
  // byte ((j * a_kb_rows) + r) * 64 (j = input block of 32 bf16), so one
  // 32-input stage of a row tile is one contiguous run and every fetched
  // cache line is used whole.  With out_kb_rows > 0 the SwiGLU epilogue
  // writes its output in that layout (out_kb_rows rows per piece column).
  int64_t a_kb_rows = 0;
  int64_t out_kb_rows = 0;
  // act_dtype DT_F8 (256-tile kernel, DT_F8 weights): the A operand is e4m3
  // codes, K-blocked in 64-input pieces whose 16-byte chunk g holds inputs
  // 8g..8g+7 and 32+8g..32+8g+7 of the piece (the packed fp8 weights' lane
  // order), each row p dequantised by a_scale[p].
  const float* a_scale = nullptr;
  // DT_F8 activations as two e4m3 terms per input (hi = e4m3(v), lo =
  // e4m3(v - hi), one scale per row): the lo codes sit a_lo_plane bytes
  // after the hi codes, in the same layout (0: one term).
  int64_t a_lo_plane = 0;
  // SwiGLU epilogue with fp8 activations: atomic max, per output row p, of
  // the bit patterns of |h| (h rounded to bf16, so non-negative floats order
  // as unsigned integers) into row_amax[p], which starts at zero.
  unsigned* row_amax = nullptr;
  // 256-tile kernel: workspace of gemm_tiled256_table_bytes(g) bytes for a
  // per-launch tile schedule; nullptr, or a shape the table does not cover,
  // keeps the in-kernel one.  tile_table_ready: the permutation that wrote
  // the offsets built the table too (launch_permute's tables); otherwise the
  // launcher builds it with a one-block kernel first (wide GEMMs only).
  int* tile_table = nullptr;
  bool tile_table_ready = false;
  ProjEpilogue pe;              // EPI_LINEAR / EPI_QKV_ROPE only
  RoutePrologue rp;             // streaming gate/up GEMM of decode batches only
};

// Element offset of (row, col) in a K-blocked bf16 matrix of `rows` rows.
__host__ __device__ inline int64_t kb_offset(int64_t row, int64_t col, int64_t rows) {
  return ((col >> 5) * rows + row) * 32 + (col & 31);
}

// Upper bound on the number of bm-row tiles of a grouping of n_assign rows
// over n_expert experts.
inline int max_row_tiles(int n_assign, int n_expert, int bm) {
  const int e = n_assign < n_expert ? n_assign : n_expert;
  return n_assign / bm + e;
}

hipError_t launch_router(const void* x, const void* wr, int n_tokens, int n_embd,
                         int n_expert, int k, bool normalize, int dtype, int* ids,
                         float* weights, hipStream_t stream);

// Decode-sized batches (bf16, n_tokens <= kDecodeMaxTokens, n_expert <= 256,
// k <= 16): router logits split over many blocks into `part`
// (router_decode_scratch_bytes, 0 when the shape does not qualify), then one
// block runs softmax + top-k and the permutation (ids, weights, order,
// offsets, err_count as launch_router + launch_permute write them); above 64
// experts and 32 tokens the top-k runs over blocks and the permutation as a
// launch of its own.
// hipErrorNotSupported when the inputs do not qualify.
constexpr int kDecodeMaxTokens = 64;
size_t router_decode_scratch_bytes(int n_tokens, int n_embd, int n_expert, int k, int dtype);
hipError_t launch_router_decode(const void* x, const void* wr, int n_tokens, int n_embd, int n_expert, int k,
                                bool normalize, int dtype, float* part, int* ids, float* weights, int* order,
                                int* offsets, int* err_count, hipStream_t stream);
// The first of those launches alone (the split partial logits into part,
// n_split_out = their count), for callers that run the top-k themselves
// (RoutePrologue).  hipErrorNotSupported when the inputs do not qualify.
hipError_t launch_router_split_logits(const void* x, const void* wr, int n_tokens, int n_embd, int n_expert, int k,
                                      int dtype, float* part, int* n_split_out, hipStream_t stream);
// The column splits launch_router_split_logits uses for n_embd inputs.
int router_decode_splits(int n_embd);

// Prefill batches (bf16, n_tokens > kDecodeMaxTokens, 32 < n_expert <= 128,
// n_embd % 128 == 0, k <= 16): router logits over 64-token tiles and
// ranges of the hidden axis into `part` (router_prefill_scratch_bytes, 0
// when the shape does not qualify), then softmax + top-k summing the ranges
// in order (ids, weights as launch_router writes them).
// hipErrorNotSupported when the inputs do not qualify.
size_t router_prefill_scratch_bytes(int n_tokens, int n_embd, int n_expert, int k, int dtype);
hipError_t launch_router_prefill(const void* x, const void* wr, int n_tokens, int n_embd, int n_expert, int k,
                                 bool normalize, int dtype, float* part, int* ids, float* weights,
                                 hipStream_t stream);

// A 256-tile GEMM's tile schedule for the permutation to build beside its
// scatter (gemm_tiled256_table_request fills it).  Table: a header int4
// {pool size, claim counter, 0, 0}, one int4 entry per hardware block
// (8 * (bpx + steal) of them), then the shared pool (up to 4 * steal).
struct TileTableReq {
  int* table = nullptr;
  int n_col = 0, ksplit = 1, bpx = 0;
  int steal = 0;            // blocks per XCD beyond bpx that take their tile from the pool
  int kblocks = 0;          // K stages of a whole tile
  int ksplit_first64 = 32;  // with ksplit == 2: the first piece's share in 64ths
};
constexpr int kPermuteMaxTables = 2;

// Batches above kPermuteChunk assignments run chunked, with a histogram
// scratch of permute_scratch_bytes() (0 for smaller batches).  Up to
// kPermuteMaxTables tile schedules over the resulting offsets are built by
// extra blocks of the same launch.
constexpr int kPermuteChunk = 2048;
size_t permute_scratch_bytes(int n_assign, int n_expert);
hipError_t launch_permute(const int* ids, int n_assign, int n_expert, int* order,
                          int* offsets, int* err_count, int* scratch, hipStream_t stream,
                          const TileTableReq* tables = nullptr, int n_tables = 0);

hipError_t launch_pack(const void* src, int src_dtype, const float* src_scales,
                       int n_out, int n_in, int n_expert, int dst_dtype, void* dst,
                       float* dst_scales, hipStream_t stream);

hipError_t launch_gemm_generic(const GroupedGemmArgs& g, hipStream_t stream);
// Returns hipErrorNotSupported when the shape or dtype is outside what the
// MFMA kernels handle; the caller then uses the generic kernel.
enum TiledVariant { TILED_AUTO = 0, TILED_128 = 1, TILED_256 = 2 };
// The tiled kernel that `variant` resolves to for g (TILED_AUTO picks the
// 256x256-tile kernel wherever it applies), or -1 if none applies.
int resolve_tiled_variant(const GroupedGemmArgs& g, int variant);
hipError_t launch_gemm_tiled(const GroupedGemmArgs& g, hipStream_t stream, int variant);
hipError_t launch_gemm_stream(const GroupedGemmArgs& g, hipStream_t stream);
// The block's down projection (d: EPI_SCATTER_WEIGHTED, fp32 per-slot rows,
// streaming-kernel operands) fused with the combine for decode batches of
// n_tokens * k <= 16 assignments: out (bf16 [n_tokens, d.N]) = [residual +]
// the slot-ordered sum, bit-identical to launch_gemm_stream(d) followed by
// launch_combine.  d.out is not written.  hipErrorNotSupported when the
// batch or operands do not qualify (the caller then launches the two).
hipError_t launch_down_combine_small(const GroupedGemmArgs& d, const void* residual, void* out, int out_dtype,
                                     int n_tokens, int k, hipStream_t stream);
bool gemm_tiled_supported(const GroupedGemmArgs& g);
bool gemm_stream_supported(const GroupedGemmArgs& g);
// Whether the streaming gate/up GEMM takes g with its routing (g.rp set):
// the shape qualifies and the grid fits one round of resident blocks.
bool gemm_stream_routed_ok(const GroupedGemmArgs& g);
// 256x256-tile bf16 kernel (gemm_tiled256.hip); launch_gemm_tiled uses it
// when it applies.
bool gemm_tiled256_supported(const GroupedGemmArgs& g);
hipError_t launch_gemm_tiled256(const GroupedGemmArgs& g, hipStream_t stream);
// K split the 256-tile kernel would use for g (1 when it does not apply).
int gemm_tiled256_ksplit(const GroupedGemmArgs& g);
// The tile schedule g would use (false: none; the shape keeps the in-kernel
// one), with r->table = g.tile_table; and its size in bytes (0: none).
bool gemm_tiled256_table_request(const GroupedGemmArgs& g, TileTableReq* r);
size_t gemm_tiled256_table_bytes(const GroupedGemmArgs& g);
// With a two-way K split: the first piece's share of the K stages, in 64ths.
int gemm_tiled256_split_first64(const GroupedGemmArgs& g);

hipError_t launch_swiglu(const void* gate, const void* up, void* out, int64_t n,
                         int dtype, hipStream_t stream);
// out[t, :] = [residual[t, :] +] sum over s = 0..k-1 (in order) of the
// K-split sum (y_0 + y_1 + ...)[s*n_tokens + t, :], partials split_stride
// elements apart; residual (out_dtype) may be null.
hipError_t launch_combine(const void* y, int y_dtype, const void* residual, void* out, int out_dtype,
                          int n_tokens, int k, int n_embd, int nsplit, int64_t split_stride,
                          hipStream_t stream);
// out[r, :] = (x[r, :] / sqrt(mean(x[r, :]^2) + eps)) * weight, fp32 arithmetic.
hipError_t launch_rms_norm(const void* x, const void* weight, float eps, void* out, int64_t n_rows,
                           int n_embd, int dtype, hipStream_t stream);
// out[c, r] = in[r, c] for an in[rows, cols] matrix (same dtype).
hipError_t launch_transpose(const void* in, void* out, int64_t rows, int64_t cols,
                            int dtype, hipStream_t stream);
// Zero rows f of y[n_assign, width] whose id is outside [0, n_expert).
hipError_t launch_zero_invalid_rows(const int* ids, int n_assign, int n_expert,
                                    void* y, int dtype, int64_t width,
                                    hipStream_t stream);
hipError_t launch_fill_zero(void* p, size_t bytes, hipStream_t stream);
// Rows of src [*, n_cols] bf16 (row p = src row order[p] % n_tokens, or row p
// when order is null), quantised to e4m3 with one scale per row: scale[p] =
// the smallest power of two 2^e with max|row| / 2^e <= 448 (e clamped to
// [-126, 126]; 1 for an all-zero row), code = RNE(v * 2^-e) saturating at
// 448, written K-blocked in 64-input pieces (piece j
// of row p at byte (j * n_rows + p) * 64, 16-byte chunk g holding inputs
// 64j + 8g + [0, 8) then 64j + 32 + 8g + [0, 8)).  n_cols % 64 == 0 and
// n_cols <= 16384.
// row_amax (may be null): max|v| of each source row as float bits, indexed
// like src (then the rows are read once); zero_out (may be null): n_rows
// words set to zero.  With dst_lo, each scaled value v is carried as two
// terms: dst_q holds hi = e4m3(v), dst_lo (same layout) lo = e4m3(v - hi).
// launch_row_absmax: amax_out[r] = max|src[r, :]| (float bits) for src
// [n_rows, n_cols] bf16, n_cols % 8 == 0; also clears zero_out[0, n_zero).
hipError_t launch_quantize_rows_kb(const void* src, const int* order, int n_rows, int n_tokens, int n_cols,
                                   const unsigned* row_amax, void* dst_q, float* dst_scale, unsigned* zero_out,
                                   hipStream_t stream, void* dst_lo = nullptr);
hipError_t launch_row_absmax(const void* src, int n_rows, int n_cols, unsigned* amax_out, unsigned* zero_out,
                             int n_zero, hipStream_t stream);
// dst (K-blocked, kb_offset with n_rows rows) row p = src row order[p] % n_tokens
// (src [n_tokens, n_cols] row-major bf16, n_cols % 32 == 0): the gate/up
// GEMM's A operand gathered into expert-sorted order.
hipError_t launch_gather_rows_kb(const void* src, const int* order, int n_rows, int n_tokens, int n_cols, void* dst,
                                 hipStream_t stream);

// Device address of the allocation-free entry point's scratch array
// (FMOE_NOALLOC_SCRATCH_BYTES, noalloc.hip) on `device`, which must be the
// current device; looked up on first use and cached per device.
hipError_t noalloc_scratch(int device, void** ptr);

// Dense src [n_in, n_part] (x @ W layout; F32 or BF16) -> rows [row0,
// row0 + n_part) of the one-expert packed weight [n_total, n_in] (pack.hip).
hipError_t launch_pack_linear(const void* src, int src_dtype, int n_in, int n_part, int row0, int n_total,
                              int dst_dtype, void* dst, float* dst_scales, hipStream_t stream);

// ---- decode attention (attention.hip)
// Paged pools [n_blocks, block_size, n_head_kv, head_dim]; rows are copied
// as 32-bit words (row_bytes a multiple of 4).  Table entries outside the
// pool read as zero rows (gather) or skip the write (scatters).
hipError_t launch_kv_gather(const void* cache, int64_t n_blocks, int block_size, int row_bytes, const int* tables,
                            int max_blocks, const int* ctx_lens, int max_ctx, int batch, void* out, hipStream_t s);
hipError_t launch_kv_scatter_decode(void* cache, int64_t n_blocks, int block_size, int row_bytes, const void* vals,
                                    const int* block_idx, const int* pos_idx, int batch, hipStream_t s);
// Where the decode step writes its new K/V rows (row b of k_new / v_new into
// slot (block_idx[b], pos_idx[b]) of each pool): done by launch_attn_decode
// once the pools have been read.
struct KvScatterDecode {
  void* k_cache = nullptr;
  void* v_cache = nullptr;
  int64_t n_blocks = 0;
  int block_size = 0;
  int row_bytes = 0;
  const int* block_idx = nullptr;
  const int* pos_idx = nullptr;
};
hipError_t launch_kv_scatter_prefill(void* cache, int64_t n_blocks, int block_size, int row_bytes, const void* vals,
                                     int seq_len, const int* tables, int max_blocks, const int* start, int batch,
                                     hipStream_t s);
// v[i] = i for i < n; pair = {pair0, pair1} when non-null.
hipError_t launch_iota(int* v, int n, int* pair, int pair0, int pair1, hipStream_t s);
hipError_t launch_fill_int(int* v, int n, int value, hipStream_t s);
// qkv [B, nq + 2 nkv] fp32 -> bias (optional), RoPE on q and k:
// q_rot fp32 [B, nq], k_new / v_new [B, nkv] in act dtype.
// qkv holds nsplit partial sums split_stride floats apart, added in order.
hipError_t launch_qkv_rope(const float* qkv, int nsplit, int64_t split_stride, const float* bq, const float* bk,
                           const float* bv, const int64_t* positions, int batch, int nq, int nkv, int head_dim,
                           double freq_base, double freq_scale, float* q_rot, void* k_new, void* v_new, int act,
                           hipStream_t s);
// out[r, :] = sum of the nsplit partials y[r, :] (+ bias) in act dtype,
// then + residual[r, :] (optional; out may alias it).
hipError_t launch_bias_cast(const float* y, int nsplit, int64_t split_stride, const float* bias, const void* residual,
                            void* out, int64_t rows, int n, int act, hipStream_t s);
// Head sizes and query-per-KV-head groups the attention kernels take.
bool attn_decode_supported(int head_dim, int group);
// Context splits of the attention (part holds batch * n_head * splits *
// (head_dim + 2) floats).
int attn_decode_splits(int max_ctx);
// One new token per sequence against max_ctx positions of the paged pools
// (zero rows at and past ctx_lens[b]) and its own k_new / v_new; out
// [B, n_head * head_dim] in dtype (the pools' and k_new / v_new's dtype).
// With `scatter` non-null the combine launch also writes k_new / v_new into
// the pools it names (after the split kernel has read them).
hipError_t launch_attn_decode(const float* q_rot, const void* k_pool, const void* v_pool, int64_t n_blocks,
                              int block_size, const int* tables, int max_blocks, const int* ctx_lens, int max_ctx,
                              const void* k_new, const void* v_new, int batch, int n_head, int n_head_kv,
                              int head_dim, int dtype, float scale, float* part, void* out, hipStream_t s,
                              const KvScatterDecode* scatter = nullptr);

}  // namespace fmoe
