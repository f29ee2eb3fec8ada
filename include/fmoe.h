/*
 * fmoe.h -- C ABI of the MI355X (gfx950) MoE FFN hot path.
 *
 * Drop-in for the reference's MoE FFN functions (stellaraccident/frank-models):
 *   moe_ffn_block  components/moe/moe_ffn_block.mlir:34-209, oracles/moe.py:51-132
 *   mul_mat_id     components/moe/mul_mat_id.mlir:22-120,   oracles/moe.py:9-48
 *   swiglu         components/activation/swiglu.mlir:16-51, oracles/activation.py:11-21
 * and the layer glue around the block:
 *   rms_norm       components/normalization/rms_norm.mlir:18-85, oracles/normalization.py:10-43
 *   MoE FFN sub-layer (ffn_norm -> moe_ffn_block -> residual add)
 *                  architectures/llm/transformer_layer_moe_prefill.mlir:205-242,
 *                  transformer_layer_moe_decode.mlir:227-255
 *
 * Conventions
 *   - Every pointer is a device pointer unless stated otherwise; every call is
 *     asynchronous on `stream` (a hipStream_t; NULL = the null stream) unless
 *     stated otherwise.
 *   - Tensor layouts are the reference's, row-major (C-contiguous):
 *       input  [n_tokens, n_embd]                 (moe_ffn_block.mlir:35)
 *       router [n_expert, n_embd]                 (moe_ffn_block.mlir:36)
 *       up/gate expert weights [n_ff, n_embd, n_expert]  (moe_ffn_block.mlir:37-38)
 *       down expert weights    [n_embd, n_ff, n_expert]  (moe_ffn_block.mlir:39)
 *       ids / routing weights  [n_expert_used, n_tokens] (moe_ffn_block.mlir:78-81)
 *     Expert weights are packed once (fmoe_pack_expert_weights) into the
 *     per-expert layout the kernels read; the block and mul_mat_id take the
 *     packed form.
 *   - The caller owns every buffer, including the workspace; the library
 *     never allocates or frees device memory.
 *   - Functions return an fmoe_status; on failure fmoe_last_error() gives a
 *     thread-local message.  No C++ exception crosses this boundary.
 */
#ifndef FMOE_H_
#define FMOE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum fmoe_status {
  FMOE_OK = 0,
  FMOE_ERR_INVALID_ARGUMENT = 1, /* null / misaligned pointer, bad flag */
  FMOE_ERR_SHAPE = 2,            /* a dimension out of range */
  FMOE_ERR_DTYPE = 3,            /* unsupported dtype or dtype combination */
  FMOE_ERR_IDS_RANGE = 4,        /* an expert id outside [0, n_expert) */
  FMOE_ERR_NO_DEVICE = 5,        /* no usable gfx950 device */
  FMOE_ERR_HIP = 6,              /* a HIP runtime call or launch failed */
  FMOE_ERR_WORKSPACE = 7         /* workspace missing or too small */
} fmoe_status;

typedef enum fmoe_dtype {
  FMOE_F32 = 0,      /* IEEE binary32 */
  FMOE_BF16 = 1,     /* bfloat16 */
  FMOE_F8E4M3FN = 2, /* OCP FP8 E4M3 (finite, NaN = 0x7F/0xFF), weights only,
                        with float32 per-output-channel scales [n_expert, n_out] */
  FMOE_F8E4M3FN_A8 = 3, /* block and sub-layer weight dtype only: FMOE_F8E4M3FN
                        weights (the same packed buffers and scales) whose
                        prefill-sized GEMMs also quantise their activations to
                        e4m3, one power-of-two scale per row (the smallest 2^e
                        with max|row| / 2^e <= 448), and run on the fp8 MFMA
                        with fp32 accumulation; decode-sized
                        batches keep bf16 activations.  Adds the activations'
                        e4m3 rounding (about 4.7% relative Frobenius error on
                        Mixtral shapes) to the FMOE_F8E4M3FN result. */
  FMOE_F8E4M3FN_A8X2 = 4 /* as FMOE_F8E4M3FN_A8, with each activation carried
                        as two e4m3 terms under its row's scale, hi = e4m3(v)
                        and lo = e4m3(v - hi), one fp8 MFMA over w * hi + w * lo:
                        every bf16 activation whose scaled magnitude is at least
                        2^-2 is represented exactly, so the result holds the
                        FMOE_F8E4M3FN tolerance (within rounding of the bf16
                        path) while the products run on the fp8 MFMA, at the
                        MFMA time of the bf16 path (two terms per input). */
} fmoe_dtype;

/* Message describing the last failure on this thread ("" if none). */
const char *fmoe_last_error(void);

/* ABI version of this header (bumped on any change to the declarations).
 * 2: the kernel-path override (fmoe_set_gemm_path and its enum) moved to
 *    fmoe_diag.h; FMOE_TIMER_QUANT added (FMOE_TIMER_COUNT 10 -> 11); dtype
 *    FMOE_F8E4M3FN_A8 (3); fmoe_moe_ffn_block_noalloc.  Packed-weight
 *    artifacts record the version they were written under.
 * 3: dtype FMOE_F8E4M3FN_A8X2 (4). */
int fmoe_abi_version(void);
#define FMOE_ABI_VERSION 3

/* Checks that the current HIP device is a gfx950; writes its ordinal and
 * architecture name (arch may be NULL).  FMOE_ERR_NO_DEVICE otherwise. */
int fmoe_device_check(int *device, char *arch, size_t arch_len);

/* Kernel timing (no counterpart in the reference, which has no profiling
 * beyond dumping linked IR, tests/conftest.py:24-30).  While enabled, each
 * kernel that fmoe_moe_ffn_block / fmoe_mul_mat_id launch is bracketed by
 * HIP events recorded on the caller's stream.  fmoe_timing_read waits for
 * the recorded events, writes the summed milliseconds and the number of
 * timed regions per kernel family (index fmoe_timer, up to n entries) and
 * clears them.  A family can be timed in more than one region per call (the
 * permutation and the token-row gather under FMOE_TIMER_PERMUTE; the two
 * e4m3 quantisation passes under FMOE_TIMER_QUANT), so per-call times are
 * the sums divided by the number of calls, not by the region counts. */
typedef enum fmoe_timer {
  FMOE_TIMER_ROUTER = 0,  /* router logits + softmax + top-k (decode batches whose gate/up GEMM
                             routes in its blocks: the logits only; GATE_UP holds the rest) */
  FMOE_TIMER_PERMUTE = 1,
  FMOE_TIMER_GATE_UP = 2, /* grouped GEMM: gate + up projections + SwiGLU (+ the top-k, see ROUTER) */
  FMOE_TIMER_DOWN = 3,    /* grouped GEMM: down projection + routing weight (decode batches of
                             at most 16 assignments: + the slot-ordered combine, one launch) */
  FMOE_TIMER_COMBINE = 4, /* slot-ordered sum (+ residual); no launch where DOWN includes it */
  FMOE_TIMER_MUL_MAT_ID = 5,
  FMOE_TIMER_NORM = 6,    /* ffn_norm RMSNorm of the sub-layer */
  FMOE_TIMER_QKV = 7,     /* decode attention: Q/K/V projection + bias + RoPE */
  FMOE_TIMER_ATTENTION = 8, /* decode attention: context splits + combine */
  FMOE_TIMER_OUT_PROJ = 9,  /* decode attention: output projection + bias */
  FMOE_TIMER_QUANT = 10,    /* e4m3 quantisation of the GEMM activations (FMOE_F8E4M3FN_A8, _A8X2) */
  FMOE_TIMER_COUNT = 11
} fmoe_timer;
int fmoe_timing_enable(int on);
int fmoe_timing_read(double *ms_out, int64_t *regions_out, int n);

/* ---------------------------------------------------------------------- */
/* SwiGLU: out[i] = gate[i] * up[i] / (1 + exp(-up[i])), silu on `up`.
 * Replaces @activation_components.swiglu (components/activation/swiglu.mlir:16-51,
 * oracles/activation.py:11-21).  dtype FMOE_F32 or FMOE_BF16 for all three. */
int fmoe_swiglu(const void *gate, const void *up, void *out, int64_t n, int dtype,
                void *stream);

/* ---------------------------------------------------------------------- */
/* Router: logits = gate_inp_w @ input^T, fp32 softmax over experts, top-k
 * (descending, exact ties to the lower expert index), optional
 * renormalisation by the slot sum.  Replaces steps 1-4 of @moe_ffn_block
 * (moe_ffn_block.mlir:50-128; oracles/moe.py:86-105).
 *   input [n_tokens, n_embd], w_router [n_expert, n_embd] in `dtype`
 *   ids_out [k, n_tokens] int32, weights_out [k, n_tokens] float32 */
int fmoe_router(const void *input, const void *w_router, int64_t n_tokens,
                int64_t n_embd, int64_t n_expert, int64_t n_expert_used,
                int normalize_weights, int dtype, int32_t *ids_out,
                float *weights_out, void *stream);

/* ---------------------------------------------------------------------- */
/* Token->expert permutation of the slot-major flat assignment order
 * f = s*n_tokens + t (the order of `collapse_shape ids [[0,1]]`,
 * mul_mat_id.mlir:50-61), grouped by expert and stable:
 *   offsets_out[e] = #assignments to experts < e  (n_expert+1 entries)
 *   order_out[offsets_out[e] + r] = r-th smallest f with ids_flat[f] == e.
 * Ids outside [0, n_expert) are left out and counted in the workspace error
 * word (fmoe_workspace_error_count).  Workspace: fmoe_permute_workspace_bytes. */
size_t fmoe_permute_workspace_bytes(int64_t n_expert_used, int64_t n_tokens,
                                    int64_t n_expert);
int fmoe_permute(const int32_t *ids, int64_t n_expert_used, int64_t n_tokens,
                 int64_t n_expert, int32_t *order_out, int32_t *offsets_out,
                 void *workspace, size_t workspace_bytes, void *stream);

/* Number of invalid expert ids seen by the last call that used this
 * workspace (synchronises `stream`).  Applies to fmoe_permute and
 * fmoe_mul_mat_id workspaces. */
int fmoe_workspace_error_count(const void *workspace, void *stream,
                               int64_t *count_out);

/* ---------------------------------------------------------------------- */
/* One-time expert-weight packing.  Replaces the per-call transpose
 * [n_out, n_in, E] -> [E, n_out, n_in] of mul_mat_id.mlir:37-48.
 *   src [n_out, n_in, n_expert] in src_dtype (F32, BF16, or F8E4M3FN codes)
 *   src_scales [n_out, n_expert] float32: required iff src_dtype == F8E4M3FN
 *   dst: fmoe_packed_weight_bytes(n_out, n_in, n_expert, dst_dtype) bytes:
 *        per-expert [n_out, n_in] weights in dst_dtype, in an internal
 *        layout that depends only on (n_out, n_in, dtype), followed by a
 *        tail the kernels may read but never use
 *   dst_scales [n_expert, n_out] float32: required iff dst_dtype == F8E4M3FN.
 * F32/BF16 -> F8E4M3FN quantises each output channel with
 * scale = absmax/448 (1 for an all-zero channel), code = RNE(w/scale),
 * saturating at +-448. */
size_t fmoe_packed_weight_bytes(int64_t n_out, int64_t n_in, int64_t n_expert,
                                int dtype);
int fmoe_pack_expert_weights(const void *src, int src_dtype, const float *src_scales,
                             int64_t n_out, int64_t n_in, int64_t n_expert,
                             int dst_dtype, void *dst, float *dst_scales,
                             void *stream);

/* ---------------------------------------------------------------------- */
/* Expert-selected matmul out[:, s, t] = W[:, :, ids[s, t]] @ input[:, s, t].
 * Replaces @moe_components.mul_mat_id (mul_mat_id.mlir:22-120,
 * oracles/moe.py:9-48).
 *   packed_w / w_scales / w_dtype: from fmoe_pack_expert_weights
 *   input [n_in, k, n_tokens], out [n_out, k, n_tokens] in act_dtype
 *   ids [k, n_tokens] int32.  Output columns of an invalid id are zero. */
size_t fmoe_mul_mat_id_workspace_bytes(int64_t n_out, int64_t n_in, int64_t n_expert,
                                       int64_t n_expert_used, int64_t n_tokens,
                                       int act_dtype);
int fmoe_mul_mat_id(const void *packed_w, const float *w_scales, int w_dtype,
                    const void *input, const int32_t *ids, void *out, int64_t n_out,
                    int64_t n_in, int64_t n_expert, int64_t n_expert_used,
                    int64_t n_tokens, int act_dtype, void *workspace,
                    size_t workspace_bytes, void *stream);

/* ---------------------------------------------------------------------- */
/* Full MoE FFN block.  Replaces @moe_ffn_components.moe_ffn_block
 * (moe_ffn_block.mlir:34-209, oracles/moe.py:51-132), same argument meaning:
 *   input [n_tokens, n_embd], w_router [n_expert, n_embd], out [n_tokens, n_embd]
 *   all in act_dtype (F32 or BF16);
 *   packed_up / packed_gate ([n_ff, n_embd] per expert) and packed_down
 *   ([n_embd, n_ff] per expert) in w_dtype, with scales when w_dtype is
 *   F8E4M3FN.  SwiGLU is gate * silu(up).  Weighted expert outputs are summed
 *   in slot order.  Dot products accumulate in fp32; with BF16 activations
 *   the SwiGLU rows, and at prefill sizes the weighted expert outputs, are
 *   held in bf16 between kernels (the sum over slots runs in fp32).
 *   Workspace: fmoe_moe_ffn_block_workspace_bytes. */
size_t fmoe_moe_ffn_block_workspace_bytes(int64_t n_tokens, int64_t n_expert,
                                          int64_t n_expert_used, int64_t n_embd,
                                          int64_t n_ff, int act_dtype, int w_dtype);
int fmoe_moe_ffn_block(const void *input, const void *w_router, const void *packed_up,
                       const void *packed_gate, const void *packed_down,
                       const float *up_scales, const float *gate_scales,
                       const float *down_scales, int w_dtype, void *out,
                       int64_t n_tokens, int64_t n_expert, int64_t n_expert_used,
                       int64_t n_embd, int64_t n_ff, int normalize_weights,
                       int act_dtype, void *workspace, size_t workspace_bytes,
                       void *stream);

/* The MoE FFN block without a workspace argument.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Arguments and results are those of fmoe_moe_ffn_block; the
 * workspace is a device-resident scratch array of FMOE_NOALLOC_SCRATCH_BYTES
 * that the library holds on every GPU it runs on until the process ends.
 * The call allocates nothing (no hipMalloc, no library allocation; kernel
 * timing is not recorded for it).  A call whose
 * fmoe_moe_ffn_block_workspace_bytes exceed FMOE_NOALLOC_SCRATCH_BYTES
 * (Mixtral shapes: about 480 tokens) fails with FMOE_ERR_WORKSPACE before
 * any device work.  Every call on one GPU shares that GPU's array and
 * leaves its contents behind: calls that overlap on one GPU (two streams,
 * two host threads) race, so the caller serialises them.
 * fmoe_moe_ffn_block_routing cannot read this scratch. */
#define FMOE_NOALLOC_SCRATCH_BYTES (64u << 20)
int fmoe_moe_ffn_block_noalloc(const void *input, const void *w_router, const void *packed_up,
                               const void *packed_gate, const void *packed_down,
                               const float *up_scales, const float *gate_scales,
                               const float *down_scales, int w_dtype, void *out,
                               int64_t n_tokens, int64_t n_expert, int64_t n_expert_used,
                               int64_t n_embd, int64_t n_ff, int normalize_weights,
                               int act_dtype, void *stream);

/* RMS normalisation of each row: out = (x / sqrt(mean(x^2) + eps)) * weight,
 * x and out [n_rows, n_embd], weight [n_embd], all of `dtype` (F32 or BF16),
 * fp32 arithmetic.  Replaces @rms_norm_linalg
 * (components/normalization/rms_norm.mlir:18-85; oracles/normalization.py:10-43).
 * out may alias x. */
int fmoe_rms_norm(const void *input, const void *weight, float eps, void *out,
                  int64_t n_rows, int64_t n_embd, int dtype, void *stream);

/* The MoE FFN sub-layer of a transformer layer:
 *   out = residual + moe_ffn_block(rms_norm(residual, ffn_norm_w, rms_eps), ...)
 * (architectures/llm/transformer_layer_moe_prefill.mlir:205-242 on the
 * flattened [n_tokens, n_embd] residual; transformer_layer_moe_decode.mlir:227-255).
 * residual, out [n_tokens, n_embd] and ffn_norm_w [n_embd] are act_dtype; the
 * other arguments are those of fmoe_moe_ffn_block.  The residual is added in
 * fp32 by the block's final reduction (one rounding of the output).  out may
 * alias residual (in-place residual update).  Workspace: fmoe_moe_ffn_sublayer_workspace_bytes; it
 * begins with a block workspace, so fmoe_moe_ffn_block_routing reads the
 * routing of the last call from it. */
size_t fmoe_moe_ffn_sublayer_workspace_bytes(int64_t n_tokens, int64_t n_expert,
                                             int64_t n_expert_used, int64_t n_embd,
                                             int64_t n_ff, int act_dtype, int w_dtype);
int fmoe_moe_ffn_sublayer(const void *residual, const void *ffn_norm_w, float rms_eps,
                          const void *w_router, const void *packed_up,
                          const void *packed_gate, const void *packed_down,
                          const float *up_scales, const float *gate_scales,
                          const float *down_scales, int w_dtype, void *out,
                          int64_t n_tokens, int64_t n_expert, int64_t n_expert_used,
                          int64_t n_embd, int64_t n_ff, int normalize_weights,
                          int act_dtype, void *workspace, size_t workspace_bytes,
                          void *stream);

/* Views into a block (or sub-layer) workspace after a call on it: the routing
 * it computed (ids/weights [k, n_tokens]), the permutation (order [k*n_tokens],
 * offsets [n_expert+1]).  Pointers are device pointers inside `workspace`. */
int fmoe_moe_ffn_block_routing(void *workspace, int64_t n_tokens, int64_t n_expert,
                               int64_t n_expert_used, int64_t n_embd, int64_t n_ff,
                               int act_dtype, int w_dtype, int32_t **ids,
                               float **weights, int32_t **order, int32_t **offsets);

/* ---------------------------------------------------------------------- */
/* The decode step's attention half (the next component after the MoE FFN
 * block on the decode path, architectures/llm/transformer_layer_moe_decode.mlir:180-209).
 *
 * Paged KV cache.  Replaces @kvcache_components.gather / scatter_decode
 * (components/kvcache/kvcache.mlir; oracles/kvcache.py:51-185) and the
 * oracle-only scatter_prefill (oracles/kvcache.py:142-185).
 *   cache: one pool [n_blocks, block_size, n_head_kv, head_dim] in dtype
 *          (F32 or BF16), 4-byte aligned, updated in place by the scatters
 *   block_tables [n_layers, batch, max_blocks_per_seq] int32,
 *   context_lens [n_layers, batch] int32 (device)
 *   gather out [batch, max_context_len, n_head_kv, head_dim]: rows at and past
 *          min(context_lens[layer, b], max_context_len) are zero
 *   scatter_decode: new_vals [batch, n_head_kv, head_dim] (cache dtype) to
 *          (block_indices[b], pos_in_blocks[b]); when several b name one
 *          slot the last b wins (the reference's sequential loop)
 *   scatter_prefill: new_vals [batch, seq_len, n_head_kv, head_dim] to
 *          positions start_positions[b] + s through the layer's block table.
 * Table entries or indices outside the pool read as zero rows (gather) or
 * skip the write (scatters): the reference would index out of bounds. */
int fmoe_kvcache_gather(const void *cache, int dtype, int64_t n_blocks, int64_t block_size,
                        int64_t n_head_kv, int64_t head_dim, int64_t layer,
                        const int32_t *block_tables, const int32_t *context_lens,
                        int64_t n_layers, int64_t batch, int64_t max_blocks_per_seq,
                        int64_t max_context_len, void *out, void *stream);
int fmoe_kvcache_scatter_decode(void *cache, int dtype, int64_t n_blocks, int64_t block_size,
                                int64_t n_head_kv, int64_t head_dim, const void *new_vals,
                                const int32_t *block_indices, const int32_t *pos_in_blocks,
                                int64_t batch, void *stream);
int fmoe_kvcache_scatter_prefill(void *cache, int dtype, int64_t n_blocks, int64_t block_size,
                                 int64_t n_head_kv, int64_t head_dim, int64_t layer,
                                 const void *new_vals, int64_t seq_len,
                                 const int32_t *block_tables, int64_t n_layers, int64_t batch,
                                 int64_t max_blocks_per_seq, const int32_t *start_positions,
                                 void *stream);

/* Dense projection weight in the reference's `x @ W` layout, src [n_in, n_out]
 * row-major (F32 or BF16; attention_block_decode.mlir:104-118), packed into
 * rows [row_offset, row_offset + n_out) of a one-expert packed weight
 * [n_out_total, n_in] of fmoe_packed_weight_bytes(n_out_total, n_in, 1,
 * dst_dtype) bytes (dst_scales [n_out_total] for F8E4M3FN, quantised per
 * output channel as fmoe_pack_expert_weights does).  The attention entry
 * points take wq | wk | wv packed as one [n_embd + 2 n_embd_kv, n_embd]
 * weight (row offsets 0, n_embd, n_embd + n_embd_kv) and wo as [n_embd, n_embd]. */
int fmoe_pack_linear_weight(const void *src, int src_dtype, int64_t n_in, int64_t n_out,
                            int64_t row_offset, int64_t n_out_total, int dst_dtype, void *dst,
                            float *dst_scales, void *stream);

/* Decode attention block.  Replaces
 * @attention_block_decode_components.attention_block_decode
 * (components/attention/attention_block_decode.mlir:52-244; oracles/attention.py
 * attention_block + attention_gqa:8-52; RoPE components/position/rope.mlir:22-110):
 *   input [batch, n_embd], positions [batch] int64,
 *   k_cached / v_cached [batch, ctx_len, n_head_kv, head_dim] (act dtype,
 *   16-byte aligned), packed_wqkv / packed_wo (+ fp8 scales) as above,
 *   biases bq [n_embd], bk, bv [n_embd_kv], bo [n_embd] float32 (read only
 *   when use_bias = 1), head_dim = n_embd / n_head = n_embd_kv / n_head_kv
 *   in {16, 32, 64, 128}, n_head / n_head_kv in {1, 2, 4, 8}.
 *   out [batch, n_embd], k_new / v_new [batch, n_head_kv, head_dim] (RoPE
 *   applied to k_new), all in act_dtype.
 * The new token attends to the ctx_len cached positions and itself, scale
 * 1/sqrt(head_dim), no mask (attention_gqa.mlir:120-137). */
size_t fmoe_attention_block_decode_workspace_bytes(int64_t batch, int64_t ctx_len, int64_t n_head,
                                                   int64_t n_head_kv, int64_t n_embd,
                                                   int64_t n_embd_kv, int act_dtype);
int fmoe_attention_block_decode(const void *input, const int64_t *positions,
                                const void *k_cached, const void *v_cached, int64_t ctx_len,
                                const void *packed_wqkv, const float *wqkv_scales,
                                const void *packed_wo, const float *wo_scales, int w_dtype,
                                const float *bq, const float *bk, const float *bv,
                                const float *bo, int use_bias, int64_t batch, int64_t n_head,
                                int64_t n_head_kv, int64_t n_embd, int64_t n_embd_kv,
                                float rope_freq_base, float rope_freq_scale, int act_dtype,
                                void *out, void *k_new, void *v_new, void *workspace,
                                size_t workspace_bytes, void *stream);

/* The decode layer's attention sequence on the paged cache: gather of
 * max_context_len positions + attention_block_decode + scatter_decode of the
 * new K/V (architectures/llm/transformer_layer_moe_decode.mlir:180-209), with
 * the cache read in place instead of gathered.  Pools in act_dtype, 16-byte
 * aligned; k_new / v_new may be null (the scatter still runs).  As in the
 * reference, positions in [min(context_lens, max_context_len),
 * max_context_len) enter the softmax as zero keys and values. */
size_t fmoe_attention_decode_paged_workspace_bytes(int64_t batch, int64_t max_context_len,
                                                   int64_t n_head, int64_t n_head_kv,
                                                   int64_t n_embd, int64_t n_embd_kv,
                                                   int act_dtype);
int fmoe_attention_decode_paged(const void *input, const int64_t *positions, void *k_cache,
                                void *v_cache, int64_t n_blocks, int64_t block_size,
                                int64_t layer, const int32_t *block_tables,
                                const int32_t *context_lens, int64_t n_layers,
                                int64_t max_blocks_per_seq, int64_t max_context_len,
                                const int32_t *block_indices, const int32_t *pos_in_blocks,
                                const void *packed_wqkv, const float *wqkv_scales,
                                const void *packed_wo, const float *wo_scales, int w_dtype,
                                const float *bq, const float *bk, const float *bv,
                                const float *bo, int use_bias, int64_t batch, int64_t n_head,
                                int64_t n_head_kv, int64_t n_embd, int64_t n_embd_kv,
                                float rope_freq_base, float rope_freq_scale, int act_dtype,
                                void *out, void *k_new, void *v_new, void *workspace,
                                size_t workspace_bytes, void *stream);

/* The decode layer's attention sub-layer: out = residual +
 * attention_decode_paged(rms_norm(residual, attn_norm_w, rms_eps), ...)
 * (architectures/llm/transformer_layer_moe_decode.mlir:174-221: attn_norm,
 * gather, attention_block_decode, scatter_decode, residual add), the
 * attention-half counterpart of fmoe_moe_ffn_sublayer.  The attention output
 * is rounded to act_dtype before the add, as the reference adds two tensors.
 * out may alias residual.  Arguments otherwise as fmoe_attention_decode_paged. */
size_t fmoe_attention_sublayer_decode_paged_workspace_bytes(int64_t batch, int64_t max_context_len,
                                                            int64_t n_head, int64_t n_head_kv,
                                                            int64_t n_embd, int64_t n_embd_kv,
                                                            int act_dtype);
int fmoe_attention_sublayer_decode_paged(const void *residual, const void *attn_norm_w,
                                         float rms_eps, const int64_t *positions, void *k_cache,
                                         void *v_cache, int64_t n_blocks, int64_t block_size,
                                         int64_t layer, const int32_t *block_tables,
                                         const int32_t *context_lens, int64_t n_layers,
                                         int64_t max_blocks_per_seq, int64_t max_context_len,
                                         const int32_t *block_indices,
                                         const int32_t *pos_in_blocks, const void *packed_wqkv,
                                         const float *wqkv_scales, const void *packed_wo,
                                         const float *wo_scales, int w_dtype, const float *bq,
                                         const float *bk, const float *bv, const float *bo,
                                         int use_bias, int64_t batch, int64_t n_head,
                                         int64_t n_head_kv, int64_t n_embd, int64_t n_embd_kv,
                                         float rope_freq_base, float rope_freq_scale,
                                         int act_dtype, void *out, void *k_new, void *v_new,
                                         void *workspace, size_t workspace_bytes, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* FMOE_H_ */
