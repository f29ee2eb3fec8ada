/*
 * fmoe_diag.h -- kernel-path override of libfmoe.so, for tests and tuning.
 *
 * No counterpart in the reference: IREE picks its kernels at compile time
 * (components/moe/mul_mat_id.mlir:22-120 is lowered once).  These calls are
 * kept out of fmoe.h because the override is process-wide: it changes the
 * kernel family of every grouped GEMM any caller launches afterwards, so a
 * production caller has no use for it.  The parity tests force each family
 * in turn with it and compare them with the oracle.
 */
#ifndef FMOE_DIAG_H_
#define FMOE_DIAG_H_
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum fmoe_gemm_path {
  FMOE_PATH_AUTO = 0,
  FMOE_PATH_GENERIC = 1, /* SIMT grouped GEMM, any shape and dtype */
  FMOE_PATH_TILED = 2,   /* MFMA tiled grouped GEMM, 128-row tiles */
  FMOE_PATH_STREAM = 3,  /* MFMA weight-streaming grouped GEMM (decode) */
  FMOE_PATH_TILED_LARGE = 4 /* MFMA tiled grouped GEMM, 256x256 tiles (prefill) */
} fmoe_gemm_path;

/* Selects the grouped-GEMM kernel family (fmoe_gemm_path) for the whole
 * process (default AUTO).  A forced family that cannot run a given GEMM
 * (dtype, shape, alignment) falls back to the AUTO choice for that GEMM.
 * Any forced family also keeps the block's down projection and combine as
 * two launches (AUTO fuses them for decode batches of at most 16
 * assignments, with the same results bit for bit).
 * FMOE_ERR_INVALID_ARGUMENT for an unknown value. */
int fmoe_set_gemm_path(int path);
int fmoe_get_gemm_path(void);
/* The family used by the last grouped GEMM launched on this thread. */
int fmoe_last_gemm_path(void);
/* The row quantiser of the fp8-activation GEMMs (FMOE_F8E4M3FN_A8 / _A8X2),
 * exposed so tests can compare its codes with the oracle bit for bit: rows
 * of src [n_rows, n_cols] bf16 (n_cols % 64 == 0, <= 16384), each scaled by
 * the smallest power of two 2^e with max|row| / 2^e <= 448 (dst_scale[r] =
 * 2^e), hi = e4m3(v) into dst_hi and, when dst_lo is not NULL, lo =
 * e4m3(v - hi) into dst_lo, both K-blocked in 64-input pieces (piece j of
 * row r at byte (j * n_rows + r) * 64, its 16-byte chunk g holding inputs
 * 64j + 8g + [0, 8) then 64j + 32 + 8g + [0, 8)).  Device pointers, 16-byte
 * aligned.  No counterpart in the reference. */
int fmoe_quantize_rows_e4m3(const void *src, int64_t n_rows, int64_t n_cols, void *dst_hi, void *dst_lo,
                            float *dst_scale, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* FMOE_DIAG_H_ */
