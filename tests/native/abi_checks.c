/* Host-side checks of the C ABI (include/fmoe.h, include/fmoe_diag.h) on a machine without a GPU.
 *
 * Built by tests/test_sanitizers.py with AddressSanitizer and
 * UndefinedBehaviorSanitizer on the host code of capi.cpp, then run: every
 * entry point is called with invalid arguments and must return the
 * documented status (never crash, never touch memory it was not given);
 * calls that pass validation must report FMOE_ERR_NO_DEVICE. */
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "fmoe.h"
#include "fmoe_diag.h"

static int failures = 0;

#define EXPECT(call, want)                                                                   \
  do {                                                                                       \
    int got_ = (call);                                                                       \
    if (got_ != (want)) {                                                                    \
      fprintf(stderr, "line %d: %s -> %d, expected %d (%s)\n", __LINE__, #call, got_, (want), \
              fmoe_last_error());                                                            \
      ++failures;                                                                            \
    }                                                                                        \
  } while (0)

int main(void) {
  /* a fake non-null device pointer: validation must fail before it is used */
  void *p = (void *)(uintptr_t)0x100000;
  char arch[32];
  int dev = -1;

  if (fmoe_abi_version() != FMOE_ABI_VERSION) ++failures;

  /* dtype, shape and flag errors */
  EXPECT(fmoe_swiglu(NULL, NULL, NULL, 4, 9, NULL), FMOE_ERR_DTYPE);
  EXPECT(fmoe_router(NULL, NULL, 4, 8, 0, 1, 0, FMOE_F32, NULL, NULL, NULL), FMOE_ERR_SHAPE);
  EXPECT(fmoe_router(NULL, NULL, 4, 8, 4, 5, 0, FMOE_F32, NULL, NULL, NULL), FMOE_ERR_SHAPE);
  EXPECT(fmoe_router(NULL, NULL, -1, 8, 4, 2, 0, FMOE_F32, NULL, NULL, NULL), FMOE_ERR_SHAPE);
  EXPECT(fmoe_router(NULL, NULL, 4, 8, 4, 2, 7, FMOE_F32, NULL, NULL, NULL), FMOE_ERR_INVALID_ARGUMENT);
  EXPECT(fmoe_router(NULL, NULL, 4, 8, 4, 2, 0, FMOE_F32, NULL, NULL, NULL), FMOE_ERR_INVALID_ARGUMENT);
  EXPECT(fmoe_permute(NULL, 2, 4, 0, NULL, NULL, NULL, 0, NULL), FMOE_ERR_SHAPE);
  EXPECT(fmoe_permute(NULL, 2, 4, 8, NULL, NULL, NULL, 0, NULL), FMOE_ERR_INVALID_ARGUMENT);
  EXPECT(fmoe_pack_expert_weights(NULL, FMOE_F8E4M3FN, NULL, 4, 4, 2, FMOE_BF16, NULL, NULL, NULL),
         FMOE_ERR_DTYPE);
  EXPECT(fmoe_mul_mat_id(NULL, NULL, FMOE_BF16, NULL, NULL, NULL, 8, 4, 2, 1, 3, FMOE_F8E4M3FN, NULL, 0, NULL),
         FMOE_ERR_DTYPE);
  EXPECT(fmoe_moe_ffn_block(NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL, FMOE_BF16, NULL, 4, 4, 2, 8, 16, 0,
                            FMOE_F32, NULL, 0, NULL),
         FMOE_ERR_DTYPE);
  EXPECT(fmoe_moe_ffn_block(p, p, p, p, p, NULL, NULL, NULL, FMOE_F8E4M3FN, p, 4, 4, 2, 64, 128, 0, FMOE_BF16, p,
                            1 << 20, NULL),
         FMOE_ERR_INVALID_ARGUMENT); /* fp8 without scales */
  EXPECT(fmoe_moe_ffn_block(p, p, p, p, p, NULL, NULL, NULL, FMOE_BF16, p, 4, 4, 2, 64, 128, 2, FMOE_BF16, p,
                            1 << 20, NULL),
         FMOE_ERR_INVALID_ARGUMENT); /* normalize flag */
  EXPECT(fmoe_rms_norm(NULL, NULL, 1e-6f, NULL, 4, 0, FMOE_F32, NULL), FMOE_ERR_SHAPE);
  EXPECT(fmoe_set_gemm_path(99), FMOE_ERR_INVALID_ARGUMENT);

  /* workspace too small / misaligned, before the device */
  size_t need = fmoe_moe_ffn_block_workspace_bytes(16, 8, 2, 64, 128, FMOE_BF16, FMOE_BF16);
  if (need == 0) ++failures;
  EXPECT(fmoe_moe_ffn_block(p, p, p, p, p, NULL, NULL, NULL, FMOE_BF16, p, 16, 8, 2, 64, 128, 0, FMOE_BF16, p,
                            need - 1, NULL),
         FMOE_ERR_WORKSPACE);
  EXPECT(fmoe_moe_ffn_block(p, p, p, p, p, NULL, NULL, NULL, FMOE_BF16, p, 16, 8, 2, 64, 128, 0, FMOE_BF16,
                            (char *)p + 4, need, NULL),
         FMOE_ERR_INVALID_ARGUMENT);
  size_t sub = fmoe_moe_ffn_sublayer_workspace_bytes(16, 8, 2, 64, 128, FMOE_BF16, FMOE_BF16);
  if (sub <= need) ++failures;
  EXPECT(fmoe_moe_ffn_sublayer(p, NULL, 1e-5f, p, p, p, p, NULL, NULL, NULL, FMOE_BF16, p, 16, 8, 2, 64, 128, 0,
                               FMOE_BF16, p, sub, NULL),
         FMOE_ERR_INVALID_ARGUMENT); /* null norm weight */

  /* empty batches are no-ops */
  EXPECT(fmoe_moe_ffn_block(NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL, FMOE_F32, NULL, 0, 4, 2, 8, 16, 0,
                            FMOE_F32, NULL, 0, NULL),
         FMOE_OK);
  EXPECT(fmoe_rms_norm(NULL, NULL, 1e-6f, NULL, 0, 8, FMOE_F32, NULL), FMOE_OK);

  /* valid calls reach the device check, which fails without a GPU */
  EXPECT(fmoe_device_check(&dev, arch, sizeof arch), FMOE_ERR_NO_DEVICE);
  EXPECT(fmoe_moe_ffn_block(p, p, p, p, p, NULL, NULL, NULL, FMOE_BF16, p, 16, 8, 2, 64, 128, 0, FMOE_BF16, p,
                            need, NULL),
         FMOE_ERR_NO_DEVICE);
  EXPECT(fmoe_rms_norm(p, p, 1e-6f, p, 4, 8, FMOE_F32, NULL), FMOE_ERR_NO_DEVICE);
  if (strlen(fmoe_last_error()) == 0) ++failures;

  /* a long arch buffer request and a tiny one do not overflow */
  EXPECT(fmoe_device_check(&dev, arch, 1), FMOE_ERR_NO_DEVICE);

  if (failures) {
    fprintf(stderr, "%d check(s) failed\n", failures);
    return 1;
  }
  puts("abi checks ok");
  return 0;
}
