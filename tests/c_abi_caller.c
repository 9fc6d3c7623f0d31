/* A plain C99 caller of libhprms.so: proves that include/hp_rms_norm_amd.h is
 * a C header and that the library links and answers from C without torch or
 * a device (argument checks, the configuration table, zero-row calls).
 * Built and run by tests/test_abi_cpu.py with gcc. */
#include <stdio.h>
#include <string.h>

#include "hp_rms_norm_amd.h"

static int failures = 0;

#define EXPECT(cond)                                              \
  do {                                                            \
    if (!(cond)) {                                                \
      fprintf(stderr, "line %d: expected %s\n", __LINE__, #cond); \
      ++failures;                                                 \
    }                                                             \
  } while (0)

int main(void) {
  void* x = (void*)0x1000;
  void* w = (void*)0x2000;
  void* r = (void*)0x3000;
  const void* parts[HPRMS_MAX_PARTS + 1];
  hprms_config c;
  int mode;

  EXPECT(hprms_abi_version() == HPRMS_ABI_VERSION);
  EXPECT(strcmp(hprms_last_error(), "") == 0);

  /* argument checks return a status and a message; nothing touches a device */
  EXPECT(hprms_fused_add_rmsnorm(x, w, r, 4, 4096, 4096, 4096, 7, 1e-6, NULL) == HPRMS_E_INVALID);
  EXPECT(strstr(hprms_last_error(), "dtype") != NULL);
  EXPECT(hprms_fused_add_rmsnorm(x, w, x, 4, 4096, 4096, 4096, HPRMS_DTYPE_BF16, 1e-6, NULL) == HPRMS_E_INVALID);
  EXPECT(hprms_fused_add_rmsnorm(x, w, r, 4, (1 << 24) + 8, (1 << 24) + 8, (1 << 24) + 8, HPRMS_DTYPE_BF16, 1e-6,
                                 NULL) == HPRMS_E_RANGE);
  EXPECT(hprms_streamer(x, r, 4, 64, 64, 64, HPRMS_DTYPE_FP16, 9, NULL) == HPRMS_E_INVALID);
  EXPECT(hprms_rmsnorm(x, r, NULL, 4, 64, 64, 64, HPRMS_DTYPE_BF16, 1e-6, NULL) == HPRMS_E_INVALID);
  EXPECT(hprms_fused_add_rmsnorm_out(x, x, r, r, w, 4, 64, 64, 64, 64, 64, HPRMS_DTYPE_BF16, 1e-6, NULL) ==
         HPRMS_E_INVALID);
  EXPECT(hprms_reduce_add_rmsnorm(x, parts, HPRMS_MAX_PARTS + 1, w, r, 4, 64, 64, 64, 64, HPRMS_DTYPE_BF16, 1e-6,
                                  NULL) == HPRMS_E_INVALID);
  EXPECT(strstr(hprms_last_error(), "nparts") != NULL);
  EXPECT(hprms_fused_add_rmsnorm_mx(x, r, x, w, r, 4, 4096, 2048, 128, 4096, 4096, 7, HPRMS_DTYPE_BF16, 1e-6, NULL) ==
         HPRMS_E_INVALID);
  EXPECT(hprms_fused_add_rmsnorm_mx(NULL, NULL, NULL, NULL, NULL, 0, 4096, 2048, 128, 4096, 4096, HPRMS_MX_FP4_E2M1,
                                    HPRMS_DTYPE_BF16, 1e-6, NULL) == HPRMS_OK);

  /* zero rows: validated, no launch, null pointers accepted */
  EXPECT(hprms_fused_add_rmsnorm(NULL, NULL, NULL, 0, 4096, 4096, 4096, HPRMS_DTYPE_BF16, 1e-6, NULL) == HPRMS_OK);
  EXPECT(hprms_fused_add_rmsnorm_fp8(NULL, NULL, NULL, NULL, NULL, 0, 4096, 4096, 4096, 4096, HPRMS_DTYPE_FP16,
                                     1e-6, NULL) == HPRMS_OK);
  EXPECT(hprms_fused_add_rmsnorm_fp8_static(NULL, NULL, NULL, NULL, NULL, 0, 4096, 4096, 4096, 4096,
                                            HPRMS_DTYPE_BF16, 1e-6, NULL) == HPRMS_OK);
  EXPECT(hprms_fused_add_rmsnorm_fp8_ub(NULL, NULL, NULL, NULL, NULL, NULL, 0, 4096, 4096, 4096, 4096,
                                        HPRMS_DTYPE_BF16, 1e-6, NULL) == HPRMS_OK);
  EXPECT(hprms_fused_add_rmsnorm_fp8_ub(x, x, NULL, x, w, r, 4, 4096, 4096, 4096, 4096, HPRMS_DTYPE_BF16, 1e-6,
                                        NULL) == HPRMS_E_INVALID);
  EXPECT(strstr(hprms_last_error(), "scale_ub") != NULL);
  EXPECT(hprms_fused_add_rmsnorm_fp8_group(NULL, NULL, NULL, NULL, NULL, 0, 4096, 4096, 32, 1, 4096, 4096,
                                           HPRMS_DTYPE_BF16, 1e-6, NULL) == HPRMS_OK);
  EXPECT(hprms_fused_add_rmsnorm_fp8_group(NULL, NULL, NULL, NULL, NULL, 0, 4000, 4000, 32, 1, 4000, 4000,
                                           HPRMS_DTYPE_BF16, 1e-6, NULL) == HPRMS_E_INVALID);
  EXPECT(hprms_reduce_add_rmsnorm(NULL, NULL, 3, NULL, NULL, 0, 4096, 4096, 4096, 4096, HPRMS_DTYPE_BF16, 1e-6,
                                  NULL) == HPRMS_OK);

  /* the table: every mode has a vector-tier kernel covering H = 4096 */
  for (mode = 0; mode <= 7; ++mode) {
    int n;
    EXPECT(hprms_select_config(4096, 4096, HPRMS_DTYPE_BF16, mode, &c) == HPRMS_OK);
    EXPECT(c.tier == 1 || c.tier == 2);
    EXPECT((long)c.lanes_per_row * c.vec_per_lane * 8 >= 4096);
    n = hprms_kernel_configs(HPRMS_DTYPE_BF16, mode, NULL, 0);
    EXPECT(n > 0);
  }
  EXPECT(hprms_select_config(4096, 4096, HPRMS_DTYPE_BF16, 8, &c) == HPRMS_E_INVALID);
  /* hidden % 8 != 0: the same shape with a tail vector (flags bit 6); below 8 elements, the general kernel */
  EXPECT(hprms_select_config(4096, 4097, HPRMS_DTYPE_BF16, 0, &c) == HPRMS_OK && c.tier == 1 && (c.flags & 96) == 96);
  EXPECT(hprms_select_config(4096, 15, HPRMS_DTYPE_BF16, 0, &c) == HPRMS_OK && c.tier == 1 && (c.flags & 96) == 96);
  EXPECT(hprms_select_config(4096, 7, HPRMS_DTYPE_BF16, 0, &c) == HPRMS_OK && c.tier == 3);
  /* on a 256-CU device the per-CU table is hprms_select_config's; a CU count of 0 is refused */
  {
    hprms_config d;
    EXPECT(hprms_select_config_cu(4096, 4096, HPRMS_DTYPE_BF16, 0, 256, &d) == HPRMS_OK);
    EXPECT(hprms_select_config(4096, 4096, HPRMS_DTYPE_BF16, 0, &c) == HPRMS_OK);
    EXPECT(c.lanes_per_row == d.lanes_per_row && c.vec_per_lane == d.vec_per_lane && c.flags == d.flags);
    EXPECT(hprms_select_config_cu(4096, 4096, HPRMS_DTYPE_BF16, 0, 0, &d) == HPRMS_E_INVALID);
  }

  if (failures) return 1;
  printf("c abi caller: ok\n");
  return 0;
}
