/* A plain C99 caller of libubridge_hip.so: the header must compile as C and
 * every call below must link and behave without a GPU (argument errors are
 * reported before any device work).  Built and run by tests/test_abi.py. */
#include <stdio.h>
#include <string.h>
#include "ubridge_hip.h"

int main(void) {
  int fails = 0;
  const char* v = ubridge_version();
  if (!v || !strstr(v, "gfx950")) { printf("version: %s\n", v ? v : "(null)"); fails++; }
  /* void entry point with the reference's signature: error through last_error */
  dequantize_block_q8_0_f32(NULL, NULL, 64, NULL);
  if (ubridge_last_error() != 1) { printf("dequant null pointers not rejected\n"); fails++; }
  if (ubridge_last_error() != 0) { printf("last_error not cleared\n"); fails++; }
  /* int-returning entry points */
  if (topsaten_moe_align_block_size(NULL, NULL, NULL, NULL, 4, 2, 0, 16, NULL) != 1) {
    printf("align E = 0 not rejected\n");
    fails++;
  }
  ubridge_last_error();
  if (ubridge_tune_set("no_such_knob", 1) == 0) { printf("unknown knob accepted\n"); fails++; }
  ubridge_last_error();
  if (ubridge_qmatmul_noalloc_max_workspace() == 0) { printf("noalloc max 0\n"); fails++; }
  printf(fails ? "FAIL\n" : "OK\n");
  return fails;
}
