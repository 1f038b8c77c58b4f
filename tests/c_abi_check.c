/* A C99 caller of the library's C ABI (include/moe_fp8.h), compiled with gcc by
 * tests/test_c_header.py: the header must build as plain C, and the calls that need no GPU
 * (sizes, layout, argument validation, error text) must work through it. */
#include <stdio.h>
#include <string.h>
#include "moe_fp8.h"

int main(void) {
  moe_fp8_layout L;
  moe_fp8_args a;
  int rc;
  memset(&a, 0, sizeof a);
  printf("sizeof_args %zu\n", sizeof(moe_fp8_args));
  printf("sizeof_layout %zu\n", sizeof(moe_fp8_layout));
  printf("workspace_64 %zu\n", moe_fp8_workspace_bytes(64));
  printf("workspace_8192 %zu\n", moe_fp8_workspace_bytes(8192));
  rc = moe_fp8_workspace_layout(64, &L);
  printf("layout_rc %d requant_block %d rows_per_item %d\n", rc, (int)L.requant_block, (int)L.rows_per_item);
  printf("packed_bytes %zu\n", moe_fp8_packed_weights_bytes());
  a.num_tokens = 16;
  rc = moe_fp8_run(&a, NULL, 0, NULL);
  printf("run_null %d %s\n", rc, moe_fp8_strerror(rc));
  a.num_tokens = -1;
  rc = moe_fp8_run(&a, NULL, 0, NULL);
  printf("run_negative %d\n", rc);
  printf("version %s\n", moe_fp8_version());
  return 0;
}
