/* Host-side memory and undefined-behaviour check of the C ABI (include/moe_fp8.h): built with
 * clang -fsanitize=address,undefined and linked with a libmoe_fp8.so whose host code carries
 * the same sanitizers (tests/test_c_abi_sanitize.py). It walks every host path that runs
 * without a GPU: workspace sizes and layouts across the regime boundaries, every argument
 * validation error of every entry point, and the error texts. Every call it makes has at
 * least one invalid argument that the library rejects before it looks at the device, so
 * nothing is launched whatever machine it runs on. Prints "ok" and exits 0 when every check
 * holds. */
#include <stddef.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
#include "moe_fp8.h"

static int failures = 0;

#define CHECK(cond)                                                         \
  do {                                                                      \
    if (!(cond)) {                                                          \
      printf("FAIL line %d: %s\n", __LINE__, #cond);                        \
      ++failures;                                                           \
    }                                                                       \
  } while (0)

/* A fake device address: never dereferenced, the calls below are all rejected first. */
static void* fake(uintptr_t a) { return (void*)a; }

static void valid_args(moe_fp8_args* a, int32_t T) {
  memset(a, 0, sizeof *a);
  a->routing_logits = fake(0x1000);
  a->routing_bias = fake(0x2000);
  a->routing_bias_dtype = MOE_FP8_BIAS_BF16;
  a->hidden_states = fake(0x3000);
  a->hidden_states_scale = fake(0x4000);
  a->gemm1_weights = fake(0x5000);
  a->gemm1_weights_scale = fake(0x6000);
  a->gemm2_weights = fake(0x7000);
  a->gemm2_weights_scale = fake(0x8000);
  a->num_tokens = T;
  a->local_expert_offset = 0;
  a->routed_scaling_factor = 2.5f;
  a->output = fake(0x9000);
  a->output_dtype = MOE_FP8_OUT_BF16;
}

/* The layout's arrays: 256-byte aligned, inside the total, in order and not overlapping. */
static void check_layout(int32_t T) {
  moe_fp8_layout L;
  size_t off[17];
  int n = 0, i;
  int rc = moe_fp8_workspace_layout(T, &L);
  CHECK(rc == MOE_FP8_OK);
  if (rc != MOE_FP8_OK) return;
  CHECK(L.total_bytes == moe_fp8_workspace_bytes(T));
  off[n++] = L.counters;     off[n++] = L.topk_ids;     off[n++] = L.topk_weights;
  off[n++] = L.expert_count; off[n++] = L.expert_start; off[n++] = L.sorted_token;
  off[n++] = L.sorted_weight; off[n++] = L.sorted_slot; off[n++] = L.token_nlocal;
  off[n++] = L.slot_rank;    off[n++] = L.block_count;  off[n++] = L.work_items;
  off[n++] = L.act;          off[n++] = L.act_scale;    off[n++] = L.partial;
  off[n++] = L.swiglu;       off[n++] = L.row_dest;
  for (i = 0; i < n; ++i) {
    CHECK(off[i] % 256 == 0);
    CHECK(off[i] <= L.total_bytes);
    if (i > 0) CHECK(off[i] >= off[i - 1]);
  }
  CHECK(L.num_tokens == T);
  CHECK(L.requant_block == 64 || L.requant_block == 128);
  CHECK(L.rows_per_item >= 16 && L.rows_per_item <= 160);
}

static void check_entry_points(int32_t T, void* ws, size_t ws_bytes) {
  moe_fp8_args a;
  moe_fp8_layout L;
  int rc;
  moe_fp8_workspace_layout(T, &L);

  /* null args */
  CHECK(moe_fp8_run(NULL, ws, ws_bytes, NULL) == MOE_FP8_EINVAL_POINTER);
  CHECK(moe_fp8_route_dispatch(NULL, 0, ws, ws_bytes, NULL) == MOE_FP8_EINVAL_POINTER);
  CHECK(moe_fp8_gemm1(NULL, ws, ws_bytes, NULL) == MOE_FP8_EINVAL_POINTER);
  CHECK(moe_fp8_gemm2_combine(NULL, ws, ws_bytes, NULL) == MOE_FP8_EINVAL_POINTER);

  /* every required pointer missing in turn */
  {
    size_t fields[] = {offsetof(moe_fp8_args, routing_logits), offsetof(moe_fp8_args, routing_bias),
                       offsetof(moe_fp8_args, hidden_states), offsetof(moe_fp8_args, hidden_states_scale),
                       offsetof(moe_fp8_args, gemm1_weights), offsetof(moe_fp8_args, gemm1_weights_scale),
                       offsetof(moe_fp8_args, gemm2_weights), offsetof(moe_fp8_args, gemm2_weights_scale),
                       offsetof(moe_fp8_args, output)};
    size_t k;
    for (k = 0; k < sizeof fields / sizeof fields[0]; ++k) {
      valid_args(&a, T);
      memset((char*)&a + fields[k], 0, sizeof(void*));
      CHECK(moe_fp8_run(&a, ws, ws_bytes, NULL) == MOE_FP8_EINVAL_POINTER);
      rc = moe_fp8_run_static(&a, NULL);
      CHECK(rc == (T > MOE_FP8_STATIC_MAX_TOKENS ? MOE_FP8_ESTATIC_TOKENS : MOE_FP8_EINVAL_POINTER));
      /* the GEMM stages do not read the routing inputs */
      CHECK(moe_fp8_gemm1(&a, ws, ws_bytes, NULL) == (k < 2 ? MOE_FP8_EWORKSPACE : MOE_FP8_EINVAL_POINTER));
    }
  }
  /* dtypes */
  valid_args(&a, T);
  a.routing_bias_dtype = 3;
  CHECK(moe_fp8_run(&a, ws, ws_bytes, NULL) == MOE_FP8_EINVAL_BIAS_DTYPE);
  a.routing_bias_dtype = -1;
  CHECK(moe_fp8_run(&a, ws, ws_bytes, NULL) == MOE_FP8_EINVAL_BIAS_DTYPE);
  valid_args(&a, T);
  a.output_dtype = 7;
  CHECK(moe_fp8_run(&a, ws, ws_bytes, NULL) == MOE_FP8_EINVAL_OUT_DTYPE);
  /* a pointer off its alignment (16: hidden states; 4: scales; 8: bf16 output), a workspace off 256 */
  valid_args(&a, T);
  a.hidden_states = fake(0x3008);
  CHECK(moe_fp8_run(&a, ws, ws_bytes, NULL) == MOE_FP8_EALIGN);
  CHECK(moe_fp8_gemm2_combine(&a, ws, ws_bytes, NULL) == MOE_FP8_EALIGN);
  valid_args(&a, T);
  a.gemm2_weights_scale = fake(0x8002);
  CHECK(moe_fp8_run_static(&a, NULL) == (T > MOE_FP8_STATIC_MAX_TOKENS ? MOE_FP8_ESTATIC_TOKENS : MOE_FP8_EALIGN));
  valid_args(&a, T);
  a.output = fake(0x9004);
  CHECK(moe_fp8_run(&a, ws, ws_bytes, NULL) == MOE_FP8_EALIGN);
  valid_args(&a, T);
  CHECK(moe_fp8_run(&a, fake(0x10080), L.total_bytes, NULL) == MOE_FP8_EALIGN);
  CHECK(moe_fp8_run_packed(&a, fake(0xa008), moe_fp8_packed_weights_bytes(), ws, ws_bytes, NULL) == MOE_FP8_EALIGN);
  /* workspace: missing or one byte short */
  valid_args(&a, T);
  CHECK(moe_fp8_run(&a, NULL, L.total_bytes, NULL) == MOE_FP8_EWORKSPACE);
  CHECK(moe_fp8_run(&a, ws, L.total_bytes - 1, NULL) == MOE_FP8_EWORKSPACE);
  CHECK(moe_fp8_route_dispatch(&a, 1, ws, L.total_bytes - 1, NULL) == MOE_FP8_EWORKSPACE);
  CHECK(moe_fp8_gemm2_combine(&a, ws, L.total_bytes - 1, NULL) == MOE_FP8_EWORKSPACE);
  CHECK(moe_fp8_run_profiled(&a, NULL, 0, ws, L.total_bytes - 1, NULL, NULL) != MOE_FP8_OK);
  /* packed weights: missing or too small, checked before anything else */
  CHECK(moe_fp8_run_packed(&a, NULL, moe_fp8_packed_weights_bytes(), ws, L.total_bytes - 1, NULL) ==
        MOE_FP8_EPACKED);
  CHECK(moe_fp8_run_packed(&a, fake(0xa000), moe_fp8_packed_weights_bytes() - 1, ws, L.total_bytes - 1, NULL) ==
        MOE_FP8_EPACKED);
  CHECK(moe_fp8_pack_weights(&a, NULL, moe_fp8_packed_weights_bytes(), NULL) == MOE_FP8_EPACKED);
  CHECK(moe_fp8_pack_weights(&a, fake(0xa000), 16, NULL) == MOE_FP8_EPACKED);
  /* the static entry: more than MOE_FP8_STATIC_MAX_TOKENS tokens, or a missing pointer */
  valid_args(&a, MOE_FP8_STATIC_MAX_TOKENS + 1);
  CHECK(moe_fp8_run_static(&a, NULL) == MOE_FP8_ESTATIC_TOKENS);
}

int main(void) {
  moe_fp8_args a;
  moe_fp8_layout L;
  size_t prev = 0;
  int32_t T;
  int code;
  static char ws_stand_in[64];   /* a non-null workspace address; never written through */

  /* sizes non-decreasing across every regime boundary; layouts consistent */
  for (T = 0; T <= 300; ++T) {
    size_t b = moe_fp8_workspace_bytes(T);
    CHECK(b >= prev);
    prev = b;
    check_layout(T);
  }
  for (T = 4088; T <= 4100; ++T) {
    size_t b = moe_fp8_workspace_bytes(T);
    CHECK(b >= prev);
    prev = b;
    check_layout(T);
  }
  check_layout(8192);
  check_layout(65536);
  check_layout(MOE_FP8_MAX_TOKENS);
  CHECK(moe_fp8_workspace_layout(-1, &L) == MOE_FP8_EINVAL_TOKENS);
  CHECK(moe_fp8_workspace_layout(MOE_FP8_MAX_TOKENS + 1, &L) == MOE_FP8_EINVAL_TOKENS);
  CHECK(moe_fp8_workspace_layout(16, NULL) == MOE_FP8_EINVAL_POINTER);
  CHECK(moe_fp8_workspace_bytes(-5) == 0);

  /* validation of every entry point at sizes of every regime */
  check_entry_points(1, ws_stand_in, sizeof ws_stand_in);
  check_entry_points(64, ws_stand_in, sizeof ws_stand_in);
  check_entry_points(65, ws_stand_in, sizeof ws_stand_in);
  check_entry_points(257, ws_stand_in, sizeof ws_stand_in);
  check_entry_points(4096, ws_stand_in, sizeof ws_stand_in);

  /* token counts out of range */
  valid_args(&a, -1);
  CHECK(moe_fp8_run(&a, ws_stand_in, 1, NULL) == MOE_FP8_EINVAL_TOKENS);
  valid_args(&a, MOE_FP8_MAX_TOKENS + 1);
  CHECK(moe_fp8_run(&a, ws_stand_in, 1, NULL) == MOE_FP8_EINVAL_TOKENS);

  /* the quantiser: dtype, pointers and token count are checked before the device */
  CHECK(moe_fp8_quantize_hidden(fake(0x1000), 9, 16, fake(0x2000), fake(0x3000), NULL) ==
        MOE_FP8_EINVAL_HIDDEN_DTYPE);
  CHECK(moe_fp8_quantize_hidden(NULL, MOE_FP8_HIDDEN_BF16, 16, fake(0x2000), fake(0x3000), NULL) ==
        MOE_FP8_EINVAL_POINTER);
  CHECK(moe_fp8_quantize_hidden(fake(0x1000), MOE_FP8_HIDDEN_BF16, -3, fake(0x2000), fake(0x3000), NULL) ==
        MOE_FP8_EINVAL_TOKENS);
  CHECK(moe_fp8_quantize_hidden(fake(0x1004), MOE_FP8_HIDDEN_BF16, 16, fake(0x2000), fake(0x3000), NULL) ==
        MOE_FP8_EALIGN);
  CHECK(moe_fp8_workspace_init(fake(0x1040), 4096, NULL) == MOE_FP8_EALIGN);

  /* the workspace clear: null or too small for the control block */
  CHECK(moe_fp8_workspace_init(NULL, 4096, NULL) == MOE_FP8_EWORKSPACE);
  CHECK(moe_fp8_workspace_init(ws_stand_in, 4, NULL) == MOE_FP8_EWORKSPACE);

  /* every error text is a non-empty string, unknown codes included */
  for (code = -20; code <= 2; ++code) {
    const char* s = moe_fp8_strerror(code);
    CHECK(s != NULL && strlen(s) > 0);
  }
  CHECK(strncmp(moe_fp8_version(), "moe_fp8 ", 8) == 0);

  if (failures == 0) printf("ok\n");
  return failures == 0 ? 0 : 1;
}
