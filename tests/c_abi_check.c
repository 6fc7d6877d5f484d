/* A plain C caller of include/moe_hip.h, built with gcc against
 * libmoe_hip.so: the binding surface a Rust (or any C-ABI) wrapper uses.
 * Runs without a GPU: it exercises only the entry points that need no device
 * (config defaults, validation before any device call, the token-count limit,
 * error codes and moe_last_error), the paths oxidizr's MoeLayer::new /
 * required_moe_dims (src/model.rs:1640-1705, :1927-1958) map onto.
 * Prints one line per check and exits non-zero on the first failure. */
#include <stdio.h>
#include <string.h>

#include "moe_hip.h"

static int failures = 0;

static void expect(int cond, const char* what) {
  printf("%s %s\n", cond ? "ok  " : "FAIL", what);
  if (!cond) ++failures;
}

int main(void) {
  moe_config c;
  moe_plan* plan = (moe_plan*)0x1;

  /* defaults: tau = 1, s = 1, unit aux coefficients, bf16, no bias, kept activations */
  moe_config_default(&c, 2048, 16, 2, 1408, 2816);
  expect(c.hidden == 2048 && c.num_experts == 16 && c.experts_per_tok == 2 &&
             c.intermediate == 1408 && c.shared_intermediate == 2816,
         "moe_config_default keeps the layer dimensions");
  expect(c.dtype == MOE_DTYPE_BF16 && c.router_temperature == 1.0f &&
             c.shared_expert_scale == 1.0f && c.aux_switch_coef == 1.0f &&
             c.aux_sqprob_coef == 1.0f && c.norm_topk_prob == 0 && c.has_router_bias == 0 &&
             c.recompute_activations == 0 && c.fused_block == 0,
         "moe_config_default sets the documented constants");
  expect(moe_check_tokens(&c, 8192) == MOE_OK, "8192 tokens are supported");
  expect(moe_check_tokens(&c, 0) == MOE_OK, "an empty batch is supported");
  expect(moe_check_tokens(&c, -1) == MOE_ERR_INVALID &&
             strstr(moe_last_error(), "negative") != NULL,
         "a negative token count is invalid");

  /* 32-bit buffer offsets: T * max(H, I, S, E8) * 2 bytes must stay below 2^31 */
  moe_config_default(&c, 7168, 256, 8, 2048, 2048);
  expect(moe_check_tokens(&c, 149796) == MOE_OK, "config 5 width: 149796 tokens fit");
  expect(moe_check_tokens(&c, 149797) == MOE_ERR_UNSUPPORTED &&
             strstr(moe_last_error(), "2^31") != NULL,
         "config 5 width: 149797 tokens exceed the 32-bit operand extent");
  c.dtype = MOE_DTYPE_F32;
  expect(moe_check_tokens(&c, 74898) == MOE_OK && moe_check_tokens(&c, 74899) == MOE_ERR_UNSUPPORTED,
         "fp32 halves the token limit");

  /* validation messages of required_moe_dims, returned before any device call */
  moe_config_default(&c, 64, 4, 5, 32, 0);
  expect(moe_plan_create(&c, 0, &plan) == MOE_ERR_INVALID && plan == NULL &&
             strstr(moe_last_error(), "must not exceed num_experts") != NULL,
         "experts_per_tok > num_experts is refused with the reference's message");
  moe_config_default(&c, 64, 4, 2, 0, 0);
  expect(moe_plan_create(&c, 0, &plan) == MOE_ERR_INVALID &&
             strstr(moe_last_error(), "intermediate_size must be non-zero") != NULL,
         "intermediate_size 0 is refused with the reference's message");
  moe_config_default(&c, 60, 4, 2, 32, 0);
  expect(moe_check_tokens(&c, 16) == MOE_ERR_INVALID &&
             strstr(moe_last_error(), "multiple of 8") != NULL,
         "hidden not a multiple of 8 is invalid");
  moe_config_default(&c, 64, 32, 17, 32, 0);
  expect(moe_check_tokens(&c, 16) == MOE_ERR_UNSUPPORTED, "experts_per_tok above 16 is unsupported");
  moe_config_default(&c, 32768, 4, 2, 32768, 0);
  expect(moe_check_tokens(&c, 1) == MOE_ERR_UNSUPPORTED &&
             strstr(moe_last_error(), "weight matrix") != NULL,
         "a 2 GiB weight matrix is unsupported");
  moe_config_default(&c, 64, 4, 2, 32, 0);
  c.router_temperature = 0.0f;
  expect(moe_check_tokens(&c, 16) == MOE_ERR_INVALID, "a zero router temperature is invalid");

  /* NULL handles are errors, not crashes */
  expect(moe_plan_destroy(NULL) == MOE_OK, "destroying a NULL plan is a no-op");
  expect(moe_saved_bytes(NULL, 16) == 0 && moe_workspace_bytes(NULL, 16) == 0,
         "buffer sizes of a NULL plan are 0");
  expect(moe_forward(NULL, NULL, 4, NULL, NULL, NULL, NULL, NULL, NULL, NULL) == MOE_ERR_INVALID &&
             strstr(moe_last_error(), "NULL") != NULL,
         "moe_forward on a NULL plan is MOE_ERR_INVALID");
  expect(moe_plan_create(NULL, 0, &plan) == MOE_ERR_INVALID, "a NULL config is invalid");
  expect(strstr(moe_version(), "gfx950") != NULL, "moe_version names gfx950");
  printf("%d failure(s)\n", failures);
  return failures ? 1 : 0;
}
