/*
 * moe_hip.h -- C ABI of the MI355X (gfx950) Mixture-of-Experts layer.
 *
 * Drop-in boundary for oxidizr's MoE layer.  In the reference the layer is
 * `struct MoeLayer<R> { moe: boostr::nn::moe::layer::MoeLayer<R> }`
 * (src/model.rs:1632-1634), whose `forward` (src/model.rs:1834-1885) returns
 * (out, aux_loss, z_loss) and whose backward is the boostr autograd graph
 * walked by `backward_wrt` (src/trainer.rs:1097).  A Rust wrapper keeps that
 * struct, its constructors and config keys, and calls these entry points
 * through a thin FFI crate (rust/moe-hip-sys).
 *
 * Conventions
 *  - Every tensor argument is a DEVICE pointer, 16-byte aligned, row-major
 *    and contiguous, in the plan's dtype unless stated.  Linear weights are
 *    [out, in] and applied as y = x W^T (src/model.rs:1422-1445).
 *  - Per-expert weights are HOST arrays of E device pointers, because oxidizr
 *    keeps every expert projection as its own tensor (src/model.rs:1661-1672).
 *  - The caller owns all memory: `saved` (state kept from forward to
 *    backward) and `workspace` (scratch) are caller-allocated device buffers
 *    of moe_saved_bytes / moe_workspace_bytes.  The library allocates only at
 *    plan creation.
 *  - Work is enqueued on `stream` (a hipStream_t); calls do not synchronise
 *    the host.  Calls on one plan must be ordered on one stream.
 *  - Entry points never abort: they return a moe_status and leave a message
 *    for moe_last_error() (thread-local).
 *  - Results are bit-reproducible run to run: no floating-point atomics,
 *    every reduction has a fixed order.
 */
#ifndef MOE_HIP_H
#define MOE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
  MOE_OK = 0,
  MOE_ERR_INVALID = 1,      /* bad argument or configuration */
  MOE_ERR_OOM = 2,          /* device allocation failed (plan creation) */
  MOE_ERR_HIP = 3,          /* HIP runtime error */
  MOE_ERR_UNSUPPORTED = 4   /* valid request this build does not implement */
} moe_status;

typedef enum { MOE_DTYPE_F32 = 0, MOE_DTYPE_BF16 = 1 } moe_dtype;

/* Layer configuration.  Keys follow oxidizr's ModelConfig / TrainerConfig
 * (src/config.rs:125-131, src/config_convert.rs:380-404); the boostr router
 * constants that the reference does not pin are explicit fields. */
typedef struct {
  int32_t hidden;               /* H  = hidden_size                                */
  int32_t num_experts;          /* E  = moe.num_experts (1..1024)                  */
  int32_t experts_per_tok;      /* k  = moe.experts_per_tok (1..min(E,16))         */
  int32_t intermediate;         /* I  = moe.intermediate_size (multiple of 8)      */
  int32_t shared_intermediate;  /* S  = total shared-expert width; 0 = none
                                   (shared_expert_enabled = false)                */
  int32_t dtype;                /* moe_dtype of x, weights, outputs, gradients     */
  int32_t norm_topk_prob;       /* 1: renormalise the k routing weights to sum 1   */
  int32_t has_router_bias;      /* 1: router Linear has a bias [E] (fp32)          */
  float router_temperature;     /* tau: probs = softmax(logits / tau)  (boostr
                                   MOE_ROUTER_TEMPERATURE, src/model.rs:1901)      */
  float shared_expert_scale;    /* s: out += s * shared(x) (src/model.rs:1923)     */
  float aux_switch_coef;        /* aux = E*(c_sw*sum_e f_e P_e + c_sq*sum_e P_e^2)  */
  float aux_sqprob_coef;        /*   (SwitchPlusSquaredProb, src/model.rs:1905)     */
  int32_t recompute_activations;/* 1: `saved` keeps the routing state only and
                                   moe_backward recomputes the expert activations
                                   first (trainer.activation_checkpointing covering
                                   this layer, src/config/activation_checkpointing.rs
                                   :25-35, src/model/recompute/segment.rs:58-170)  */
  int32_t fused_block;          /* 1: the plan runs the block's whole MoE sub-block
                                   through moe_block_forward / moe_block_backward:
                                   post_attention_layernorm (RMSNorm) before the
                                   layer and the residual add after it
                                   (src/model.rs:2792-2800, :2822-2826)           */
  float rms_norm_eps;           /* RMSNorm eps (cfg.rms_norm_eps); fused_block only */
} moe_config;

/* Fills cfg with the documented defaults: tau = 1, s = 1, c_sw = c_sq = 1,
 * no renormalisation, no router bias, bf16, activations kept. */
void moe_config_default(moe_config* cfg, int32_t hidden, int32_t num_experts,
                        int32_t experts_per_tok, int32_t intermediate,
                        int32_t shared_intermediate);

typedef struct moe_plan moe_plan;

/* Replaces MoeLayer::new / with_ids validation (src/model.rs:1640-1772,
 * required_moe_dims :1927-1958).  Binds the plan to `device`. */
moe_status moe_plan_create(const moe_config* cfg, int device, moe_plan** plan);
moe_status moe_plan_destroy(moe_plan* plan);

/* Whether a call over num_tokens tokens is supported by a plan of this
 * configuration, without a device: MOE_OK, MOE_ERR_INVALID (bad config or
 * negative count) or MOE_ERR_UNSUPPORTED (above 2^24 tokens, or an operand of
 * num_tokens x max(H, I, S, E rounded up to 8) elements reaching 2^31 bytes:
 * buffer loads take 32-bit offsets; split such a batch).  The forward and
 * backward entry points make the same check.  No reference counterpart (the
 * limit of this implementation; callers that batch tokens query it). */
moe_status moe_check_tokens(const moe_config* cfg, int64_t num_tokens);

/* Device-free self-check of this implementation's workspace plan for a call
 * over num_tokens tokens: every scratch region a launch uses, sized from the
 * launch's own grid and split arithmetic, fits the region moe_workspace_bytes
 * plans for it, and the regions of the forward (and of the backward) do not
 * overlap.  MOE_OK, or the moe_check_tokens errors, or MOE_ERR_INVALID naming
 * the region that does not fit.  No reference counterpart (a test of this
 * implementation's sizing, callable without a GPU). */
moe_status moe_workspace_check(const moe_config* cfg, int64_t num_tokens);

/* Bytes of the caller-owned buffers for a call over num_tokens tokens. */
size_t moe_saved_bytes(const moe_plan* plan, int64_t num_tokens);
size_t moe_workspace_bytes(const moe_plan* plan, int64_t num_tokens);

typedef struct {
  const void* router;              /* [E, H]   router.gate.weight                 */
  const float* router_bias;        /* [E] fp32 or NULL                             */
  const void* const* gate;         /* E x [I, H]  experts.{e}.gate_proj.weight    */
  const void* const* up;           /* E x [I, H]  experts.{e}.up_proj.weight      */
  const void* const* down;         /* E x [H, I]  experts.{e}.down_proj.weight    */
  const void* shared_gate;         /* [S, H] or NULL  shared_expert.gate_proj     */
  const void* shared_up;           /* [S, H] or NULL  shared_expert.up_proj       */
  const void* shared_down;         /* [H, S] or NULL  shared_expert.down_proj     */
} moe_weights;

typedef struct {
  void* router;                    /* [E, H]                                      */
  float* router_bias;              /* [E] fp32, or NULL (skip)                     */
  void* const* gate;               /* E x [I, H]; expert e written iff has_grad[e] */
  void* const* up;                 /* E x [I, H]                                  */
  void* const* down;               /* E x [H, I]                                  */
  void* shared_gate;               /* [S, H] or NULL                              */
  void* shared_up;                 /* [S, H] or NULL                              */
  void* shared_down;               /* [H, S] or NULL                              */
} moe_grads;

/* Forward over x [T, H] (the reference flattens [B, S, H] to [T, H],
 * src/model.rs:1878).  Writes out [T, H], and the fp32 scalars *aux_loss and
 * *z_loss (device pointers; MoeOutput::aux_loss / z_loss, src/model.rs:1884).
 * `saved` receives routing and activations for moe_backward; it must stay
 * untouched until then.  saved == NULL makes a forward-only call (the
 * need_grad = 0 case: eval under no_grad, src/eval/run.rs:74): no state
 * outlives the call, the routing and activations live in `workspace`, and the
 * gate / up pre-activations that only a backward reads are not computed into
 * memory.  Replaces MoeLayer::forward (src/model.rs:1834). */
moe_status moe_forward(moe_plan* plan, void* stream, int64_t num_tokens, const void* x,
                       const moe_weights* w, void* out, float* aux_loss, float* z_loss,
                       void* saved, void* workspace);

/* Forward-only call (as moe_forward with saved == NULL) that allocates
 * nothing: its scratch is a static device array of the library, 64 MiB per
 * GPU (held until the process ends), instead of a caller workspace, and it
 * creates no events (per-stage profiling is skipped for it).  Returns
 * MOE_ERR_UNSUPPORTED when num_tokens needs more scratch than that (the
 * forward regions of moe_workspace_bytes; decode-sized batches fit).  Every
 * call on one GPU shares that GPU's array, so calls that overlap on one GPU
 * (other streams, other plans, other threads) race; order them.  Under HIP
 * graph capture, call it once eagerly first with the same weight pointer
 * tables: a table change while the stream captures is refused with
 * MOE_ERR_UNSUPPORTED (the upload could not be replayed safely).  A captured
 * call reads the plan's device pointer tables when it replays, so replay it
 * only while the plan's last call used the same tables.  No counterpart in
 * the reference: for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops). */
moe_status moe_forward_noalloc(moe_plan* plan, void* stream, int64_t num_tokens, const void* x,
                               const moe_weights* w, void* out, float* aux_loss, float* z_loss);

/* Backward of the forward that filled `saved` (same x, weights, num_tokens).
 * d_out [T, H]; d_aux, d_z: device fp32 scalars dL/d(aux_loss), dL/d(z_loss)
 * (the trainer's alpha/n and gamma/n, src/trainer.rs:399-421), or NULL for 0.
 * Writes dx [T, H] and every weight gradient (overwriting, not accumulating).
 * has_grad (device uint8 [E], may be NULL) receives 1 for experts that saw at
 * least one token; experts with has_grad 0 have no gradient entry
 * (src/trainer.rs:556-566) and their buffers are left untouched.  With
 * num_tokens = 0 has_grad and the dense gradients (router, router bias, shared
 * expert) are set to zero.  Weight and gradient pointer tables are uploaded
 * when they change, without synchronising the stream.
 * Replaces the boostr GradFn chain walked by backward_wrt (src/trainer.rs:1097). */
moe_status moe_backward(moe_plan* plan, void* stream, int64_t num_tokens, const void* d_out,
                        const float* d_aux, const float* d_z, const void* x,
                        const moe_weights* w, const void* saved, void* workspace, void* dx,
                        const moe_grads* g, uint8_t* has_grad);

/* The MoE sub-block of a decoder block, for plans created with fused_block = 1
 * (src/model.rs:2792-2800 MLA arm, :2822-2826 legacy arm: residual = h;
 * x = post_attention_layernorm(h); (y, aux, z) = ffn(x); out = y + residual).
 * h [T, H]; norm_weight [H] (dtype) is post_attention_layernorm.weight;
 * RMSNorm(h) = h / sqrt(mean(h^2) + rms_norm_eps) * norm_weight with fp32
 * statistics.  The residual add is fused into the combine: out is rounded once.
 * `saved` as for moe_forward (NULL: forward only). */
moe_status moe_block_forward(moe_plan* plan, void* stream, int64_t num_tokens, const void* h,
                             const void* norm_weight, const moe_weights* w, void* out,
                             float* aux_loss, float* z_loss, void* saved, void* workspace);

/* Backward of moe_block_forward: dh [T, H] = d_out (the residual's path) +
 * the RMSNorm backward of the layer's input gradient; d_norm_weight [H]
 * (dtype, overwritten) = sum_t dx_t * h_t * rstd_t, reduced in a fixed order.
 * The layer's weight gradients and has_grad as for moe_backward. */
moe_status moe_block_backward(moe_plan* plan, void* stream, int64_t num_tokens,
                              const void* d_out, const float* d_aux, const float* d_z,
                              const void* h, const void* norm_weight, const moe_weights* w,
                              const void* saved, void* workspace, void* dh,
                              void* d_norm_weight, const moe_grads* g, uint8_t* has_grad);

/* Routing and dispatch only, from given fp32 logits [T, E] (no reference
 * counterpart; lets a caller check top-k and the permutation bit-exactly on
 * identical logits).  Fills the routing fields of `saved`. */
moe_status moe_route_from_logits(moe_plan* plan, void* stream, int64_t num_tokens,
                                 const float* logits, void* saved, void* workspace);

/* Byte offset and size of one field inside `saved` (for tests and callers
 * that want the routing decisions). */
typedef enum {
  MOE_SAVED_LOGITS = 0,   /* fp32 [T, E] */
  MOE_SAVED_PROBS,        /* fp32 [T, E] */
  MOE_SAVED_LSE,          /* fp32 [T] */
  MOE_SAVED_TOPK_IDX,     /* int32 [T, k], slot 0 = largest logit, ties -> lower index */
  MOE_SAVED_TOPK_W,       /* fp32 [T, k] */
  MOE_SAVED_COUNTS,       /* int32 [E] */
  MOE_SAVED_OFFSETS,      /* int32 [E + 1] */
  MOE_SAVED_PERM,         /* int32 [T*k]: expert-major position -> t*k + j */
  MOE_SAVED_INV_PERM,     /* int32 [T*k]: t*k + j -> position */
  MOE_SAVED_MEAN_PROB,    /* fp32 [E]: P_e = mean_t probs[t, e] */
  MOE_SAVED_X_PERM,       /* 0 bytes: the expert GEMMs read each assignment's token
                             row of x through the permutation (no permuted copy) */
  MOE_SAVED_GATE_ACT,     /* dtype [T*k, I]: x W_g^T */
  MOE_SAVED_UP_ACT,       /* dtype [T*k, I]: x W_u^T */
  MOE_SAVED_SWIGLU,       /* dtype [T*k, I]: silu(gate) * up */
  MOE_SAVED_EXPERT_OUT,   /* dtype [T*k, H]: per-assignment expert output; 0 bytes in
                             a training forward's `saved` (the backward does not
                             read it), present in the forward-only state */
  MOE_SAVED_RSTD,         /* fp32 [T]: 1 / RMS of h (fused_block plans only) */
  MOE_SAVED_NORM_X,       /* dtype [T, H]: RMSNorm(h), the layer input (fused_block only) */
  MOE_SAVED_NUM_FIELDS
} moe_saved_field;
moe_status moe_saved_field_range(const moe_plan* plan, int64_t num_tokens, int32_t field,
                                 size_t* offset, size_t* bytes);

/* Per-stage device timing with HIP events recorded on the call's stream
 * around each stage whose bit (1 << moe_stage) is set in stage_mask; -1 times
 * every stage, 0 (the default) none. */
typedef enum {
  MOE_STAGE_ROUTER_GEMM = 0, MOE_STAGE_ROUTE, MOE_STAGE_DISPATCH, MOE_STAGE_GATHER,
  MOE_STAGE_GATEUP_FWD, MOE_STAGE_DOWN_FWD, MOE_STAGE_SHARED_FWD, MOE_STAGE_COMBINE_FWD,
  MOE_STAGE_LOSSES, MOE_STAGE_COMBINE_BWD, MOE_STAGE_DOWN_DGRAD, MOE_STAGE_DOWN_WGRAD,
  MOE_STAGE_GATEUP_DGRAD, MOE_STAGE_GATEUP_WGRAD, MOE_STAGE_SHARED_BWD, MOE_STAGE_ROUTER_BWD,
  MOE_STAGE_DX, MOE_STAGE_RECOMPUTE, MOE_STAGE_NORM_FWD, MOE_STAGE_NORM_BWD, MOE_NUM_STAGES
} moe_stage;
const char* moe_stage_name(int32_t stage);
moe_status moe_plan_set_profiling(moe_plan* plan, int32_t stage_mask);
/* The shared expert runs on a second stream of the plan, and the backward's
 * routed weight gradients on a third (each forked from and joined back into
 * the call's stream inside every call), so that independent GEMMs fill each
 * other's partial rounds of work.  on = 0 runs everything on the call's
 * stream instead (serial order, for per-kernel measurements); on = 2 uses the
 * second stream only; on = 1 is the default.  Results are bitwise the same
 * every way.  No reference counterpart (scheduling knob of this
 * implementation). */
moe_status moe_plan_set_shared_overlap(moe_plan* plan, int32_t on);
/* Synchronises the pending events, then returns the accumulated milliseconds
 * and launch counts per stage since the last reset (arrays of MOE_NUM_STAGES). */
moe_status moe_plan_stage_times(moe_plan* plan, float* ms, int32_t* calls, int32_t reset);

const char* moe_last_error(void);
const char* moe_version(void);

#ifdef __cplusplus
}
#endif
#endif /* MOE_HIP_H */
