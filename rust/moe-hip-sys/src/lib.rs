//! Rust binding of `libmoe_hip.so`, the MI355X (gfx950) Mixture-of-Experts
//! layer declared in `include/moe_hip.h`.
//!
//! oxidizr's MoE layer is `struct MoeLayer<R> { moe: boostr::nn::moe::layer::MoeLayer<R> }`
//! (reference `src/model.rs:1632-1634`); its forward returns `(out, aux_loss,
//! z_loss)` (`src/model.rs:1834-1885`) and its backward is the boostr autograd
//! graph walked by `backward_wrt` (`src/trainer.rs:1097`). This crate is the
//! thin FFI layer a Rust caller links instead of that inner field:
//!
//! * [`ffi`]: the `extern "C"` block and `#[repr(C)]` structs, one to one with
//!   the header;
//! * [`Plan`], [`Config`], [`MoeHipError`]: a safe owner of a `moe_plan`
//!   (destroyed on drop) whose calls map status codes to errors, with
//!   [`MoeHipError::is_oom`] for the trainer's out-of-memory guard
//!   (`src/oom_guard.rs:24-45`);
//! * [`grad`]: `MoeHipGradFn`, the three-output backward that leaves no
//!   gradient entry for an expert no token reached (`src/trainer.rs:556-566`).
//!
//! Every tensor argument is a device pointer (HIP), 16-byte aligned,
//! row-major; per-expert weights are host arrays of device pointers because
//! oxidizr keeps each expert projection as its own tensor
//! (`src/model.rs:1661-1672`).

use std::ffi::{c_void, CStr};
use std::fmt;

pub mod grad;

/// Raw declarations of `include/moe_hip.h`.
pub mod ffi {
    use std::ffi::c_void;
    use std::os::raw::c_char;

    pub type MoeStatus = i32;
    pub const MOE_OK: MoeStatus = 0;
    pub const MOE_ERR_INVALID: MoeStatus = 1;
    pub const MOE_ERR_OOM: MoeStatus = 2;
    pub const MOE_ERR_HIP: MoeStatus = 3;
    pub const MOE_ERR_UNSUPPORTED: MoeStatus = 4;

    pub const MOE_DTYPE_F32: i32 = 0;
    pub const MOE_DTYPE_BF16: i32 = 1;

    /// `moe_saved_field` indices.
    pub const MOE_SAVED_LOGITS: i32 = 0;
    pub const MOE_SAVED_PROBS: i32 = 1;
    pub const MOE_SAVED_LSE: i32 = 2;
    pub const MOE_SAVED_TOPK_IDX: i32 = 3;
    pub const MOE_SAVED_TOPK_W: i32 = 4;
    pub const MOE_SAVED_COUNTS: i32 = 5;
    pub const MOE_SAVED_OFFSETS: i32 = 6;
    pub const MOE_SAVED_PERM: i32 = 7;
    pub const MOE_SAVED_INV_PERM: i32 = 8;
    pub const MOE_SAVED_MEAN_PROB: i32 = 9;
    pub const MOE_NUM_STAGES: usize = 20;

    #[repr(C)]
    #[derive(Clone, Copy, Debug, Default)]
    pub struct MoeConfigC {
        pub hidden: i32,
        pub num_experts: i32,
        pub experts_per_tok: i32,
        pub intermediate: i32,
        pub shared_intermediate: i32,
        pub dtype: i32,
        pub norm_topk_prob: i32,
        pub has_router_bias: i32,
        pub router_temperature: f32,
        pub shared_expert_scale: f32,
        pub aux_switch_coef: f32,
        pub aux_sqprob_coef: f32,
        pub recompute_activations: i32,
        pub fused_block: i32,
        pub rms_norm_eps: f32,
    }

    #[repr(C)]
    #[derive(Clone, Copy, Debug)]
    pub struct MoeWeightsC {
        pub router: *const c_void,
        pub router_bias: *const f32,
        pub gate: *const *const c_void,
        pub up: *const *const c_void,
        pub down: *const *const c_void,
        pub shared_gate: *const c_void,
        pub shared_up: *const c_void,
        pub shared_down: *const c_void,
    }

    #[repr(C)]
    #[derive(Clone, Copy, Debug)]
    pub struct MoeGradsC {
        pub router: *mut c_void,
        pub router_bias: *mut f32,
        pub gate: *const *mut c_void,
        pub up: *const *mut c_void,
        pub down: *const *mut c_void,
        pub shared_gate: *mut c_void,
        pub shared_up: *mut c_void,
        pub shared_down: *mut c_void,
    }

    /// Opaque `moe_plan`.
    #[repr(C)]
    pub struct MoePlan {
        _private: [u8; 0],
    }

    extern "C" {
        pub fn moe_config_default(cfg: *mut MoeConfigC, hidden: i32, num_experts: i32,
                                  experts_per_tok: i32, intermediate: i32,
                                  shared_intermediate: i32);
        pub fn moe_plan_create(cfg: *const MoeConfigC, device: i32,
                               plan: *mut *mut MoePlan) -> MoeStatus;
        pub fn moe_plan_destroy(plan: *mut MoePlan) -> MoeStatus;
        pub fn moe_check_tokens(cfg: *const MoeConfigC, num_tokens: i64) -> MoeStatus;
        pub fn moe_workspace_check(cfg: *const MoeConfigC, num_tokens: i64) -> MoeStatus;
        pub fn moe_saved_bytes(plan: *const MoePlan, num_tokens: i64) -> usize;
        pub fn moe_workspace_bytes(plan: *const MoePlan, num_tokens: i64) -> usize;
        pub fn moe_forward(plan: *mut MoePlan, stream: *mut c_void, num_tokens: i64,
                           x: *const c_void, w: *const MoeWeightsC, out: *mut c_void,
                           aux_loss: *mut f32, z_loss: *mut f32, saved: *mut c_void,
                           workspace: *mut c_void) -> MoeStatus;
        pub fn moe_forward_noalloc(plan: *mut MoePlan, stream: *mut c_void, num_tokens: i64,
                                   x: *const c_void, w: *const MoeWeightsC, out: *mut c_void,
                                   aux_loss: *mut f32, z_loss: *mut f32) -> MoeStatus;
        pub fn moe_backward(plan: *mut MoePlan, stream: *mut c_void, num_tokens: i64,
                            d_out: *const c_void, d_aux: *const f32, d_z: *const f32,
                            x: *const c_void, w: *const MoeWeightsC, saved: *const c_void,
                            workspace: *mut c_void, dx: *mut c_void, g: *const MoeGradsC,
                            has_grad: *mut u8) -> MoeStatus;
        pub fn moe_block_forward(plan: *mut MoePlan, stream: *mut c_void, num_tokens: i64,
                                 h: *const c_void, norm_weight: *const c_void,
                                 w: *const MoeWeightsC, out: *mut c_void, aux_loss: *mut f32,
                                 z_loss: *mut f32, saved: *mut c_void,
                                 workspace: *mut c_void) -> MoeStatus;
        pub fn moe_block_backward(plan: *mut MoePlan, stream: *mut c_void, num_tokens: i64,
                                  d_out: *const c_void, d_aux: *const f32, d_z: *const f32,
                                  h: *const c_void, norm_weight: *const c_void,
                                  w: *const MoeWeightsC, saved: *const c_void,
                                  workspace: *mut c_void, dh: *mut c_void,
                                  d_norm_weight: *mut c_void, g: *const MoeGradsC,
                                  has_grad: *mut u8) -> MoeStatus;
        pub fn moe_route_from_logits(plan: *mut MoePlan, stream: *mut c_void, num_tokens: i64,
                                     logits: *const f32, saved: *mut c_void,
                                     workspace: *mut c_void) -> MoeStatus;
        pub fn moe_saved_field_range(plan: *const MoePlan, num_tokens: i64, field: i32,
                                     offset: *mut usize, bytes: *mut usize) -> MoeStatus;
        pub fn moe_stage_name(stage: i32) -> *const c_char;
        pub fn moe_plan_set_profiling(plan: *mut MoePlan, stage_mask: i32) -> MoeStatus;
        pub fn moe_plan_set_shared_overlap(plan: *mut MoePlan, on: i32) -> MoeStatus;
        pub fn moe_plan_stage_times(plan: *mut MoePlan, ms: *mut f32, calls: *mut i32,
                                    reset: i32) -> MoeStatus;
        pub fn moe_last_error() -> *const c_char;
        pub fn moe_version() -> *const c_char;
    }
}

/// A failed call: the status code and `moe_last_error()` of the calling thread.
#[derive(Clone, Debug, PartialEq, Eq)]
pub struct MoeHipError {
    pub status: i32,
    pub message: String,
}

impl MoeHipError {
    /// Device memory ran out (plan creation): the trainer maps this to its
    /// out-of-memory guard instead of a model error.
    pub fn is_oom(&self) -> bool {
        self.status == ffi::MOE_ERR_OOM
    }
}

impl fmt::Display for MoeHipError {
    fn fmt(&self, f: &mut fmt::Formatter<'_>) -> fmt::Result {
        write!(f, "moe_hip status {}: {}", self.status, self.message)
    }
}

impl std::error::Error for MoeHipError {}

pub type Result<T> = std::result::Result<T, MoeHipError>;

/// Maps a status to `Ok` or the thread's last error message.
pub fn check(status: i32) -> Result<()> {
    if status == ffi::MOE_OK {
        return Ok(());
    }
    // SAFETY: moe_last_error returns a NUL-terminated thread-local string
    // that stays valid until the next call on this thread.
    let message = unsafe { CStr::from_ptr(ffi::moe_last_error()) }.to_string_lossy().into_owned();
    Err(MoeHipError { status, message })
}

/// Layer configuration with the reference's keys (`num_experts`,
/// `experts_per_tok`, `moe.intermediate_size`, `shared_expert_enabled`;
/// reference `src/config.rs:125-131`) and the documented defaults of the
/// boostr router constants the reference does not pin.
#[derive(Clone, Copy, Debug)]
pub struct Config(pub ffi::MoeConfigC);

impl Config {
    /// `shared_width` is the total shared-expert width: the routed
    /// intermediate size when `shared_expert_enabled` (None means true,
    /// `src/config.rs:127-129`), 0 otherwise.
    pub fn new(hidden: i32, num_experts: i32, experts_per_tok: i32, intermediate: i32,
               shared_width: i32, bf16: bool) -> Config {
        let mut c = ffi::MoeConfigC::default();
        // SAFETY: c is a valid, writable MoeConfigC.
        unsafe {
            ffi::moe_config_default(&mut c, hidden, num_experts, experts_per_tok, intermediate,
                                    shared_width)
        };
        c.dtype = if bf16 { ffi::MOE_DTYPE_BF16 } else { ffi::MOE_DTYPE_F32 };
        Config(c)
    }

    /// Validation of `required_moe_dims` (`src/model.rs:1927-1958`) and the
    /// token limit of this implementation, without a device.
    pub fn check_tokens(&self, num_tokens: i64) -> Result<()> {
        // SAFETY: self.0 is a valid MoeConfigC.
        check(unsafe { ffi::moe_check_tokens(&self.0, num_tokens) })
    }
}

/// Per-expert device pointer tables of one call, kept alive while the call
/// reads them (the library copies them before it returns).
pub struct ExpertTables<P> {
    pub gate: Vec<P>,
    pub up: Vec<P>,
    pub down: Vec<P>,
}

/// A `moe_plan` bound to one device; destroyed on drop. Calls on one plan
/// must be ordered on one stream (the plan is not `Sync`).
pub struct Plan {
    raw: *mut ffi::MoePlan,
    pub config: Config,
}

// A plan may move to another thread; it is not shared between threads.
unsafe impl Send for Plan {}

impl Plan {
    /// Replaces `MoeLayer::new` / `with_ids` validation (`src/model.rs:1640-1772`).
    pub fn new(config: Config, device: i32) -> Result<Plan> {
        let mut raw = std::ptr::null_mut();
        // SAFETY: config.0 is valid; raw receives the plan or stays NULL.
        check(unsafe { ffi::moe_plan_create(&config.0, device, &mut raw) })?;
        Ok(Plan { raw, config })
    }

    pub fn saved_bytes(&self, num_tokens: i64) -> usize {
        // SAFETY: self.raw is a live plan.
        unsafe { ffi::moe_saved_bytes(self.raw, num_tokens) }
    }

    pub fn workspace_bytes(&self, num_tokens: i64) -> usize {
        // SAFETY: self.raw is a live plan.
        unsafe { ffi::moe_workspace_bytes(self.raw, num_tokens) }
    }

    pub fn raw(&self) -> *mut ffi::MoePlan {
        self.raw
    }

    /// `moe_forward` (`saved` null for a forward-only call, the reference's
    /// eval under no_grad, `src/eval/run.rs:74`).
    ///
    /// # Safety
    /// Every pointer must be a device buffer of the size the header states for
    /// `num_tokens`, valid until the stream has run the call.
    #[allow(clippy::too_many_arguments)]
    pub unsafe fn forward(&mut self, stream: *mut c_void, num_tokens: i64, x: *const c_void,
                          w: &ffi::MoeWeightsC, out: *mut c_void, aux: *mut f32, z: *mut f32,
                          saved: *mut c_void, workspace: *mut c_void) -> Result<()> {
        check(ffi::moe_forward(self.raw, stream, num_tokens, x, w, out, aux, z, saved, workspace))
    }

    /// `moe_backward`: writes `dx`, every weight gradient of an expert that
    /// received a token, and `has_grad` (device, E bytes).
    ///
    /// # Safety
    /// As for [`Plan::forward`]; `saved` is the buffer the forward filled.
    #[allow(clippy::too_many_arguments)]
    pub unsafe fn backward(&mut self, stream: *mut c_void, num_tokens: i64, d_out: *const c_void,
                           d_aux: *const f32, d_z: *const f32, x: *const c_void,
                           w: &ffi::MoeWeightsC, saved: *const c_void, workspace: *mut c_void,
                           dx: *mut c_void, g: &ffi::MoeGradsC, has_grad: *mut u8) -> Result<()> {
        check(ffi::moe_backward(self.raw, stream, num_tokens, d_out, d_aux, d_z, x, w, saved,
                                workspace, dx, g, has_grad))
    }

    /// Byte range of one field of `saved` (e.g. `MOE_SAVED_COUNTS`).
    pub fn saved_field_range(&self, num_tokens: i64, field: i32) -> Result<(usize, usize)> {
        let (mut off, mut bytes) = (0usize, 0usize);
        // SAFETY: self.raw is a live plan; off and bytes are writable.
        check(unsafe { ffi::moe_saved_field_range(self.raw, num_tokens, field, &mut off, &mut bytes) })?;
        Ok((off, bytes))
    }
}

impl Drop for Plan {
    fn drop(&mut self) {
        if !self.raw.is_null() {
            // SAFETY: self.raw came from moe_plan_create and is destroyed once.
            unsafe { ffi::moe_plan_destroy(self.raw) };
            self.raw = std::ptr::null_mut();
        }
    }
}

/// `moe_weights` over per-expert pointer tables (host arrays of device pointers).
pub fn weights(router: *const c_void, router_bias: *const f32,
               tables: &ExpertTables<*const c_void>,
               shared: Option<[*const c_void; 3]>) -> ffi::MoeWeightsC {
    let [sg, su, sd] = shared.unwrap_or([std::ptr::null(); 3]);
    ffi::MoeWeightsC {
        router,
        router_bias,
        gate: tables.gate.as_ptr(),
        up: tables.up.as_ptr(),
        down: tables.down.as_ptr(),
        shared_gate: sg,
        shared_up: su,
        shared_down: sd,
    }
}

/// `moe_grads` over per-expert gradient pointer tables.
pub fn grads(router: *mut c_void, router_bias: *mut f32, tables: &ExpertTables<*mut c_void>,
             shared: Option<[*mut c_void; 3]>) -> ffi::MoeGradsC {
    let [sg, su, sd] = shared.unwrap_or([std::ptr::null_mut(); 3]);
    ffi::MoeGradsC {
        router,
        router_bias,
        gate: tables.gate.as_ptr(),
        up: tables.up.as_ptr(),
        down: tables.down.as_ptr(),
        shared_gate: sg,
        shared_up: su,
        shared_down: sd,
    }
}

/// The library's version string (names the target, gfx950).
pub fn version() -> String {
    // SAFETY: moe_version returns a static NUL-terminated string.
    unsafe { CStr::from_ptr(ffi::moe_version()) }.to_string_lossy().into_owned()
}
