//! `MoeHipGradFn`: the backward of one MoE layer call, for boostr's autograd.
//!
//! In the reference the layer's backward is the boostr graph built by
//! `boostr::nn::moe::layer::MoeLayer::forward` and walked by `backward_wrt`
//! (`src/trainer.rs:1097`); `backward_and_merge` (`src/trainer.rs:1087-1111`)
//! then accumulates, per parameter id, whatever gradient the walk produced and
//! skips ids without one. An expert that received no token must therefore
//! produce *no* entry, not a zero tensor (`src/trainer.rs:556-566`,
//! `src/model/recompute/segment.rs:284-286`); every expert with a token, the
//! router and the shared expert always get one.
//!
//! boostr's `GradFn` trait (`src/trainer.rs:1148` uses it) lives in the
//! boostr crate, which the reference does not vendor, so its exact method
//! signatures are not restated here. This module holds everything that does
//! not depend on them: the forward that records what the backward needs, the
//! `moe_backward` call, and the parameter-ordered gradient list with the
//! absent entries. A `GradFn` impl in the trainer forwards its backward to
//! [`MoeHipGradFn::backward`] and turns the returned `(param_index, buffer)`
//! pairs into its `GradStore` entries.
//!
//! Two rules keep the backward off the host's critical path:
//! * the scratch comes from one [`SharedWorkspace`] per device and stream,
//!   sized once for the largest batch (layers on one stream run one after
//!   another, so they never use it at the same time); no call allocates it;
//! * which experts get an entry is read from the forward's expert counts,
//!   copied to pinned host memory right after the forward without waiting
//!   ([`RoutedExperts`]). By the time the backward runs that copy has long
//!   completed, so the backward never waits on the stream; `moe_backward`
//!   gets `has_grad = NULL`.

use std::ffi::c_void;
use std::sync::{Arc, Mutex};

use crate::{ffi, grads, weights, ExpertTables, Plan, Result};

/// Device memory, pinned host memory and events of the trainer's runtime
/// (the client's device and stream). The trainer implements it over its
/// runtime; tests can implement it over any HIP allocator.
pub trait DeviceAlloc {
    type Buffer;
    /// Page-locked host memory (device-to-host copies into it run
    /// asynchronously on the stream).
    type Pinned;
    /// A marker recorded on a stream.
    type Event;
    /// A device buffer of `bytes` bytes, 16-byte aligned. Freeing a buffer
    /// (dropping it) must be ordered after the work already enqueued on the
    /// stream that used it, as a stream-ordered caching allocator does.
    fn alloc(&self, bytes: usize) -> Result<Self::Buffer>;
    fn ptr(buf: &Self::Buffer) -> *mut c_void;
    /// Pinned host memory of `bytes` bytes.
    fn alloc_pinned(&self, bytes: usize) -> Result<Self::Pinned>;
    fn pinned_bytes(buf: &Self::Pinned) -> &[u8];
    /// Enqueues a copy of `bytes` bytes from device memory into `dst` on
    /// `stream`, after the work already enqueued there; returns at once.
    fn copy_to_pinned_async(&self, stream: *mut c_void, src: *const c_void,
                            dst: &mut Self::Pinned, bytes: usize) -> Result<()>;
    /// Records an event on `stream` after the work already enqueued there.
    fn record_event(&self, stream: *mut c_void) -> Result<Self::Event>;
    /// Blocks the host until `event` has completed.
    fn event_synchronize(&self, event: &Self::Event) -> Result<()>;
}

/// Scratch shared by every MoE layer call on one device and stream
/// (`moe_workspace_bytes`: 2.7 GB at T = 8192, H = 7168, E = 256). It grows
/// only when a call needs more than it holds; [`SharedWorkspace::reserve`]
/// sizes it for the largest batch once, at model construction, so that no
/// step allocates. Calls on other streams may overlap and need a workspace
/// of their own.
pub struct SharedWorkspace<A: DeviceAlloc> {
    buf: Option<A::Buffer>,
    bytes: usize,
}

impl<A: DeviceAlloc> Default for SharedWorkspace<A> {
    fn default() -> Self {
        SharedWorkspace { buf: None, bytes: 0 }
    }
}

impl<A: DeviceAlloc> SharedWorkspace<A> {
    pub fn new() -> Self {
        Self::default()
    }

    /// Grows the buffer to the workspace of `plan` for `max_tokens` tokens.
    pub fn reserve(&mut self, alloc: &A, plan: &Plan, max_tokens: i64) -> Result<()> {
        self.ensure(alloc, plan.workspace_bytes(max_tokens)).map(|_| ())
    }

    /// The buffer's device address, grown to at least `bytes` first. The old
    /// buffer is dropped through the allocator, which frees it only after the
    /// stream's queued kernels (the `DeviceAlloc::alloc` contract).
    pub fn ensure(&mut self, alloc: &A, bytes: usize) -> Result<*mut c_void> {
        let bytes = bytes.max(1);
        if self.buf.is_none() || self.bytes < bytes {
            self.buf = None;
            self.buf = Some(alloc.alloc(bytes)?);
            self.bytes = bytes;
        }
        Ok(A::ptr(self.buf.as_ref().expect("workspace buffer")))
    }

    /// Bytes currently held.
    pub fn bytes(&self) -> usize {
        self.bytes
    }
}

/// Which experts received a token in one forward: the `counts` field of
/// `saved` (int32 [E]) copied into pinned host memory behind an event,
/// queued right after `moe_forward` and never waited for there.
pub struct RoutedExperts<A: DeviceAlloc> {
    copy: Option<(A::Pinned, A::Event)>,
    num_experts: usize,
}

impl<A: DeviceAlloc> RoutedExperts<A> {
    /// Queues the copy of the forward's counts on `stream` (after the
    /// forward). `num_tokens = 0` routes nothing and copies nothing.
    pub fn record(alloc: &A, plan: &Plan, stream: *mut c_void, num_tokens: i64,
                  saved: *const c_void) -> Result<Self> {
        let num_experts = plan.config.0.num_experts as usize;
        if num_tokens == 0 {
            return Ok(RoutedExperts { copy: None, num_experts });
        }
        let (off, bytes) = plan.saved_field_range(num_tokens, ffi::MOE_SAVED_COUNTS)?;
        let mut host = alloc.alloc_pinned(bytes)?;
        // the field lies inside `saved` (moe_saved_field_range)
        let src = (saved as *const u8).wrapping_add(off) as *const c_void;
        alloc.copy_to_pinned_async(stream, src, &mut host, bytes)?;
        let event = alloc.record_event(stream)?;
        Ok(RoutedExperts { copy: Some((host, event)), num_experts })
    }

    /// One byte per expert: 1 when the expert received a token. Waits for
    /// the copy's event, which completed long before a backward asks.
    pub fn mask(&self, alloc: &A) -> Result<Vec<u8>> {
        let Some((host, event)) = &self.copy else {
            return Ok(vec![0u8; self.num_experts]);
        };
        alloc.event_synchronize(event)?;
        Ok(routed_mask(A::pinned_bytes(host), self.num_experts))
    }
}

/// `counts` (int32 [E], native byte order) to one byte per expert:
/// 1 when the count is positive.
pub fn routed_mask(counts: &[u8], num_experts: usize) -> Vec<u8> {
    counts
        .chunks_exact(4)
        .take(num_experts)
        .map(|c| (i32::from_ne_bytes([c[0], c[1], c[2], c[3]]) > 0) as u8)
        .collect()
}

/// Shapes and element size of one layer (from its `Config`).
#[derive(Clone, Copy, Debug)]
pub struct LayerShape {
    pub hidden: usize,
    pub num_experts: usize,
    pub intermediate: usize,
    pub shared: usize,
    pub elt: usize,
    pub router_bias: bool,
}

impl LayerShape {
    pub fn of(plan: &Plan) -> LayerShape {
        let c = &plan.config.0;
        LayerShape {
            hidden: c.hidden as usize,
            num_experts: c.num_experts as usize,
            intermediate: c.intermediate as usize,
            shared: c.shared_intermediate as usize,
            elt: if c.dtype == ffi::MOE_DTYPE_BF16 { 2 } else { 4 },
            router_bias: c.has_router_bias != 0,
        }
    }
}

/// Position of a parameter in `MoeLayer::trainable_parameters`
/// (`src/model.rs:1887-1897`): router gate (and its bias), then experts
/// 0..E-1 each (gate, up, down), then the shared expert (gate, up, down).
#[derive(Clone, Copy, Debug, PartialEq, Eq)]
pub enum Param {
    RouterGate,
    RouterBias,
    ExpertGate(usize),
    ExpertUp(usize),
    ExpertDown(usize),
    SharedGate,
    SharedUp,
    SharedDown,
}

impl Param {
    /// Index in the reference order, given the layer's shape.
    pub fn index(self, s: &LayerShape) -> usize {
        let base = if s.router_bias { 2 } else { 1 };
        match self {
            Param::RouterGate => 0,
            Param::RouterBias => 1,
            Param::ExpertGate(e) => base + 3 * e,
            Param::ExpertUp(e) => base + 3 * e + 1,
            Param::ExpertDown(e) => base + 3 * e + 2,
            Param::SharedGate => base + 3 * s.num_experts,
            Param::SharedUp => base + 3 * s.num_experts + 1,
            Param::SharedDown => base + 3 * s.num_experts + 2,
        }
    }
}

/// What one forward leaves for its backward: the plan, the call's inputs
/// (device pointers owned by the graph), the `saved` buffer and the routed
/// experts.
pub struct MoeHipGradFn<A: DeviceAlloc> {
    pub plan: Arc<Mutex<Plan>>,
    pub stream: *mut c_void,
    pub num_tokens: i64,
    pub x: *const c_void,
    pub router: *const c_void,
    pub router_bias: *const f32,
    pub experts: ExpertTables<*const c_void>,
    pub shared: Option<[*const c_void; 3]>,
    pub saved: A::Buffer,
    pub routed: RoutedExperts<A>,
}

/// Gradients of one backward: `dx` and `(parameter, buffer)` pairs in the
/// reference's parameter order, with no pair for an expert that received no
/// token.
pub struct MoeHipGrads<B> {
    pub dx: B,
    pub params: Vec<(Param, B)>,
}

impl<A: DeviceAlloc> MoeHipGradFn<A> {
    /// `MoeLayer::forward` (`src/model.rs:1834-1885`) over x [T, H] on
    /// `stream`: allocates `saved` (owned by the graph, like the reference's
    /// activations), takes the scratch from `workspace`, calls `moe_forward`
    /// into `out` / `aux` / `z` and queues the copy of the expert counts.
    /// Returns what the backward needs.
    ///
    /// # Safety
    /// Every pointer must be a device buffer of the size the header states
    /// for `num_tokens`, valid until the backward has run on the stream.
    #[allow(clippy::too_many_arguments)]
    pub unsafe fn forward(plan: Arc<Mutex<Plan>>, alloc: &A, workspace: &mut SharedWorkspace<A>,
                          stream: *mut c_void, num_tokens: i64, x: *const c_void,
                          router: *const c_void, router_bias: *const f32,
                          experts: ExpertTables<*const c_void>,
                          shared: Option<[*const c_void; 3]>, out: *mut c_void, aux: *mut f32,
                          z: *mut f32) -> Result<Self> {
        let routed;
        let saved;
        {
            let mut p = plan.lock().expect("moe plan lock");
            saved = alloc.alloc(p.saved_bytes(num_tokens).max(1))?;
            let ws = workspace.ensure(alloc, p.workspace_bytes(num_tokens))?;
            let w = weights(router, router_bias, &experts, shared);
            p.forward(stream, num_tokens, x, &w, out, aux, z, A::ptr(&saved), ws)?;
            routed = RoutedExperts::record(alloc, &p, stream, num_tokens, A::ptr(&saved))?;
        }
        Ok(MoeHipGradFn { plan, stream, num_tokens, x, router, router_bias, experts, shared,
                          saved, routed })
    }

    /// The backward of the three outputs `(out, aux_loss, z_loss)`: `d_out`
    /// [T, H] and the device scalars `d_aux`, `d_z` (the trainer's alpha / n
    /// and gamma / n, `src/trainer.rs:399-421`; null for 0). The scratch
    /// comes from `workspace`, the gradient tensors from `alloc` (fresh
    /// parameter-shaped tensors, as the reference's graph produces); nothing
    /// waits on the stream.
    pub fn backward(&self, alloc: &A, workspace: &mut SharedWorkspace<A>, d_out: *const c_void,
                    d_aux: *const f32, d_z: *const f32) -> Result<MoeHipGrads<A::Buffer>> {
        let mut plan = self.plan.lock().expect("moe plan lock");
        let s = LayerShape::of(&plan);
        let (h, e, i, sh, b) = (s.hidden, s.num_experts, s.intermediate, s.shared, s.elt);
        let t = self.num_tokens as usize;
        let mask = self.routed.mask(alloc)?;
        let ws = workspace.ensure(alloc, plan.workspace_bytes(self.num_tokens))?;
        let dx = alloc.alloc((t * h * b).max(1))?;
        let router = alloc.alloc(e * h * b)?;
        let bias = if s.router_bias { Some(alloc.alloc(e * 4)?) } else { None };
        let mut gate = Vec::with_capacity(e);
        let mut up = Vec::with_capacity(e);
        let mut down = Vec::with_capacity(e);
        for _ in 0..e {
            gate.push(alloc.alloc(i * h * b)?);
            up.push(alloc.alloc(i * h * b)?);
            down.push(alloc.alloc(h * i * b)?);
        }
        let shared = if sh > 0 {
            Some([alloc.alloc(sh * h * b)?, alloc.alloc(sh * h * b)?, alloc.alloc(h * sh * b)?])
        } else {
            None
        };
        let g_tables = ExpertTables {
            gate: gate.iter().map(A::ptr).collect(),
            up: up.iter().map(A::ptr).collect(),
            down: down.iter().map(A::ptr).collect(),
        };
        let g = grads(A::ptr(&router), bias.as_ref().map_or(std::ptr::null_mut(), |x| A::ptr(x) as *mut f32),
                      &g_tables, shared.as_ref().map(|s| [A::ptr(&s[0]), A::ptr(&s[1]), A::ptr(&s[2])]));
        let w = weights(self.router, self.router_bias, &self.experts, self.shared);
        // SAFETY: every pointer is a live device buffer of the header's size
        // for num_tokens; `saved` is the buffer this layer's forward filled;
        // has_grad is not requested (the forward's counts give the mask).
        unsafe {
            plan.backward(self.stream, self.num_tokens, d_out, d_aux, d_z, self.x, &w,
                          A::ptr(&self.saved), ws, A::ptr(&dx), &g, std::ptr::null_mut())?;
        }
        Ok(MoeHipGrads { dx, params: ordered(mask, router, bias, gate, up, down, shared) })
    }
}

/// The gradient list in the reference's parameter order; experts whose
/// routed byte is 0 contribute no pair (their buffers were left untouched by
/// the library and are dropped here).
pub fn ordered<B>(routed: Vec<u8>, router: B, bias: Option<B>, gate: Vec<B>, up: Vec<B>,
                  down: Vec<B>, shared: Option<[B; 3]>) -> Vec<(Param, B)> {
    let mut out = vec![(Param::RouterGate, router)];
    if let Some(b) = bias {
        out.push((Param::RouterBias, b));
    }
    for (ex, ((g, u), d)) in gate.into_iter().zip(up).zip(down).enumerate() {
        if routed[ex] == 0 {
            continue; // no token reached this expert: no gradient entry
        }
        out.push((Param::ExpertGate(ex), g));
        out.push((Param::ExpertUp(ex), u));
        out.push((Param::ExpertDown(ex), d));
    }
    if let Some([g, u, d]) = shared {
        out.push((Param::SharedGate, g));
        out.push((Param::SharedUp, u));
        out.push((Param::SharedDown, d));
    }
    out
}

#[cfg(test)]
mod tests {
    use super::*;

    #[test]
    fn unrouted_experts_get_no_entry_and_order_follows_the_reference() {
        let out = ordered(vec![1, 0, 1], "r", Some("b"), vec!["g0", "g1", "g2"],
                          vec!["u0", "u1", "u2"], vec!["d0", "d1", "d2"], Some(["sg", "su", "sd"]));
        let names: Vec<_> = out.iter().map(|(_, b)| *b).collect();
        assert_eq!(names, ["r", "b", "g0", "u0", "d0", "g2", "u2", "d2", "sg", "su", "sd"]);
        let s = LayerShape { hidden: 8, num_experts: 3, intermediate: 4, shared: 4, elt: 2,
                             router_bias: true };
        let idx: Vec<_> = out.iter().map(|(p, _)| p.index(&s)).collect();
        assert_eq!(idx, [0, 1, 2, 3, 4, 8, 9, 10, 11, 12, 13]);
    }

    #[test]
    fn routed_mask_reads_positive_counts() {
        let counts: Vec<u8> = [3i32, 0, 1, 0].iter().flat_map(|c| c.to_ne_bytes()).collect();
        assert_eq!(routed_mask(&counts, 4), [1, 0, 1, 0]);
    }
}
