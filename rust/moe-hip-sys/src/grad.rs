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
//! not depend on them: the state a forward hands to the backward, the
//! `moe_backward` call, and the parameter-ordered gradient list with the
//! absent entries. A `GradFn` impl in the trainer forwards its backward to
//! [`MoeHipGradFn::backward`] and turns the returned `(param_index, buffer)`
//! pairs into its `GradStore` entries.

use std::ffi::c_void;
use std::sync::{Arc, Mutex};

use crate::{ffi, grads, weights, ExpertTables, Plan, Result};

/// Device memory the gradients are written into. The trainer implements it
/// over its runtime's tensors (allocation on the client's device, raw pointer
/// access); tests can implement it over any device allocator.
pub trait DeviceAlloc {
    type Buffer;
    /// A device buffer of `bytes` bytes, 16-byte aligned.
    fn alloc(&self, bytes: usize) -> Result<Self::Buffer>;
    fn ptr(buf: &Self::Buffer) -> *mut c_void;
    /// Copies `n` bytes from device memory to the host, ordered after the
    /// work already enqueued on `stream` (one small copy per backward: the
    /// `has_grad` mask).
    fn copy_to_host(&self, stream: *mut c_void, src: *const c_void, dst: &mut [u8]) -> Result<()>;
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
/// (device pointers owned by the graph) and the `saved` buffer.
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
}

/// Gradients of one backward: `dx` and `(parameter, buffer)` pairs in the
/// reference's parameter order, with no pair for an expert that received no
/// token.
pub struct MoeHipGrads<B> {
    pub dx: B,
    pub params: Vec<(Param, B)>,
}

impl<A: DeviceAlloc> MoeHipGradFn<A> {
    /// The backward of the three outputs `(out, aux_loss, z_loss)`: `d_out`
    /// [T, H] and the device scalars `d_aux`, `d_z` (the trainer's alpha / n
    /// and gamma / n, `src/trainer.rs:399-421`; null for 0).
    pub fn backward(&self, alloc: &A, d_out: *const c_void, d_aux: *const f32, d_z: *const f32)
        -> Result<MoeHipGrads<A::Buffer>> {
        let mut plan = self.plan.lock().expect("moe plan lock");
        let s = LayerShape::of(&plan);
        let (h, e, i, sh, b) = (s.hidden, s.num_experts, s.intermediate, s.shared, s.elt);
        let t = self.num_tokens as usize;
        let dx = alloc.alloc(t * h * b)?;
        let workspace = alloc.alloc(plan.workspace_bytes(self.num_tokens).max(1))?;
        let has_grad = alloc.alloc(e.max(16))?;
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
        // for num_tokens; `saved` is the buffer this layer's forward filled.
        unsafe {
            plan.backward(self.stream, self.num_tokens, d_out, d_aux, d_z, self.x, &w,
                          A::ptr(&self.saved), A::ptr(&workspace), A::ptr(&dx), &g,
                          A::ptr(&has_grad) as *mut u8)?;
        }
        let mut mask = vec![0u8; e];
        alloc.copy_to_host(self.stream, A::ptr(&has_grad), &mut mask)?;
        Ok(MoeHipGrads { dx, params: ordered(mask, router, bias, gate, up, down, shared) })
    }
}

/// The gradient list in the reference's parameter order; experts whose
/// `has_grad` byte is 0 contribute no pair (their buffers were left
/// untouched by the library and are dropped here).
pub fn ordered<B>(has_grad: Vec<u8>, router: B, bias: Option<B>, gate: Vec<B>, up: Vec<B>,
                  down: Vec<B>, shared: Option<[B; 3]>) -> Vec<(Param, B)> {
    let mut out = vec![(Param::RouterGate, router)];
    if let Some(b) = bias {
        out.push((Param::RouterBias, b));
    }
    for (ex, ((g, u), d)) in gate.into_iter().zip(up).zip(down).enumerate() {
        if has_grad[ex] == 0 {
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
}
