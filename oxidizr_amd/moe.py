"""Host-side mirror of oxidizr's MoE layer over the HIP C ABI.

Mirrors `MoeLayer` in the reference (src/model.rs:1632-1958):
  * config keys num_experts, experts_per_tok, intermediate_size,
    shared_expert_enabled (None means true), trainer load_balance_alpha and
    z_loss_alpha (src/config.rs:125-131, :64-67, src/config_convert.rs:380-404);
  * validation messages of required_moe_dims (src/model.rs:1927-1958);
  * parameter names and order: router.gate.weight, experts.{i}.{gate,up,down}_proj.weight,
    shared_expert.{gate,up,down}_proj.weight (src/model.rs:1887-1897, :4890-4910);
  * forward(x [B, S, H]) -> (out, aux_loss, z_loss) (src/model.rs:1834-1885);
  * experts that receive no token get no gradient (src/trainer.rs:556-566):
    their .grad stays None.
PyTorch provides device memory and the stream only; the arithmetic runs in
libmoe_hip.so.
"""
import ctypes
import dataclasses
from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib


class ModelError(ValueError):
    """Configuration error (the reference's boostr::error::Error::ModelError)."""


@dataclass
class MoeConfig:
    hidden_size: int
    num_experts: Optional[int]
    experts_per_tok: Optional[int]
    intermediate_size: Optional[int]
    shared_expert_enabled: Optional[bool] = None
    # Width of the shared expert. The reference builds it with the routed
    # intermediate size (src/model.rs:1680-1684); wider or several shared
    # experts are expressed as one SwiGLU of the summed width.
    shared_intermediate_size: Optional[int] = None
    load_balance_alpha: float = 0.01
    z_loss_alpha: float = 1e-3
    # boostr router constants (MOE_ROUTER_TEMPERATURE, MoeRouterConfig defaults,
    # SwitchPlusSquaredProb coefficients, moe_shared_expert_scale); the
    # reference does not pin their values, these are the documented defaults.
    router_temperature: float = 1.0
    norm_topk_prob: bool = False
    aux_switch_coef: float = 1.0
    aux_sqprob_coef: float = 1.0
    shared_expert_scale: float = 1.0
    router_bias: bool = False
    # trainer.activation_checkpointing covering this layer
    # (src/config/activation_checkpointing.rs:25-35): keep only the routing
    # state between forward and backward and recompute the expert activations.
    recompute_activations: bool = False
    # Block path (moe_block_forward / moe_block_backward): the plan also runs
    # post_attention_layernorm (RMSNorm, cfg.rms_norm_eps) before the layer and
    # the residual add after it (src/model.rs:2792-2800). boostr's
    # default_rms_norm_eps is not pinned by the reference; 1e-6 is the default.
    fused_block: bool = False
    rms_norm_eps: float = 1e-6

    def has_shared_expert(self) -> bool:
        return True if self.shared_expert_enabled is None else bool(self.shared_expert_enabled)

    def required_moe_dims(self):
        """(num_experts, experts_per_tok, intermediate), as src/model.rs:1939-1958."""
        if self.num_experts is None:
            raise ModelError("moe config missing while building an MoE FfnLayer")
        if self.experts_per_tok is None:
            raise ModelError("num_experts set but experts_per_tok is missing")
        if self.intermediate_size is None:
            raise ModelError("MoE requires cfg.moe.intermediate_size")
        if self.intermediate_size == 0:
            raise ModelError("MoE cfg.moe.intermediate_size must be non-zero")
        if self.experts_per_tok > self.num_experts:
            raise ModelError(f"MoE experts_per_tok ({self.experts_per_tok}) must not exceed "
                             f"num_experts ({self.num_experts})")
        return self.num_experts, self.experts_per_tok, self.intermediate_size

    def shared_width(self) -> int:
        if not self.has_shared_expert():
            return 0
        return self.shared_intermediate_size or self.intermediate_size


def _dtype_code(dtype):
    if dtype == torch.bfloat16:
        return _lib.MOE_DTYPE_BF16
    if dtype == torch.float32:
        return _lib.MOE_DTYPE_F32
    raise ModelError(f"unsupported MoE dtype {dtype} (float32 or bfloat16)")


def _p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


# Scratch shared by every plan on a device: a call uses its workspace only
# while its kernels run on the call's stream, so layers that run one after
# another on one stream can share one buffer (sized for the largest call).
# Keyed by (device, stream): calls on different streams may overlap and get
# buffers of their own.
_WORKSPACES = {}


def shared_workspace(device, nbytes):
    """A device buffer of at least nbytes shared per (device, current stream)."""
    stream = torch.cuda.current_stream(device)
    key = (str(device), stream.cuda_stream)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        # the old buffer may still be read by queued kernels: the caching
        # allocator hands it out again only after this stream reaches here
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device)
        _WORKSPACES[key] = ws
    return ws


class Plan:
    """A moe_plan bound to one device, plus reusable scratch buffers."""

    def __init__(self, cfg: MoeConfig, dtype=torch.bfloat16, device=None):
        E, k, I = cfg.required_moe_dims()
        L = _lib.load()
        self.cfg = cfg
        self.dtype = dtype
        self.device = torch.device(device or "cuda")
        c = _lib.MoeConfigC()
        L.moe_config_default(ctypes.byref(c), cfg.hidden_size, E, k, I, cfg.shared_width())
        c.dtype = _dtype_code(dtype)
        c.norm_topk_prob = int(cfg.norm_topk_prob)
        c.has_router_bias = int(cfg.router_bias)
        c.router_temperature = cfg.router_temperature
        c.shared_expert_scale = cfg.shared_expert_scale
        c.aux_switch_coef = cfg.aux_switch_coef
        c.aux_sqprob_coef = cfg.aux_sqprob_coef
        c.recompute_activations = int(cfg.recompute_activations)
        c.fused_block = int(cfg.fused_block)
        c.rms_norm_eps = cfg.rms_norm_eps
        self.c = c
        h = ctypes.c_void_p()
        idx = self.device.index if self.device.index is not None else torch.cuda.current_device()
        self.device = torch.device("cuda", idx)
        _lib.check(L.moe_plan_create(ctypes.byref(c), idx, ctypes.byref(h)))
        self.h = h

    def __del__(self):
        h = getattr(self, "h", None)
        if h:
            _lib.load().moe_plan_destroy(h)
            self.h = None

    # -- buffers
    def saved_bytes(self, T):
        return _lib.load().moe_saved_bytes(self.h, T)

    def workspace_bytes(self, T):
        return _lib.load().moe_workspace_bytes(self.h, T)

    def new_saved(self, T):
        return torch.empty(max(self.saved_bytes(T), 1), dtype=torch.uint8, device=self.device)

    def workspace(self, T):
        return shared_workspace(self.device, self.workspace_bytes(T))

    def check_tokens(self, T):
        """Raises MoeError when a call over T tokens is not supported."""
        _lib.check(_lib.load().moe_check_tokens(ctypes.byref(self.c), T))

    def saved_field(self, saved, T, name):
        """View of one field of a saved buffer as a typed tensor."""
        f = _lib.SAVED_FIELDS.index(name)
        off, nb = ctypes.c_size_t(), ctypes.c_size_t()
        _lib.check(_lib.load().moe_saved_field_range(self.h, T, f, ctypes.byref(off),
                                                     ctypes.byref(nb)))
        if nb.value == 0:
            raise ValueError(f"saved field {name!r} is not kept by this plan (0 bytes)")
        raw = saved[off.value:off.value + nb.value]
        E, k, H, I = self.c.num_experts, self.c.experts_per_tok, self.c.hidden, self.c.intermediate
        shapes = {
            "logits": ((T, E), torch.float32), "probs": ((T, E), torch.float32),
            "lse": ((T,), torch.float32), "topk_idx": ((T, k), torch.int32),
            "topk_w": ((T, k), torch.float32), "counts": ((E,), torch.int32),
            "offsets": ((E + 1,), torch.int32), "perm": ((T * k,), torch.int32),
            "inv_perm": ((T * k,), torch.int32), "mean_prob": ((E,), torch.float32),
            "x_perm": ((T * k, H), self.dtype), "gate_act": ((T * k, I), self.dtype),
            "up_act": ((T * k, I), self.dtype), "swiglu": ((T * k, I), self.dtype),
            "expert_out": ((T * k, H), self.dtype),
        }
        shp, dt = shapes[name]
        return raw.view(dt).view(shp)

    # -- calls
    @staticmethod
    def _stream():
        return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def weights_struct(self, router, gate, up, down, router_bias=None, shared=None):
        w = _lib.MoeWeightsC()
        w.router = router.data_ptr()
        w.router_bias = router_bias.data_ptr() if router_bias is not None else None
        tabs = [_lib.ptr_array([t.data_ptr() for t in ts]) for ts in (gate, up, down)]
        w.gate = ctypes.cast(tabs[0], ctypes.c_void_p)
        w.up = ctypes.cast(tabs[1], ctypes.c_void_p)
        w.down = ctypes.cast(tabs[2], ctypes.c_void_p)
        if shared is not None:
            w.shared_gate, w.shared_up, w.shared_down = (t.data_ptr() for t in shared)
        return w, tabs

    def grads_struct(self, router, gate, up, down, router_bias=None, shared=None):
        g = _lib.MoeGradsC()
        g.router = router.data_ptr()
        g.router_bias = router_bias.data_ptr() if router_bias is not None else None
        tabs = [_lib.ptr_array([t.data_ptr() for t in ts]) for ts in (gate, up, down)]
        g.gate = ctypes.cast(tabs[0], ctypes.c_void_p)
        g.up = ctypes.cast(tabs[1], ctypes.c_void_p)
        g.down = ctypes.cast(tabs[2], ctypes.c_void_p)
        if shared is not None:
            g.shared_gate, g.shared_up, g.shared_down = (t.data_ptr() for t in shared)
        return g, tabs

    def forward(self, x2d, wstruct, out=None, saved=None, aux=None, z=None, need_grad=True):
        """need_grad=False: forward-only call (eval under no_grad); no saved
        state is allocated or returned."""
        T = x2d.shape[0]
        if out is None:
            out = torch.empty_like(x2d)
        if saved is None and need_grad:
            saved = self.new_saved(T)
        if aux is None:
            aux = torch.empty((), dtype=torch.float32, device=self.device)
        if z is None:
            z = torch.empty((), dtype=torch.float32, device=self.device)
        ws = self.workspace(T)
        _lib.check(_lib.load().moe_forward(self.h, self._stream(), T, _p(x2d), ctypes.byref(wstruct),
                                           _p(out), _p(aux), _p(z), _p(saved), _p(ws)))
        return out, aux, z, saved

    def forward_noalloc(self, x2d, wstruct, out, aux, z):
        """Forward-only call into caller-allocated outputs through
        moe_forward_noalloc: the library's static scratch, no workspace."""
        _lib.check(_lib.load().moe_forward_noalloc(self.h, self._stream(), x2d.shape[0], _p(x2d),
                                                   ctypes.byref(wstruct), _p(out), _p(aux),
                                                   _p(z)))
        return out, aux, z

    def backward(self, x2d, dout, wstruct, gstruct, saved, dx=None, d_aux=None, d_z=None,
                 has_grad=None):
        T = x2d.shape[0]
        if dx is None:
            dx = torch.empty_like(x2d)
        ws = self.workspace(T)
        _lib.check(_lib.load().moe_backward(self.h, self._stream(), T, _p(dout), _p(d_aux), _p(d_z),
                                            _p(x2d), ctypes.byref(wstruct), _p(saved), _p(ws),
                                            _p(dx), ctypes.byref(gstruct), _p(has_grad)))
        return dx

    def block_forward(self, h2d, norm_w, wstruct, out=None, saved=None, aux=None, z=None,
                      need_grad=True):
        """out = MoE(RMSNorm(h)) + h on a fused_block plan."""
        T = h2d.shape[0]
        if out is None:
            out = torch.empty_like(h2d)
        if saved is None and need_grad:
            saved = self.new_saved(T)
        if aux is None:
            aux = torch.empty((), dtype=torch.float32, device=self.device)
        if z is None:
            z = torch.empty((), dtype=torch.float32, device=self.device)
        ws = self.workspace(T)
        _lib.check(_lib.load().moe_block_forward(self.h, self._stream(), T, _p(h2d), _p(norm_w),
                                                 ctypes.byref(wstruct), _p(out), _p(aux), _p(z),
                                                 _p(saved), _p(ws)))
        return out, aux, z, saved

    def block_backward(self, h2d, norm_w, dout, wstruct, gstruct, saved, dh=None, d_norm_w=None,
                       d_aux=None, d_z=None, has_grad=None):
        T = h2d.shape[0]
        if dh is None:
            dh = torch.empty_like(h2d)
        if d_norm_w is None:
            d_norm_w = torch.empty_like(norm_w)
        ws = self.workspace(T)
        _lib.check(_lib.load().moe_block_backward(self.h, self._stream(), T, _p(dout), _p(d_aux),
                                                  _p(d_z), _p(h2d), _p(norm_w),
                                                  ctypes.byref(wstruct), _p(saved), _p(ws),
                                                  _p(dh), _p(d_norm_w), ctypes.byref(gstruct),
                                                  _p(has_grad)))
        return dh, d_norm_w

    def route_from_logits(self, logits, saved=None):
        T = logits.shape[0]
        if saved is None:
            saved = self.new_saved(T)
        ws = self.workspace(T)
        _lib.check(_lib.load().moe_route_from_logits(self.h, self._stream(), T, _p(logits),
                                                     _p(saved), _p(ws)))
        return saved

    def set_profiling(self, stages=None):
        """Time the named stages (all when None, none when []) with HIP events."""
        L = _lib.load()
        if stages is None:
            mask = -1
        else:
            names = [L.moe_stage_name(i).decode() for i in range(_lib.NUM_STAGES)]
            mask = 0
            for s in stages:
                mask |= 1 << names.index(s)
        _lib.check(L.moe_plan_set_profiling(self.h, mask))

    def set_shared_overlap(self, on=True):
        """Side streams of the plan: True / 1 (default) runs the shared expert
        and the routed weight gradients on streams of their own; 2 the shared
        expert only; False / 0 everything in serial order on the call's
        stream."""
        _lib.check(_lib.load().moe_plan_set_shared_overlap(self.h, int(on)))

    def stage_times(self, reset=True):
        ms = (ctypes.c_float * _lib.NUM_STAGES)()
        calls = (ctypes.c_int32 * _lib.NUM_STAGES)()
        _lib.check(_lib.load().moe_plan_stage_times(self.h, ms, calls, int(reset)))
        L = _lib.load()
        return {L.moe_stage_name(i).decode(): (ms[i], calls[i]) for i in range(_lib.NUM_STAGES)}


class _RoutedExperts:
    """Which experts received a token in a forward, copied to pinned host
    memory right after the forward's dispatch (non-blocking). An expert with no
    token gets no gradient entry (src/trainer.rs:556-566); by the time the
    backward asks, the copy has long completed, so reading it does not stall
    the launch pipeline the way a device-to-host copy in the backward would."""

    def __init__(self, counts, num_experts):
        self.num_experts = num_experts
        if counts is None:  # no token: no expert is routed
            self.host, self.event = None, None
            return
        self.host = torch.empty(counts.shape, dtype=counts.dtype, pin_memory=True)
        self.host.copy_(counts, non_blocking=True)
        self.event = torch.cuda.Event()
        self.event.record()

    def get(self):
        if self.host is None:
            return [False] * self.num_experts
        self.event.synchronize()
        return [c > 0 for c in self.host.tolist()]


def _routed_experts_async(plan, saved, T):
    E = plan.c.num_experts
    return _RoutedExperts(plan.saved_field(saved, T, "counts") if T > 0 else None, E)


class _MoeFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, layer, x2d, router, router_bias, *params):
        E = layer.num_experts
        gate, up, down = params[0:E], params[E:2 * E], params[2 * E:3 * E]
        shared = params[3 * E:3 * E + 3] if layer.shared_expert is not None else None
        plan = layer.plan(x2d)
        w, keep = plan.weights_struct(router, gate, up, down, router_bias, shared)
        out, aux, z, saved = plan.forward(x2d, w)
        ctx.layer = layer
        ctx.plan = plan
        ctx.saved = saved
        ctx.routed = _routed_experts_async(plan, saved, x2d.shape[0])
        ctx.save_for_backward(x2d, router, router_bias if router_bias is not None else x2d.new_empty(0),
                              *params)
        ctx.has_bias = router_bias is not None
        return out, aux, z

    @staticmethod
    def backward(ctx, dout, daux, dz):
        layer, plan = ctx.layer, ctx.plan
        x2d, router, router_bias, *params = ctx.saved_tensors
        if not ctx.has_bias:
            router_bias = None
        E = layer.num_experts
        gate, up, down = params[0:E], params[E:2 * E], params[2 * E:3 * E]
        shared = params[3 * E:3 * E + 3] if layer.shared_expert is not None else None
        w, keep_w = plan.weights_struct(router, gate, up, down, router_bias, shared)
        g_router = torch.empty_like(router)
        g_bias = torch.empty_like(router_bias) if router_bias is not None else None
        g_gate = [torch.empty_like(t) for t in gate]
        g_up = [torch.empty_like(t) for t in up]
        g_down = [torch.empty_like(t) for t in down]
        g_shared = [torch.empty_like(t) for t in shared] if shared is not None else None
        g, keep_g = plan.grads_struct(g_router, g_gate, g_up, g_down, g_bias, g_shared)
        dout = dout.contiguous() if dout is not None else torch.zeros_like(x2d)
        daux = (daux if daux is not None else torch.zeros((), device=x2d.device)).float().contiguous()
        dz = (dz if dz is not None else torch.zeros((), device=x2d.device)).float().contiguous()
        dx = plan.backward(x2d, dout, w, g, ctx.saved, d_aux=daux, d_z=dz)
        hg = ctx.routed.get()  # experts that get a gradient entry, known since the forward
        ctx.saved = None
        def keep(lst):
            return [t if hg[e] else None for e, t in enumerate(lst)]
        grads = keep(g_gate) + keep(g_up) + keep(g_down)
        if g_shared is not None:
            grads += g_shared
        return (None, dx, g_router, g_bias, *grads)


class Expert(torch.nn.Module):
    """SwiGLU expert down(silu(gate x) * up x) (src/model.rs:1284-1290)."""

    def __init__(self, hidden, intermediate, dtype, device):
        super().__init__()
        kw = dict(dtype=dtype, device=device)
        self.gate_proj = torch.nn.Linear(hidden, intermediate, bias=False, **kw)
        self.up_proj = torch.nn.Linear(hidden, intermediate, bias=False, **kw)
        self.down_proj = torch.nn.Linear(intermediate, hidden, bias=False, **kw)


class Router(torch.nn.Module):
    def __init__(self, hidden, num_experts, bias, dtype, device):
        super().__init__()
        self.gate = torch.nn.Linear(hidden, num_experts, bias=False, dtype=dtype, device=device)
        self.bias = (torch.nn.Parameter(torch.zeros(num_experts, dtype=torch.float32, device=device))
                     if bias else None)


class MoeLayer(torch.nn.Module):
    """Drop-in MoE layer: forward(x [B, S, H]) -> (out, aux_loss, z_loss)."""

    def __init__(self, cfg: MoeConfig, dtype=torch.bfloat16, device="cuda"):
        super().__init__()
        E, k, I = cfg.required_moe_dims()
        self.cfg = cfg
        self.num_experts = E
        self.router = Router(cfg.hidden_size, E, cfg.router_bias, dtype, device)
        self.experts = torch.nn.ModuleList(
            [Expert(cfg.hidden_size, I, dtype, device) for _ in range(E)])
        S = cfg.shared_width()
        self.shared_expert = Expert(cfg.hidden_size, S, dtype, device) if S else None
        self._dtype = dtype
        self._plans = {}

    def plan(self, x2d):
        key = (x2d.device, x2d.dtype)
        p = self._plans.get(key)
        if p is None:
            p = Plan(self.cfg, x2d.dtype, x2d.device)
            self._plans[key] = p
        return p

    def trainable_parameters(self):
        """(name, parameter) in the reference order: router gate, experts 0..E-1
        (gate, up, down), then the shared expert (src/model.rs:1887-1897)."""
        out = [("router.gate.weight", self.router.gate.weight)]
        if self.router.bias is not None:
            out.append(("router.gate.bias", self.router.bias))
        for i, e in enumerate(self.experts):
            for n in ("gate_proj", "up_proj", "down_proj"):
                out.append((f"experts.{i}.{n}.weight", getattr(e, n).weight))
        if self.shared_expert is not None:
            for n in ("gate_proj", "up_proj", "down_proj"):
                out.append((f"shared_expert.{n}.weight", getattr(self.shared_expert, n).weight))
        return out

    def forward(self, x):
        if x.dim() != 3:
            raise ModelError(f"MoE expects [B, Seq, Hidden], got {list(x.shape)}")
        B, S, H = x.shape
        x2d = x.reshape(B * S, H).contiguous()
        params = ([e.gate_proj.weight for e in self.experts] +
                  [e.up_proj.weight for e in self.experts] +
                  [e.down_proj.weight for e in self.experts])
        if self.shared_expert is not None:
            params += [self.shared_expert.gate_proj.weight, self.shared_expert.up_proj.weight,
                       self.shared_expert.down_proj.weight]
        tracked = [x2d, self.router.gate.weight] + params
        if self.router.bias is not None:
            tracked.append(self.router.bias)
        if not (torch.is_grad_enabled() and any(t.requires_grad for t in tracked)):
            # no backward can follow: forward-only call, no saved state
            plan = self.plan(x2d)
            shared = params[3 * self.num_experts:] if self.shared_expert is not None else None
            E = self.num_experts
            w, keep = plan.weights_struct(self.router.gate.weight, params[0:E], params[E:2 * E],
                                          params[2 * E:3 * E], self.router.bias, shared)
            out, aux, z, _ = plan.forward(x2d, w, need_grad=False)
            return out.reshape(B, S, H), aux, z
        out, aux, z = _MoeFunction.apply(self, x2d, self.router.gate.weight, self.router.bias,
                                         *params)
        return out.reshape(B, S, H), aux, z


class _MoeBlockFunction(torch.autograd.Function):
    """Autograd node of the MoE sub-block (RMSNorm -> MoE -> residual add)."""

    @staticmethod
    def forward(ctx, block, h2d, norm_w, router, router_bias, *params):
        layer = block.ffn
        E = layer.num_experts
        gate, up, down = params[0:E], params[E:2 * E], params[2 * E:3 * E]
        shared = params[3 * E:3 * E + 3] if layer.shared_expert is not None else None
        plan = layer.plan(h2d)
        w, keep = plan.weights_struct(router, gate, up, down, router_bias, shared)
        out, aux, z, saved = plan.block_forward(h2d, norm_w, w)
        ctx.block, ctx.plan, ctx.saved = block, plan, saved
        ctx.routed = _routed_experts_async(plan, saved, h2d.shape[0])
        ctx.has_bias = router_bias is not None
        ctx.save_for_backward(h2d, norm_w, router,
                              router_bias if router_bias is not None else h2d.new_empty(0), *params)
        return out, aux, z

    @staticmethod
    def backward(ctx, dout, daux, dz):
        layer, plan = ctx.block.ffn, ctx.plan
        h2d, norm_w, router, router_bias, *params = ctx.saved_tensors
        if not ctx.has_bias:
            router_bias = None
        E = layer.num_experts
        gate, up, down = params[0:E], params[E:2 * E], params[2 * E:3 * E]
        shared = params[3 * E:3 * E + 3] if layer.shared_expert is not None else None
        w, keep_w = plan.weights_struct(router, gate, up, down, router_bias, shared)
        g_router = torch.empty_like(router)
        g_bias = torch.empty_like(router_bias) if router_bias is not None else None
        g_gate = [torch.empty_like(t) for t in gate]
        g_up = [torch.empty_like(t) for t in up]
        g_down = [torch.empty_like(t) for t in down]
        g_shared = [torch.empty_like(t) for t in shared] if shared is not None else None
        g, keep_g = plan.grads_struct(g_router, g_gate, g_up, g_down, g_bias, g_shared)
        dout = dout.contiguous() if dout is not None else torch.zeros_like(h2d)
        daux = (daux if daux is not None else torch.zeros((), device=h2d.device)).float().contiguous()
        dz = (dz if dz is not None else torch.zeros((), device=h2d.device)).float().contiguous()
        dh, d_norm_w = plan.block_backward(h2d, norm_w, dout, w, g, ctx.saved, d_aux=daux, d_z=dz)
        hg = ctx.routed.get()
        ctx.saved = None

        def keep(lst):
            return [t if hg[e] else None for e, t in enumerate(lst)]
        grads = keep(g_gate) + keep(g_up) + keep(g_down)
        if g_shared is not None:
            grads += g_shared
        return (None, dh, d_norm_w, g_router, g_bias, *grads)


class MoeBlock(torch.nn.Module):
    """The MoE sub-block of a decoder block (src/model.rs:2792-2800):
    forward(h [B, S, H]) -> (MoE(post_attention_layernorm(h)) + h, aux, z),
    run as one fused_block plan."""

    def __init__(self, cfg: MoeConfig, dtype=torch.bfloat16, device="cuda"):
        super().__init__()
        cfg = dataclasses.replace(cfg, fused_block=True)
        self.post_attention_layernorm = torch.nn.Module()
        self.post_attention_layernorm.weight = torch.nn.Parameter(
            torch.ones(cfg.hidden_size, dtype=dtype, device=device))
        self.ffn = MoeLayer(cfg, dtype=dtype, device=device)

    def trainable_parameters(self):
        return ([("post_attention_layernorm.weight", self.post_attention_layernorm.weight)] +
                self.ffn.trainable_parameters())

    def forward(self, h):
        if h.dim() != 3:
            raise ModelError(f"MoE expects [B, Seq, Hidden], got {list(h.shape)}")
        B, S, H = h.shape
        h2d = h.reshape(B * S, H).contiguous()
        layer = self.ffn
        params = ([e.gate_proj.weight for e in layer.experts] +
                  [e.up_proj.weight for e in layer.experts] +
                  [e.down_proj.weight for e in layer.experts])
        if layer.shared_expert is not None:
            params += [layer.shared_expert.gate_proj.weight, layer.shared_expert.up_proj.weight,
                       layer.shared_expert.down_proj.weight]
        norm_w = self.post_attention_layernorm.weight
        tracked = [h2d, norm_w, layer.router.gate.weight] + params
        if layer.router.bias is not None:
            tracked.append(layer.router.bias)
        if not (torch.is_grad_enabled() and any(t.requires_grad for t in tracked)):
            plan = layer.plan(h2d)
            E = layer.num_experts
            shared = params[3 * E:] if layer.shared_expert is not None else None
            w, keep = plan.weights_struct(layer.router.gate.weight, params[0:E], params[E:2 * E],
                                          params[2 * E:3 * E], layer.router.bias, shared)
            out, aux, z, _ = plan.block_forward(h2d, norm_w, w, need_grad=False)
            return out.reshape(B, S, H), aux, z
        out, aux, z = _MoeBlockFunction.apply(self, h2d, norm_w, layer.router.gate.weight,
                                              layer.router.bias, *params)
        return out.reshape(B, S, H), aux, z
