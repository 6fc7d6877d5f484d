"""Packed-expert storage of one MoE layer and its safetensors loader / saver.

On disk an oxidizr checkpoint keeps every expert projection as its own tensor
under the reference's parameter names (src/model.rs:4867-4912):

    layers.{L}.moe.router.gate.weight                      [E, H]
    layers.{L}.moe.experts.{e}.{gate,up}_proj.weight       [I, H]
    layers.{L}.moe.experts.{e}.down_proj.weight            [H, I]
    layers.{L}.moe.shared_expert.{gate,up,down}_proj.weight

written with the decoder prefix "model." (src/checkpoint_names.rs:13-37).
`PackedExperts` holds the same weights as one contiguous device tensor per
projection kind ([E, I, H] gate and up, [E, H, I] down): expert e is the view
`gate[e]`, whose address the plan's pointer table takes as is, so the grouped
GEMMs read the packed tensor in place (no per-expert allocation, no copy per
call) while the on-disk names stay unchanged.
"""
from dataclasses import dataclass
from typing import Dict, List, Optional, Sequence

import torch

CHECKPOINT_DECODER_PREFIX = "model."


def to_checkpoint_name(param_name: str) -> str:
    """src/checkpoint_names.rs:22-28: every name but lm_head.* gets "model."."""
    if param_name.startswith("lm_head."):
        return param_name
    return CHECKPOINT_DECODER_PREFIX + param_name


def from_checkpoint_name(name: str) -> str:
    """src/checkpoint_names.rs:34-36: strips a leading "model." when present."""
    return name[len(CHECKPOINT_DECODER_PREFIX):] if name.startswith(CHECKPOINT_DECODER_PREFIX) else name


def moe_layer_names(layer: int, num_experts: int, shared: bool) -> List[str]:
    """Parameter names of one MoE layer in the reference's order: router, then
    experts 0..E-1 (gate, up, down), then the shared expert
    (src/model.rs:4889-4912)."""
    p = f"layers.{layer}.moe"
    names = [f"{p}.router.gate.weight"]
    for e in range(num_experts):
        names += [f"{p}.experts.{e}.{n}.weight" for n in ("gate_proj", "up_proj", "down_proj")]
    if shared:
        names += [f"{p}.shared_expert.{n}.weight" for n in ("gate_proj", "up_proj", "down_proj")]
    return names


class CheckpointError(ValueError):
    pass


def _check_shape(name, t, shape):
    # message of src/model.rs:516-525 (ensure_shape)
    if tuple(t.shape) != tuple(shape):
        raise CheckpointError(f"shape mismatch for '{name}': expected {list(shape)}, "
                              f"got {list(t.shape)}")


@dataclass
class PackedExperts:
    router: torch.Tensor                  # [E, H]
    gate: torch.Tensor                    # [E, I, H]
    up: torch.Tensor                      # [E, I, H]
    down: torch.Tensor                    # [E, H, I]
    shared: Optional[Sequence[torch.Tensor]] = None   # ([S, H], [S, H], [H, S])

    @classmethod
    def empty(cls, hidden, num_experts, intermediate, shared_intermediate=0,
              dtype=torch.bfloat16, device="cuda"):
        H, E, I, S = hidden, num_experts, intermediate, shared_intermediate
        kw = dict(dtype=dtype, device=device)
        sh = ((torch.empty(S, H, **kw), torch.empty(S, H, **kw), torch.empty(H, S, **kw))
              if S else None)
        return cls(torch.empty(E, H, **kw), torch.empty(E, I, H, **kw), torch.empty(E, I, H, **kw),
                   torch.empty(E, H, I, **kw), sh)

    def experts(self):
        """(gate, up, down) lists of per-expert views into the packed tensors."""
        return list(self.gate.unbind(0)), list(self.up.unbind(0)), list(self.down.unbind(0))

    def weights_struct(self, plan, router_bias=None):
        """moe_weights of `plan` pointing into the packed storage."""
        g, u, d = self.experts()
        return plan.weights_struct(self.router, g, u, d, router_bias, self.shared)

    def grads_struct(self, plan, router_bias=None):
        """moe_grads of `plan` pointing into `self` used as gradient storage."""
        g, u, d = self.experts()
        return plan.grads_struct(self.router, g, u, d, router_bias, self.shared)

    def named_tensors(self, layer: int) -> Dict[str, torch.Tensor]:
        """{parameter name: view} in the reference's order."""
        E = self.gate.shape[0]
        names = moe_layer_names(layer, E, self.shared is not None)
        views = [self.router]
        for e in range(E):
            views += [self.gate[e], self.up[e], self.down[e]]
        if self.shared is not None:
            views += list(self.shared)
        return dict(zip(names, views))


def load_packed(files, layer: int, hidden: int, num_experts: int, intermediate: int,
                shared_intermediate: int = 0, dtype=None, device="cuda") -> PackedExperts:
    """Reads one MoE layer from safetensors file(s) written under the
    checkpoint names and packs it on `device` (dtype: the file's unless given).
    Each tensor is copied straight into its slice of the packed storage."""
    from safetensors import safe_open

    if isinstance(files, str):
        files = [files]
    handles = [safe_open(f, framework="pt", device="cpu") for f in files]
    where = {}
    for h in handles:
        for k in h.keys():
            where[k] = h
    want = moe_layer_names(layer, num_experts, shared_intermediate > 0)
    missing = [n for n in want if to_checkpoint_name(n) not in where]
    if missing:
        raise CheckpointError(f"checkpoint has no tensor '{to_checkpoint_name(missing[0])}'"
                              f" ({len(missing)} MoE tensors of layer {layer} missing)")
    first = where[to_checkpoint_name(want[0])].get_tensor(to_checkpoint_name(want[0]))
    dt = dtype if dtype is not None else first.dtype
    pk = PackedExperts.empty(hidden, num_experts, intermediate, shared_intermediate, dt, device)
    H, I, S = hidden, intermediate, shared_intermediate
    shapes = {"router.gate": (num_experts, H), "gate_proj": (I, H), "up_proj": (I, H),
              "down_proj": (H, I)}
    for name, view in pk.named_tensors(layer).items():
        key = to_checkpoint_name(name)
        t = where[key].get_tensor(key)
        if ".shared_expert." in name:
            shape = {"gate_proj": (S, H), "up_proj": (S, H), "down_proj": (H, S)}[name.split(".")[-2]]
        elif name.endswith("router.gate.weight"):
            shape = shapes["router.gate"]
        else:
            shape = shapes[name.split(".")[-2]]
        _check_shape(key, t, shape)
        view.copy_(t.to(dt))
    return pk


def save_packed(path: str, layer: int, packed: PackedExperts, metadata=None):
    """Writes one MoE layer under the checkpoint names (one tensor per expert
    projection, as the reference stores them)."""
    from safetensors.torch import save_file

    tensors = {to_checkpoint_name(n): v.detach().cpu().contiguous()
               for n, v in packed.named_tensors(layer).items()}
    save_file(tensors, path, metadata=metadata)
