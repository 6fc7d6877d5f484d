"""Shared helpers of the GPU parity tests: seeded inputs, one GPU forward +
backward through the C ABI, and the same pass on the CPU oracle."""
import dataclasses

import numpy as np
import torch

from oracle import moe_oracle as mo
from oxidizr_amd.moe import MoeConfig, Plan
from oxidizr_amd.synth import host_problem


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    nb = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (nb if nb > 0 else 1.0))


class Case:
    def __init__(self, T, H, E, k, I, S=0, dtype="f32", w_std=0.1, seed=0, bias=None,
                 norm_topk=False, tau=1.0, shared_scale=1.0, aux_switch=1.0, aux_sqprob=1.0,
                 recompute=False):
        self.T, self.H, self.E, self.k, self.I, self.S = T, H, E, k, I, S
        self.dtype = dtype
        self.tdtype = torch.float32 if dtype == "f32" else torch.bfloat16
        self.bias = bias
        self.p = host_problem(T, H, E, k, I, S, w_std=w_std, seed=seed, bias=bias, dtype=dtype)
        self.cfg = MoeConfig(hidden_size=H, num_experts=E, experts_per_tok=k, intermediate_size=I,
                             shared_expert_enabled=S > 0, shared_intermediate_size=S or None,
                             router_temperature=tau, norm_topk_prob=norm_topk,
                             aux_switch_coef=aux_switch, aux_sqprob_coef=aux_sqprob,
                             shared_expert_scale=shared_scale, router_bias=bias is not None,
                             recompute_activations=recompute)
        self.ocfg = mo.make_cfg(T, H, E, k, I, S, norm_topk=norm_topk, has_bias=bias is not None,
                                tau=tau, shared_scale=shared_scale, aux_switch=aux_switch,
                                aux_sqprob=aux_sqprob)

    def __repr__(self):
        return f"Case(T={self.T},H={self.H},E={self.E},k={self.k},I={self.I},S={self.S},{self.dtype})"


def gpu_run(case, d_aux=0.0, d_z=0.0, backward=True, nan_fill=True, dout=None, x=None,
            overlap=True, need_grad=True, backwards=1):
    """Forward (+ backward) on cuda:0. Returns a dict of numpy results.
    need_grad=False: forward-only call without saved state (out, aux, z only).
    backwards > 1: that many backward calls on the same plan and buffers, the
    device synchronised between them (the results of the last one)."""
    dev = torch.device("cuda:0")
    p = case.p
    dt = case.tdtype
    t = {n: torch.tensor(v, device=dev).to(dt) for n, v in p.items() if n != "router_bias"}
    if x is not None:
        t["x"] = torch.tensor(x, device=dev).to(dt)
    if dout is not None:
        t["dout"] = torch.tensor(dout, device=dev).to(dt)
    bias = torch.tensor(p["router_bias"], device=dev) if case.bias is not None else None
    T = t["x"].shape[0]
    plan = Plan(case.cfg, dt, dev)
    plan.set_shared_overlap(overlap)
    gate, up, down = (list(t[n].unbind(0)) for n in ("gate", "up", "down"))
    shared = (t["shared_gate"], t["shared_up"], t["shared_down"]) if case.S else None
    w, _keep = plan.weights_struct(t["router"], gate, up, down, bias, shared)
    out, aux, z, saved = plan.forward(t["x"], w, need_grad=need_grad)
    res = {"out": out, "aux": aux, "z": z}
    if need_grad:
        for f in ("logits", "probs", "lse", "topk_idx", "topk_w", "counts", "offsets", "perm",
                  "inv_perm"):
            res[f] = plan.saved_field(saved, T, f)
    if backward and need_grad:
        fill = float("nan") if nan_fill else 0.0
        g_router = torch.empty_like(t["router"])
        g_bias = torch.empty_like(bias) if bias is not None else None
        g_gate = [torch.full_like(a, fill) for a in gate]
        g_up = [torch.full_like(a, fill) for a in up]
        g_down = [torch.full_like(a, fill) for a in down]
        g_sh = [torch.empty_like(a) for a in shared] if shared else None
        g, _keep2 = plan.grads_struct(g_router, g_gate, g_up, g_down, g_bias, g_sh)
        has_grad = torch.full((case.E,), 7, dtype=torch.uint8, device=dev)
        da = torch.tensor(float(d_aux), device=dev)
        dz = torch.tensor(float(d_z), device=dev)
        for i in range(backwards):
            if i:
                torch.cuda.synchronize()
            dx = plan.backward(t["x"], t["dout"], w, g, saved, d_aux=da, d_z=dz,
                               has_grad=has_grad)
        res.update({"dx": dx, "router": g_router, "router_bias": g_bias,
                    "gate": torch.stack(g_gate), "up": torch.stack(g_up),
                    "down": torch.stack(g_down), "has_grad": has_grad})
        if g_sh:
            res.update({"shared_gate": g_sh[0], "shared_up": g_sh[1], "shared_down": g_sh[2]})
    torch.cuda.synchronize()
    outn = {}
    for n, v in res.items():
        if v is None:
            outn[n] = None
        elif v.dtype == torch.bfloat16:
            outn[n] = v.float().cpu().numpy()
        else:
            outn[n] = v.cpu().numpy()
    return outn


def oracle_run(case, logits, d_aux=0.0, d_z=0.0, backward=True, dout=None, x=None):
    """The CPU oracle (float64) on the same inputs, routed from the given logits."""
    p = dict(case.p)
    if x is not None:
        p["x"] = x
    if dout is not None:
        p["dout"] = dout
    o = mo.MoeOracle(case.ocfg, 64)
    out, aux, z = o.forward(p["x"], p["router"], p["gate"], p["up"], p["down"],
                            p.get("router_bias"), p.get("shared_gate"), p.get("shared_up"),
                            p.get("shared_down"), logits_in=logits)
    res = {"out": out, "aux": aux, "z": z, "oracle": o}
    for f in ("logits", "probs", "lse", "topk_idx", "topk_w", "counts", "offsets", "perm",
              "inv_perm"):
        res[f] = o.get(f)
    if backward:
        res.update(o.backward(p["dout"], d_aux=d_aux, d_z=d_z))
    return res


def rounded(a, tdtype):
    """a as the device dtype sees it (float64 numpy)."""
    return torch.tensor(np.asarray(a, np.float64)).to(tdtype).double().numpy()


def gpu_block_run(case, h, norm_w, eps, d_aux=0.0, d_z=0.0, recompute=False):
    """moe_block_forward + moe_block_backward on cuda:0 (fused_block plan)."""
    dev = torch.device("cuda:0")
    p = case.p
    dt = case.tdtype
    t = {n: torch.tensor(v, device=dev).to(dt) for n, v in p.items() if n != "router_bias"}
    ht = torch.tensor(h, device=dev).to(dt)
    nw = torch.tensor(norm_w, device=dev).to(dt)
    bias = torch.tensor(p["router_bias"], device=dev) if case.bias is not None else None
    T = ht.shape[0]
    cfg = dataclasses.replace(case.cfg, fused_block=True, rms_norm_eps=eps,
                              recompute_activations=recompute)
    plan = Plan(cfg, dt, dev)
    gate, up, down = (list(t[n].unbind(0)) for n in ("gate", "up", "down"))
    shared = (t["shared_gate"], t["shared_up"], t["shared_down"]) if case.S else None
    w, _keep = plan.weights_struct(t["router"], gate, up, down, bias, shared)
    out, aux, z, saved = plan.block_forward(ht, nw, w)
    res = {"out": out, "aux": aux, "z": z, "logits": plan.saved_field(saved, T, "logits")}
    g_router = torch.empty_like(t["router"])
    g_gate = [torch.full_like(a, float("nan")) for a in gate]
    g_up = [torch.full_like(a, float("nan")) for a in up]
    g_down = [torch.full_like(a, float("nan")) for a in down]
    g_sh = [torch.empty_like(a) for a in shared] if shared else None
    g, _keep2 = plan.grads_struct(g_router, g_gate, g_up, g_down, None, g_sh)
    has_grad = torch.full((case.E,), 7, dtype=torch.uint8, device=dev)
    da = torch.tensor(float(d_aux), device=dev)
    dz = torch.tensor(float(d_z), device=dev)
    dh, dnw = plan.block_backward(ht, nw, t["dout"], w, g, saved, d_aux=da, d_z=dz,
                                  has_grad=has_grad)
    res.update({"dh": dh, "norm_weight": dnw, "router": g_router, "gate": torch.stack(g_gate),
                "up": torch.stack(g_up), "down": torch.stack(g_down), "has_grad": has_grad})
    if g_sh:
        res.update({"shared_gate": g_sh[0], "shared_up": g_sh[1], "shared_down": g_sh[2]})
    torch.cuda.synchronize()
    return {n: (v.float().cpu().numpy() if isinstance(v, torch.Tensor) else v)
            for n, v in res.items()}
