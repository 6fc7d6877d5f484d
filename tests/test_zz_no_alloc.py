"""moe_forward_noalloc: the forward-only entry point that allocates nothing
(its scratch is the library's static device array), through the C ABI.

Its results must be the bits of moe_forward with saved == NULL (the existing
forward-only entry point, on a workspace of its own) for the same inputs, on
two calls in a row on one plan, the second with a smaller input (the static
scratch keeps the first call's contents). A token count whose forward needs
more scratch than the static array holds is refused on the host.
"""
import numpy as np
import pytest
import torch

from oxidizr_amd import _lib
from oxidizr_amd.moe import MoeConfig, Plan
from tests.gpu_helpers import Case

pytestmark = pytest.mark.gpu


def _tensors(case, dev):
    return {n: torch.tensor(v, device=dev).to(case.tdtype) for n, v in case.p.items()
            if n != "router_bias"}


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_forward_noalloc_matches_forward(dtype):
    dev = torch.device("cuda:0")
    case = Case(T=300, H=128, E=16, k=2, I=64, S=64, dtype=dtype, w_std=0.05, seed=51)
    t = _tensors(case, dev)
    plan = Plan(case.cfg, case.tdtype, dev)
    gate, up, down = (list(t[n].unbind(0)) for n in ("gate", "up", "down"))
    shared = (t["shared_gate"], t["shared_up"], t["shared_down"])
    w, _keep = plan.weights_struct(t["router"], gate, up, down, None, shared)
    # 300 tokens (tiled kernels, fused router in bf16), then 40 (small-token
    # kernels in bf16): the second call is smaller than the first
    for T in (300, 40):
        x = t["x"][:T].contiguous()
        ref_out, ref_aux, ref_z, _ = plan.forward(x, w, need_grad=False)
        out = torch.full_like(x, float("nan"))
        aux = torch.full((), float("nan"), device=dev)
        z = torch.full((), float("nan"), device=dev)
        plan.forward_noalloc(x, w, out, aux, z)
        torch.cuda.synchronize()
        assert torch.equal(out, ref_out), T
        assert torch.equal(aux, ref_aux) and torch.equal(z, ref_z), T
        assert bool(torch.isfinite(out).all()), T


def test_forward_noalloc_refuses_oversized_batches():
    dev = torch.device("cuda:0")
    cfg = MoeConfig(hidden_size=4096, num_experts=128, experts_per_tok=8, intermediate_size=1536,
                    shared_expert_enabled=False)
    plan = Plan(cfg, torch.bfloat16, dev)
    aux = torch.empty((), device=dev)
    z = torch.empty((), device=dev)
    w = _lib.MoeWeightsC()  # never read: the size check comes first
    big = 4096
    assert plan.c.hidden * plan.c.experts_per_tok * 2 * big > 64 << 20
    xb = torch.zeros(big, 4096, dtype=torch.bfloat16, device=dev)
    with pytest.raises(_lib.MoeError, match="static scratch") as e:
        plan.forward_noalloc(xb, w, torch.empty_like(xb), aux, z)
    assert e.value.status == 4


def test_forward_noalloc_under_graph_capture():
    """A captured moe_forward_noalloc replays the eager call's bits, every
    replay, with eager calls of the plan between the replays; a capture whose
    pointer tables differ from the plan's last call is refused on the host
    (the table upload cannot be recorded safely) and leaves the plan usable."""
    dev = torch.device("cuda:0")
    case = Case(T=300, H=128, E=16, k=2, I=64, S=64, dtype="bf16", w_std=0.05, seed=53)
    t = _tensors(case, dev)
    plan = Plan(case.cfg, case.tdtype, dev)
    gate, up, down = (list(t[n].unbind(0)) for n in ("gate", "up", "down"))
    shared = (t["shared_gate"], t["shared_up"], t["shared_down"])
    w, _keep = plan.weights_struct(t["router"], gate, up, down, None, shared)
    x = t["x"].contiguous()
    x_other = torch.flip(x, dims=[0]).contiguous()
    ref_out, ref_aux, ref_z, _ = plan.forward(x, w, need_grad=False)
    oth_out, _, _, _ = plan.forward(x_other, w, need_grad=False)
    out, aux, z = torch.empty_like(x), torch.empty((), device=dev), torch.empty((), device=dev)
    plan.forward_noalloc(x, w, out, aux, z)  # eager call first: the tables are on the device
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        plan.forward_noalloc(x, w, out, aux, z)
    torch.cuda.synchronize()
    eo = torch.empty_like(x)
    for replay in range(3):
        out.fill_(float("nan"))
        aux.fill_(float("nan"))
        z.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        print(f"replay {replay}", flush=True)
        assert torch.equal(out, ref_out), replay
        assert torch.equal(aux, ref_aux) and torch.equal(z, ref_z), replay
        # eager work of the plan between replays (same tables, other tokens)
        plan.forward_noalloc(x_other, w, eo, torch.empty((), device=dev),
                             torch.empty((), device=dev))
        torch.cuda.synchronize()
        assert torch.equal(eo, oth_out), replay
    # new weight tensors (same values) give new pointer tables: refused while capturing
    gate2, up2, down2 = ([p.clone() for p in ps] for ps in (gate, up, down))
    w2, _keep2 = plan.weights_struct(t["router"], gate2, up2, down2, None, shared)
    out2 = torch.zeros_like(x)
    graph2 = torch.cuda.CUDAGraph()
    with pytest.raises(_lib.MoeError, match="capturing") as e:
        with torch.cuda.graph(graph2):
            out2.fill_(1.0)  # keeps the refused capture non-empty
            plan.forward_noalloc(x, w2, out2, aux, z)
    assert e.value.status == 4
    torch.cuda.synchronize()
    del graph2
    # the plan still holds the first tables, and takes the new ones eagerly
    o1 = torch.empty_like(x)
    plan.forward_noalloc(x, w, o1, aux, z)
    o2 = torch.empty_like(x)
    plan.forward_noalloc(x, w2, o2, aux, z)
    torch.cuda.synchronize()
    assert torch.equal(o1, ref_out) and torch.equal(o2, ref_out)
