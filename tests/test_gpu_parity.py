"""GPU parity of the HIP MoE layer against the CPU oracle, through the C ABI.

Bars:
  * routing: on identical fp32 logits, top-k indices, expert counts, offsets
    and the dispatch permutation match the oracle bit-exactly;
  * fp32: outputs and gradients within 1e-5 relative (L2) error;
  * bf16: outputs and gradients within 1e-2 relative L2 error.
The oracle routes from the GPU's own logits (logits_in), so both sides take
the same routing decisions; the GPU logits themselves are compared with
tolerance.
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import moe_oracle as mo
from oxidizr_amd import _lib
from oxidizr_amd.moe import MoeConfig, MoeLayer, Plan
from oxidizr_amd.synth import zipf_bias
from tests.gpu_helpers import Case, gpu_block_run, gpu_run, oracle_run, rel, rounded

pytestmark = pytest.mark.gpu

GRAD_NAMES = ("dx", "router", "gate", "up", "down")


def _routing_equal(g, o):
    np.testing.assert_array_equal(g["topk_idx"], o["topk_idx"])
    np.testing.assert_array_equal(g["counts"], o["counts"])
    np.testing.assert_array_equal(g["offsets"], o["offsets"])
    np.testing.assert_array_equal(g["perm"], o["perm"])
    np.testing.assert_array_equal(g["inv_perm"], o["inv_perm"])


def _check(case, g, o, tol, backward=True):
    errs = {"out": rel(g["out"], o["out"]),
            "logits": rel(g["logits"], case_logits_ref(case)),
            "probs": rel(g["probs"], o["probs"]),
            "topk_w": rel(g["topk_w"], o["topk_w"])}
    errs["aux"] = abs(float(g["aux"]) - o["aux"]) / max(abs(o["aux"]), 1e-30)
    errs["z"] = abs(float(g["z"]) - o["z"]) / max(abs(o["z"]), 1e-30)
    if backward:
        np.testing.assert_array_equal(g["has_grad"], o["has_grad"])
        hg = o["has_grad"].astype(bool)
        errs["dx"] = rel(g["dx"], o["x"])
        errs["d_router"] = rel(g["router"], o["router"])
        if case.bias is not None:
            errs["d_router_bias"] = rel(g["router_bias"], o["router_bias"])
        for n in ("gate", "up", "down"):
            errs["d_" + n] = rel(g[n][hg], o[n][hg])
            # experts with no routed token have no gradient entry: untouched buffers
            assert np.isnan(g[n][~hg]).all(), n
        if case.S:
            for n in ("shared_gate", "shared_up", "shared_down"):
                errs["d_" + n] = rel(g[n], o[n])
    bad = {n: e for n, e in errs.items() if not e <= tol}
    assert not bad, f"{case}: over tolerance {tol}: {bad} (all: {errs})"
    return errs


def case_logits_ref(case):
    p = case.p
    lg = p["x"].astype(np.float64) @ p["router"].astype(np.float64).T
    if case.bias is not None:
        lg = lg + p["router_bias"]
    return lg


# ---------------------------------------------------------------- routing

@pytest.mark.parametrize("T,E,k", [(1, 4, 2), (257, 8, 2), (1000, 16, 2), (777, 64, 6),
                                   (64, 128, 8), (300, 256, 8), (40, 5, 5), (129, 1000, 16)])
def test_routing_bitexact_on_identical_logits(T, E, k):
    rng = np.random.default_rng(T * 7 + E)
    # small integers: many exact ties, which must go to the lower expert index
    logits = rng.integers(-3, 4, size=(T, E)).astype(np.float32)
    cfg = MoeConfig(hidden_size=8, num_experts=E, experts_per_tok=k, intermediate_size=8,
                    shared_expert_enabled=False)
    dev = torch.device("cuda:0")
    plan = Plan(cfg, torch.bfloat16, dev)
    saved = plan.route_from_logits(torch.tensor(logits, device=dev))
    torch.cuda.synchronize()
    oc = mo.make_cfg(T, 8, E, k, 8)
    probs, lse, idx, w = mo.route(oc, logits.astype(np.float64))
    counts, offsets, perm, inv = mo.dispatch(idx, E)
    f = lambda n: plan.saved_field(saved, T, n).cpu().numpy()
    np.testing.assert_array_equal(f("topk_idx"), idx)
    np.testing.assert_array_equal(f("counts"), counts)
    np.testing.assert_array_equal(f("offsets"), offsets)
    np.testing.assert_array_equal(f("perm"), perm)
    np.testing.assert_array_equal(f("inv_perm"), inv)
    assert rel(f("probs"), probs) < 1e-6
    assert rel(f("lse"), lse) < 1e-6
    assert rel(f("topk_w"), w) < 1e-6


# ---------------------------------------------------------------- fp32

FP32_CASES = [
    dict(T=96, H=64, E=8, k=2, I=48, S=32),
    dict(T=100, H=72, E=5, k=3, I=40, S=24, bias=True, norm_topk=True, tau=1.5,
         shared_scale=0.5, aux_switch=0.3, aux_sqprob=2.0),
    dict(T=1024, H=384, E=8, k=2, I=1024, S=0),     # BASELINE config 1 (fp32, CPU-runnable)
    dict(T=33, H=136, E=12, k=12, I=16, S=0),       # k == E: every expert selected
    dict(T=150, H=64, E=10, k=6, I=32, S=16),       # 4 < k <= 8 (dx gathers sized for k <= 8)
    dict(T=130, H=3592, E=6, k=2, I=32, S=0, bias=True),  # fused router over 57 k-chunks
    dict(T=130, H=3592, E=72, k=2, I=16, S=0, bias=True),  # E > 64: router k-loop split in two chunks
    dict(T=200, H=64, E=1020, k=5, I=16, S=16),     # E not a multiple of 8, most experts empty
    dict(T=100, H=64, E=4, k=1, I=32, S=0),         # top-1 routing
]


@pytest.mark.parametrize("spec", FP32_CASES)
def test_fp32_forward_backward_parity(spec):
    spec = dict(spec)
    bias = zipf_bias(spec["E"], beta=0.5) if spec.pop("bias", False) else None
    case = Case(**spec, dtype="f32", bias=bias)
    g = gpu_run(case, d_aux=0.01, d_z=0.001)
    o = oracle_run(case, g["logits"], d_aux=0.01, d_z=0.001)
    _routing_equal(g, o)
    _check(case, g, o, 1e-5)


def test_fp32_unrouted_expert_keeps_no_gradient():
    bias = np.array([0, 0, -1e4, 0, 0, -1e4], np.float32)  # experts 2 and 5 never chosen
    case = Case(T=80, H=64, E=6, k=2, I=32, S=0, dtype="f32", bias=bias)
    g = gpu_run(case, d_aux=0.1)
    o = oracle_run(case, g["logits"], d_aux=0.1)
    assert list(g["has_grad"]) == [1, 1, 0, 1, 1, 0]
    _check(case, g, o, 1e-5)


# ---------------------------------------------------------------- bf16

BF16_CASES = [
    # shapes of BASELINE configs 2, 3, 5 scaled down; skewed routing with empty experts
    dict(T=512, H=256, E=16, k=2, I=176, S=352),
    dict(T=384, H=128, E=64, k=6, I=64, S=128, skew=3.0),
    dict(T=256, H=256, E=256, k=8, I=128, S=128),
    dict(T=200, H=192, E=20, k=4, I=88, S=0, bias=True, norm_topk=True),
    # >= 512 rows per expert: the row-grouped GEMMs run half-height tail tiles
    # after every full tile (the tail order of configs 2 and 3)
    dict(T=1300, H=128, E=4, k=3, I=96, S=32, bias=True, half_last=True),
    dict(T=1280, H=136, E=4, k=2, I=200, S=0, half_last=True),
    # k above 8: dx's gathers sized for k <= 16
    dict(T=160, H=64, E=12, k=10, I=48, S=16),
    # fused router with a partial last expert block (E = 40) and router bias
    dict(T=300, H=200, E=40, k=4, I=64, S=0, bias=True),
    # tiled router (E > 64) with its k-loop split in four chunks (H >= 7168),
    # a partial last 128-row tile and a partial expert tile (E = 136)
    dict(T=200, H=7176, E=136, k=4, I=32, S=16, bias=True),
    # the largest plan limits: E = 1024 experts, k = 16
    dict(T=300, H=64, E=1024, k=16, I=16, S=0),
    # top-1 routing, fused router and tiled router
    dict(T=300, H=128, E=8, k=1, I=64, S=32),
    dict(T=260, H=128, E=72, k=1, I=64, S=0, bias=True),
    # just above the small-token paths (T = 65); the fused router over a wide
    # H whose last 128-column chunk is partial (H = 3592 = 28 * 128 + 8)
    dict(T=65, H=128, E=32, k=4, I=64, S=16),
    dict(T=100, H=3592, E=16, k=2, I=32, S=0, bias=True),
    # the fused router's scatter-gather over rows of more than 512 16-byte
    # vectors (H = 4104: a second chunk of one vector) and a ragged last group
    dict(T=90, H=4104, E=8, k=3, I=32, S=0),
    # k = 16 on the fused router: a token's earlier group entries span four
    # 64-entry ballot rounds of the scatter-gather
    dict(T=120, H=64, E=24, k=16, I=16, S=0),
]


@pytest.mark.parametrize("spec", BF16_CASES)
def test_bf16_forward_backward_parity(spec):
    spec = dict(spec)
    skew = spec.pop("skew", None)
    half_last = spec.pop("half_last", False)
    bias = None
    if skew is not None:
        bias = zipf_bias(spec["E"], s=1.2, beta=skew)
    elif spec.pop("bias", False):
        bias = zipf_bias(spec["E"], beta=0.5)
    case = Case(**spec, dtype="bf16", w_std=0.05, bias=bias)
    g = gpu_run(case, d_aux=0.01, d_z=0.001)
    o = oracle_run(case, g["logits"], d_aux=0.01, d_z=0.001)
    _routing_equal(g, o)
    if skew is not None:
        assert (g["counts"] == 0).any(), "skewed case should leave some experts empty"
    if half_last:  # the case must hold both kinds of last row tile (256-row tiles)
        counts = np.asarray(g["counts"])
        assert spec["T"] * spec["k"] >= 512 * spec["E"]
        tails = counts % 256
        assert ((tails > 0) & (tails <= 128)).any() and (tails > 128).any(), counts
    _check(case, g, o, 1e-2)


TALL_CASES = [
    # E = 2, k = 2: every expert receives all T tokens, so the counts are T.
    # 300 and 320 rows: one 256-row tile that also takes the 44 / 64-row tail
    # (tall tile); 321: the tail (65 rows) keeps its own tile.
    dict(T=300, H=128, E=2, k=2, I=96, S=0),
    dict(T=320, H=320, E=2, k=2, I=296, S=32),
    dict(T=321, H=128, E=2, k=2, I=64, S=0),
    # 350 and 384 rows (tails of 94 and 128 rows, group by group): the full
    # tile and the tail run as two 192-row tiles (192 + 158, 192 + 192)
    dict(T=350, H=136, E=2, k=2, I=88, S=16),
    dict(T=384, H=128, E=2, k=2, I=64, S=0),
    # 560 rows = 2 x 256 + 48 with >= 512 rows per expert (tails run last):
    # the second full tile is tall; I = 296 leaves a last column tile of 40
    # (the input gradient of the down projection runs it at full width)
    dict(T=560, H=136, E=2, k=2, I=296, S=0),
    # random counts around 300 rows (some merged tails, some not), router bias
    dict(T=1200, H=128, E=8, k=2, I=88, S=16, bias=True),
]


@pytest.mark.parametrize("spec", TALL_CASES)
def test_bf16_tall_tile_parity(spec):
    """Row groups whose last full 256-row tile also takes a tail of at most 64
    rows (one 320-row tile instead of a full and a quarter tile)."""
    spec = dict(spec)
    bias = zipf_bias(spec["E"], beta=0.3) if spec.pop("bias", False) else None
    case = Case(**spec, dtype="bf16", w_std=0.05, bias=bias)
    g = gpu_run(case, d_aux=0.01, d_z=0.001)
    o = oracle_run(case, g["logits"], d_aux=0.01, d_z=0.001)
    _routing_equal(g, o)
    counts = np.asarray(g["counts"])
    merged = (counts > 256) & (counts % 256 > 0) & (counts % 256 <= 64)
    if spec["T"] in (321, 350, 384):
        assert not merged.any(), counts
    else:
        assert merged.any(), counts
    _check(case, g, o, 1e-2)


ROWS384_CASES = [
    # >= 65536 routed rows and >= 768 rows per expert: the row-grouped GEMMs
    # run 384-row tiles.  E = 2, k = 2: both experts receive all T rows, so the
    # last tile of T = 86 * 384 + r rows is a 384-row tile (r = 360), a tall
    # tile (r = 300), a full tile (r = 220), a three-quarter half tile (r = 160)
    # or a quarter half tile (r = 60)
    dict(T=86 * 384 + 360, H=64, E=2, k=2, I=64, S=16),
    dict(T=86 * 384 + 300, H=72, E=2, k=2, I=72, S=0),
    dict(T=86 * 384 + 220, H=64, E=2, k=2, I=296, S=0),
    dict(T=86 * 384 + 160, H=136, E=2, k=2, I=64, S=0),
    dict(T=86 * 384 + 60, H=64, E=2, k=2, I=88, S=16),
    # random loads over 8 experts with router bias
    dict(T=33000, H=64, E=8, k=2, I=64, S=0, bias=True),
]


@pytest.mark.parametrize("spec", ROWS384_CASES)
def test_bf16_rows384_parity(spec):
    """Row-grouped GEMMs on 384-row tiles (their tails on the 256-row family)."""
    spec = dict(spec)
    bias = zipf_bias(spec["E"], beta=0.3) if spec.pop("bias", False) else None
    assert spec["T"] * spec["k"] >= 65536 and spec["T"] * spec["k"] >= 768 * spec["E"]
    case = Case(**spec, dtype="bf16", w_std=0.05, bias=bias)
    g = gpu_run(case, d_aux=0.01, d_z=0.001)
    o = oracle_run(case, g["logits"], d_aux=0.01, d_z=0.001)
    _routing_equal(g, o)
    _check(case, g, o, 1e-2)


DENSE384_CASES = [
    # The shared expert's dense GEMMs over T tokens and S = 2816 columns (11
    # tiles of 256, 22 of 128): 25-26 row tiles of 256 rows take two rounds of
    # 256 CUs (the gate/up forward three), 17 of 384 rows one (two), so the
    # gate/up forward and the down projection's input gradient run 384-row
    # tiles.  Their last row tile has 56 rows (a quarter tile) or 356 (a
    # 384-row tile with 28 padding rows).
    dict(T=6200, H=64, E=2, k=1, I=64, S=2816),
    dict(T=6500, H=72, E=4, k=2, I=64, S=2816),
    # S = 1408 (six tiles of 256, the last half wide): only the down
    # projection's input gradient switches (43 -> 29 row tiles)
    dict(T=11000, H=64, E=2, k=1, I=64, S=1408),
]


def _dense_rounds(T, N, bm, bn, cus=256):
    return -(-(-(-T // bm) * -(-N // bn)) // cus)


@pytest.mark.parametrize("spec", DENSE384_CASES)
def test_bf16_dense384_shared_parity(spec):
    """The shared expert's dense GEMMs on 384-row tiles (a 384-row tile is
    chosen when it fills fewer rounds of the CUs at 1.4 times the cost of a
    256-row tile; the last row tile runs on the 256-row family)."""
    T, S = spec["T"], spec["S"]
    assert 1.4 * _dense_rounds(T, S, 384, 256) < _dense_rounds(T, S, 256, 256)
    case = Case(**spec, dtype="bf16", w_std=0.05)
    g = gpu_run(case, d_aux=0.01, d_z=0.001)
    o = oracle_run(case, g["logits"], d_aux=0.01, d_z=0.001)
    _routing_equal(g, o)
    _check(case, g, o, 1e-2)


SKINNY_CASES = [
    # T <= 64: the forward streams expert weights (skinny kernels); backward
    # runs the tiled kernels on the skinny forward's saved activations
    dict(T=48, H=256, E=32, k=4, I=96, S=64),
    dict(T=64, H=136, E=4, k=4, I=40, S=0),        # every expert gets all 64 tokens
    dict(T=7, H=72, E=6, k=2, I=24, S=16),
    dict(T=64, H=200, E=8, k=2, I=72, S=24),       # ~16 rows per expert: both kernels
]


@pytest.mark.parametrize("spec", SKINNY_CASES)
def test_bf16_small_token_path_forward_backward(spec):
    case = Case(**spec, dtype="bf16", w_std=0.05)
    g = gpu_run(case, d_aux=0.01, d_z=0.001)
    o = oracle_run(case, g["logits"], d_aux=0.01, d_z=0.001)
    _routing_equal(g, o)
    _check(case, g, o, 1e-2)


def test_bf16_small_token_forward():
    # BASELINE config 4 shape scaled in H and I: 64 tokens, 128 experts, top-8, no shared
    case = Case(T=64, H=512, E=128, k=8, I=192, S=0, dtype="bf16", w_std=0.05)
    g = gpu_run(case, backward=False)
    o = oracle_run(case, g["logits"], backward=False)
    _routing_equal(g, o)
    _check(case, g, o, 1e-2, backward=False)


# ---------------------------------------------------------------- reproducibility

@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_bitwise_reproducible(dtype):
    case = Case(T=300, H=128, E=16, k=4, I=64, S=64, dtype=dtype, w_std=0.05)
    a = gpu_run(case, d_aux=0.01, d_z=0.001)
    b = gpu_run(case, d_aux=0.01, d_z=0.001)
    for n in ("out", "aux", "z", "dx", "router", "gate", "up", "down", "shared_down"):
        np.testing.assert_array_equal(np.nan_to_num(a[n]), np.nan_to_num(b[n]), err_msg=n)


@pytest.mark.parametrize("dtype,S,E", [("f32", 128, 16), ("bf16", 128, 16), ("bf16", 0, 16),
                                       ("bf16", 64, 2)])
def test_shared_stream_overlap_is_bitwise_serial(dtype, S, E):
    # the shared expert on the plan's second stream and the weight gradients
    # (and the forward's mean probabilities and losses) on its third give the
    # same bits as the serial order: no result depends on how the streams
    # interleave.  E = 2: 640 rows per expert, so the row-grouped GEMMs also
    # run their half-height tiles last.
    case = Case(T=640, H=128, E=E, k=2, I=64, S=S, dtype=dtype, w_std=0.05, seed=5)
    a = gpu_run(case, d_aux=0.01, d_z=0.001, overlap=True)
    b = gpu_run(case, d_aux=0.01, d_z=0.001, overlap=False)
    c = gpu_run(case, d_aux=0.01, d_z=0.001, overlap=2)  # shared-expert stream only
    names = ["out", "aux", "z", "dx", "router", "gate", "up", "down"]
    if S:
        names += ["shared_gate", "shared_up", "shared_down"]
    for n in names:
        np.testing.assert_array_equal(np.nan_to_num(a[n]), np.nan_to_num(b[n]), err_msg=n)
        np.testing.assert_array_equal(np.nan_to_num(c[n]), np.nan_to_num(b[n]), err_msg=n)


@pytest.mark.parametrize("skew", [0.0, 3.0])
def test_repeated_backward_is_bitwise_first(skew):
    # A plan's later backward calls may launch the gate/up weight gradient with
    # only its persistent workgroups (when the previous call's expert counts
    # ran whole experts per XCD); the first call launches the full grid.  Both
    # compute every tile once: the same bits.  E = 16 balanced (whole experts
    # per XCD) and skewed (tiles dealt over the XCDs).
    bias = zipf_bias(16, s=1.2, beta=skew) if skew else None
    case = Case(T=2048, H=128, E=16, k=2, I=64, S=0, dtype="bf16", w_std=0.05, seed=9,
                bias=bias)
    a = gpu_run(case, d_aux=0.01)
    b = gpu_run(case, d_aux=0.01, backwards=3)
    for n in ("dx", "router", "gate", "up", "down"):
        np.testing.assert_array_equal(np.nan_to_num(a[n]), np.nan_to_num(b[n]), err_msg=n)


def _whole_experts_per_xcd(counts):
    """Whether the gate/up weight gradient runs whole experts per XCD for these
    counts: experts ranked by count (ties by index) dealt to the 8 XCDs in a
    snake, and the busiest XCD within 8 % of the mean."""
    E = len(counts)
    rank = sorted(range(E), key=lambda e: (-int(counts[e]), e))
    load = [0] * 8
    for r, e in enumerate(rank):
        x = r % 8 if (r // 8) % 2 == 0 else 7 - r % 8
        load[x] += int(counts[e])
    return 100 * 8 * max(load) <= 108 * sum(load)


@pytest.mark.parametrize("shape", [dict(E=64, H=256, I=128), dict(E=16, H=1280, I=512)])
def test_repeated_backward_alternating_routing_on_one_plan(shape):
    # From its second backward a plan launches the gate/up weight gradient with
    # only its persistent workgroups when the previous call's counts ran whole
    # experts per XCD: here the grids (512 and 384 blocks) exceed the 256
    # persistent ones.  Alternating balanced and skewed routing on one plan
    # makes that expectation stale every other call (persistent over dealt
    # tiles, then a full grid over whole experts); each call must still give
    # the bits of a fresh plan's first backward.
    E, H, I = shape["E"], shape["H"], shape["I"]
    common = dict(T=2048, H=H, E=E, k=2, I=I, S=0, dtype="bf16", w_std=0.05, seed=21)
    bal = Case(bias=np.zeros(E, np.float32), **common)
    skw = Case(bias=zipf_bias(E, s=1.2, beta=3.0), **common)
    ref = {"bal": gpu_run(bal, d_aux=0.01), "skw": gpu_run(skw, d_aux=0.01)}
    assert _whole_experts_per_xcd(ref["bal"]["counts"]), "balanced case must run whole experts"
    assert not _whole_experts_per_xcd(ref["skw"]["counts"]), "skewed case must deal tiles"
    dev = torch.device("cuda:0")
    dt = torch.bfloat16
    t = {n: torch.tensor(v, device=dev).to(dt) for n, v in bal.p.items() if n != "router_bias"}
    biases = {"bal": torch.tensor(bal.p["router_bias"], device=dev),
              "skw": torch.tensor(skw.p["router_bias"], device=dev)}
    plan = Plan(bal.cfg, dt, dev)
    gate, up, down = (list(t[n].unbind(0)) for n in ("gate", "up", "down"))
    g_router, g_bias = torch.empty_like(t["router"]), torch.empty(E, device=dev)
    g_gate = [torch.empty_like(a) for a in gate]
    g_up = [torch.empty_like(a) for a in up]
    g_down = [torch.empty_like(a) for a in down]
    g, _keep_g = plan.grads_struct(g_router, g_gate, g_up, g_down, g_bias, None)
    da = torch.tensor(0.01, device=dev)
    dz = torch.tensor(0.0, device=dev)
    for call, name in enumerate(["bal", "skw", "bal", "skw", "skw", "bal", "bal"]):
        for a in g_gate + g_up + g_down:
            a.fill_(float("nan"))
        w, _keep_w = plan.weights_struct(t["router"], gate, up, down, biases[name], None)
        out, aux, z, saved = plan.forward(t["x"], w)
        dx = plan.backward(t["x"], t["dout"], w, g, saved, d_aux=da, d_z=dz)
        torch.cuda.synchronize()
        print(f"call {call} {name}", flush=True)
        got = {"dx": dx, "router": g_router, "gate": torch.stack(g_gate),
               "up": torch.stack(g_up), "down": torch.stack(g_down)}
        for n, v in got.items():
            np.testing.assert_array_equal(np.nan_to_num(v.float().cpu().numpy()),
                                          np.nan_to_num(ref[name][n]), err_msg=f"{call} {name} {n}")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_batch_invariance(dtype):
    # Routing is per token (reference tests/data_parallel.rs:333-347), and no
    # reduction crosses tokens in out or (with d_aux = d_z = 0) in dx: a token's
    # rows are bitwise the same whether it is processed alone or in a batch.
    # Both batches above 64 tokens, so both run the same (tiled) kernels.
    case = Case(T=256, H=128, E=16, k=2, I=64, S=64, dtype=dtype, w_std=0.05, seed=3)
    full = gpu_run(case)
    sub = gpu_run(case, x=case.p["x"][:100], dout=case.p["dout"][:100])
    np.testing.assert_array_equal(full["out"][:100], sub["out"])
    np.testing.assert_array_equal(full["dx"][:100], sub["dx"])
    np.testing.assert_array_equal(full["topk_idx"][:100], sub["topk_idx"])


def test_small_batch_path_agrees_with_tiled_path():
    # 37 tokens take the small-token (weight-streaming) forward in bf16, 256 the
    # tiled one: same routing, outputs within the bf16 bar.
    case = Case(T=256, H=128, E=16, k=2, I=64, S=64, dtype="bf16", w_std=0.05, seed=3)
    full = gpu_run(case)
    sub = gpu_run(case, x=case.p["x"][:37], dout=case.p["dout"][:37])
    np.testing.assert_array_equal(full["topk_idx"][:37], sub["topk_idx"])
    assert rel(sub["out"], full["out"][:37]) < 1e-2
    assert rel(sub["dx"], full["dx"][:37]) < 1e-2


# ---------------------------------------------------------------- forward only

@pytest.mark.parametrize("dtype,T", [("f32", 300), ("bf16", 300), ("bf16", 40), ("bf16", 9)])
def test_forward_only_matches_training_forward(dtype, T):
    # saved == NULL (eval under no_grad, reference src/eval/run.rs:74): the same
    # kernels without the gate / up pre-activation stores, so the same bits
    case = Case(T=T, H=128, E=16, k=2, I=64, S=64, dtype=dtype, w_std=0.05, seed=11)
    a = gpu_run(case, backward=False)
    b = gpu_run(case, backward=False, need_grad=False)
    for n in ("out", "aux", "z"):
        np.testing.assert_array_equal(a[n], b[n], err_msg=n)


def test_layer_under_no_grad_matches_grad_path():
    torch.manual_seed(0)
    dev = torch.device("cuda:0")
    cfg = MoeConfig(hidden_size=128, num_experts=8, experts_per_tok=2, intermediate_size=64)
    layer = MoeLayer(cfg, dtype=torch.bfloat16, device=dev)
    x = torch.randn(2, 50, 128, device=dev).to(torch.bfloat16)
    out_g, aux_g, z_g = layer(x)
    with torch.no_grad():
        out_n, aux_n, z_n = layer(x)
    assert out_g.requires_grad and not out_n.requires_grad
    assert torch.equal(out_g.detach(), out_n)
    assert torch.equal(aux_g.detach(), aux_n) and torch.equal(z_g.detach(), z_n)


# ---------------------------------------------------------------- recompute policy

@pytest.mark.parametrize("dtype,T", [("f32", 300), ("bf16", 300), ("bf16", 40), ("bf16", 9)])
def test_recompute_activations_is_bitwise_equal(dtype, T):
    # recompute_activations keeps only the routing state; the backward rebuilds
    # the activations with the forward's own launches, so every output and
    # gradient is the same bits as with the activations kept
    kw = dict(T=T, H=128, E=16, k=2, I=64, S=64, dtype=dtype, w_std=0.05, seed=13)
    keep = Case(**kw)
    rec = Case(recompute=True, **kw)
    a = gpu_run(keep, d_aux=0.01, d_z=0.001)
    b = gpu_run(rec, d_aux=0.01, d_z=0.001)
    for n in ("out", "aux", "z", "dx", "router", "gate", "up", "down", "shared_gate",
              "shared_up", "shared_down", "has_grad", "topk_idx", "perm"):
        np.testing.assert_array_equal(np.nan_to_num(a[n]), np.nan_to_num(b[n]), err_msg=n)
    # and the recomputing path against the oracle itself (the reference keeps
    # the recomputed layer numerically right: src/model/recompute/segment.rs:337-362)
    o = oracle_run(rec, b["logits"], d_aux=0.01, d_z=0.001)
    _routing_equal(b, o)
    _check(rec, b, o, 1e-5 if dtype == "f32" else 1e-2)


def test_recompute_shrinks_saved_state():
    dev = torch.device("cuda:0")
    kw = dict(hidden_size=256, num_experts=16, experts_per_tok=2, intermediate_size=128,
              shared_intermediate_size=128)
    keep = Plan(MoeConfig(**kw), torch.bfloat16, dev)
    rec = Plan(MoeConfig(recompute_activations=True, **kw), torch.bfloat16, dev)
    T = 1000
    # routing state only: no [T*k, I] / [T, S] activation is kept (a kept
    # forward holds G / U / A and the shared G / U / A; neither keeps a
    # [T*k, H] row: the GEMMs read x through the permutation and the expert
    # outputs Y are transient)
    act = 2 * (T * 2 * 128 * 3 + T * 128 * 3)
    assert keep.saved_bytes(T) - rec.saved_bytes(T) >= act
    for plan in (keep, rec):
        for field in ("x_perm", "expert_out"):
            off, nb = ctypes.c_size_t(), ctypes.c_size_t()
            _lib.check(_lib.load().moe_saved_field_range(
                plan.h, T, _lib.SAVED_FIELDS.index(field), ctypes.byref(off), ctypes.byref(nb)))
            assert nb.value == 0, field
    assert rec.saved_bytes(T) < 40 * T * 16
    assert rec.workspace_bytes(T) > keep.workspace_bytes(T)


# ---------------------------------------------------------------- block path (RMSNorm + residual)

BLOCK_CASES = [("f32", 300, 1e-5), ("bf16", 300, 1e-2), ("bf16", 40, 1e-2)]


@pytest.mark.parametrize("dtype,T,tol", BLOCK_CASES)
def test_block_forward_backward_parity(dtype, T, tol):
    # moe_block_forward / moe_block_backward against the block oracle
    # (RMSNorm -> layer -> residual add, float64), routed from the GPU's logits
    case = Case(T=T, H=128, E=16, k=2, I=64, S=64, dtype=dtype, w_std=0.05, seed=21)
    rng = np.random.default_rng(21)
    h = rounded(2.0 * rng.standard_normal((T, 128)), case.tdtype)
    nw = rounded(1.0 + 0.2 * rng.standard_normal(128), case.tdtype)
    eps = 1e-5
    g = gpu_block_run(case, h, nw, eps, d_aux=0.01, d_z=0.001)
    p = case.p
    o = mo.MoeBlockOracle(case.ocfg, eps)
    out, aux, z = o.forward(h, nw, p["router"], p["gate"], p["up"], p["down"], None,
                            p["shared_gate"], p["shared_up"], p["shared_down"],
                            logits_in=g["logits"])
    og = o.backward(p["dout"], d_aux=0.01, d_z=0.001)
    np.testing.assert_array_equal(g["has_grad"], og["has_grad"])
    hg = og["has_grad"].astype(bool)
    errs = {"out": rel(g["out"], out), "dh": rel(g["dh"], og["h"]),
            "d_norm_weight": rel(g["norm_weight"], og["norm_weight"]),
            "d_router": rel(g["router"], og["router"]),
            "aux": abs(float(g["aux"]) - aux) / abs(aux), "z": abs(float(g["z"]) - z) / abs(z)}
    for n in ("gate", "up", "down"):
        errs["d_" + n] = rel(g[n][hg], og[n][hg])
    for n in ("shared_gate", "shared_up", "shared_down"):
        errs["d_" + n] = rel(g[n], og[n])
    bad = {n: e for n, e in errs.items() if not e <= tol}
    assert not bad, f"over tolerance {tol}: {bad} (all: {errs})"


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_block_recompute_is_bitwise_equal(dtype):
    case = Case(T=200, H=128, E=8, k=2, I=64, S=64, dtype=dtype, w_std=0.05, seed=23)
    rng = np.random.default_rng(23)
    h = rounded(rng.standard_normal((200, 128)), case.tdtype)
    nw = rounded(1.0 + 0.2 * rng.standard_normal(128), case.tdtype)
    a = gpu_block_run(case, h, nw, 1e-6, d_aux=0.01)
    b = gpu_block_run(case, h, nw, 1e-6, d_aux=0.01, recompute=True)
    for n in ("out", "aux", "z", "dh", "norm_weight", "router", "gate", "up", "down",
              "shared_gate", "shared_up", "shared_down"):
        np.testing.assert_array_equal(np.nan_to_num(a[n]), np.nan_to_num(b[n]), err_msg=n)
    # the recomputed block against the block oracle
    p = case.p
    o = mo.MoeBlockOracle(case.ocfg, 1e-6)
    out, aux, z = o.forward(h, nw, p["router"], p["gate"], p["up"], p["down"], None,
                            p["shared_gate"], p["shared_up"], p["shared_down"],
                            logits_in=b["logits"])
    og = o.backward(p["dout"], d_aux=0.01, d_z=0.0)
    tol = 1e-5 if dtype == "f32" else 1e-2
    hg = og["has_grad"].astype(bool)
    errs = {"out": rel(b["out"], out), "dh": rel(b["dh"], og["h"]),
            "d_norm_weight": rel(b["norm_weight"], og["norm_weight"]),
            "d_router": rel(b["router"], og["router"])}
    for n in ("gate", "up", "down"):
        errs["d_" + n] = rel(b[n][hg], og[n][hg])
    for n in ("shared_gate", "shared_up", "shared_down"):
        errs["d_" + n] = rel(b[n], og[n])
    bad = {n: e for n, e in errs.items() if not e <= tol}
    assert not bad, f"over tolerance {tol}: {bad} (all: {errs})"


def test_block_plan_rejects_plain_entry_points():
    dev = torch.device("cuda:0")
    cfg = MoeConfig(hidden_size=64, num_experts=4, experts_per_tok=2, intermediate_size=32,
                    fused_block=True)
    plan = Plan(cfg, torch.float32, dev)
    x = torch.zeros(8, 64, device=dev)
    gate = [torch.zeros(32, 64, device=dev) for _ in range(4)]
    down = [torch.zeros(64, 32, device=dev) for _ in range(4)]
    w, _k = plan.weights_struct(torch.zeros(4, 64, device=dev), gate, gate, down)
    with pytest.raises(Exception, match="fused_block"):
        plan.forward(x, w)


# ---------------------------------------------------------------- packed experts from a checkpoint

def test_layer_from_packed_checkpoint_matches(tmp_path):
    # weights saved under the checkpoint names, loaded into packed [E, I, H]
    # storage on the GPU: the plan reads the packed tensors in place and gives
    # the same bits as the same weights held in memory
    from oxidizr_amd.checkpoint import PackedExperts, load_packed, save_packed
    case = Case(T=200, H=128, E=8, k=2, I=64, S=64, dtype="bf16", w_std=0.05, seed=31)
    p = case.p
    src = PackedExperts(*(torch.tensor(p[n]).to(torch.bfloat16)
                          for n in ("router", "gate", "up", "down")),
                        shared=tuple(torch.tensor(p[n]).to(torch.bfloat16)
                                     for n in ("shared_gate", "shared_up", "shared_down")))
    path = str(tmp_path / "moe.safetensors")
    save_packed(path, 0, src)
    dev = torch.device("cuda:0")
    pk = load_packed(path, 0, 128, 8, 64, 64, device=dev)
    plan = Plan(case.cfg, torch.bfloat16, dev)
    w, _keep = pk.weights_struct(plan)
    x = torch.tensor(p["x"], device=dev).to(torch.bfloat16)
    dout = torch.tensor(p["dout"], device=dev).to(torch.bfloat16)
    out, aux, z, saved = plan.forward(x, w)
    # gradients into packed [E, I, H] / [E, H, I] storage as well
    gpk = PackedExperts.empty(128, 8, 64, 64, dtype=torch.bfloat16, device=dev)
    for t in (gpk.gate, gpk.up, gpk.down):
        t.fill_(float("nan"))
    g, _keep_g = gpk.grads_struct(plan)
    has_grad = torch.empty(8, dtype=torch.uint8, device=dev)
    dx = plan.backward(x, dout, w, g, saved, d_aux=torch.tensor(0.01, device=dev),
                       d_z=torch.tensor(0.0, device=dev), has_grad=has_grad)
    torch.cuda.synchronize()
    logits = plan.saved_field(saved, 200, "logits").cpu().numpy()
    o = oracle_run(case, logits, d_aux=0.01)
    got = {"out": out.float().cpu().numpy(), "aux": aux.cpu().numpy(), "z": z.cpu().numpy(),
           "logits": logits, "has_grad": has_grad.cpu().numpy(), "dx": dx.float().cpu().numpy()}
    for f in ("probs", "topk_w", "topk_idx", "counts", "offsets", "perm", "inv_perm"):
        got[f] = plan.saved_field(saved, 200, f).cpu().numpy()
    for n in ("router", "gate", "up", "down"):
        got[n] = getattr(gpk, n).float().cpu().numpy()
    got["shared_gate"], got["shared_up"], got["shared_down"] = (
        t.float().cpu().numpy() for t in gpk.shared)
    _routing_equal(got, o)
    _check(case, got, o, 1e-2)
    # and the same bits as the same weights held as separate tensors
    ref = gpu_run(case, d_aux=0.01)
    np.testing.assert_array_equal(got["out"], ref["out"])
    np.testing.assert_array_equal(got["dx"], ref["dx"])
    assert float(aux) == float(ref["aux"])


# ---------------------------------------------------------------- the drop-in module

def _layer_from_case(case, dev):
    layer = MoeLayer(case.cfg, dtype=case.tdtype, device=dev)
    p = case.p
    with torch.no_grad():
        layer.router.gate.weight.copy_(torch.tensor(p["router"]))
        for e, ex in enumerate(layer.experts):
            ex.gate_proj.weight.copy_(torch.tensor(p["gate"][e]))
            ex.up_proj.weight.copy_(torch.tensor(p["up"][e]))
            ex.down_proj.weight.copy_(torch.tensor(p["down"][e]))
        if case.S:
            for n in ("gate", "up", "down"):
                getattr(layer.shared_expert, f"{n}_proj").weight.copy_(
                    torch.tensor(p[f"shared_{n}"]))
        if case.bias is not None:
            layer.router.bias.copy_(torch.tensor(p["router_bias"]))
    return layer


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_moe_layer_autograd_backward_matches_oracle(dtype):
    # MoeLayer(x [B, S, H]) -> (out, aux, z), then loss.backward() through the
    # autograd node: the Python stand-in of the Rust GradFn. Gradients land in
    # .grad in the reference's parameter order; an expert without a token gets
    # no gradient entry (.grad stays None, src/trainer.rs:556-566).
    bias = np.array([0, 0, -1e4, 0, 0, 0, 0, -1e4], np.float32)  # experts 2, 7 never chosen
    case = Case(T=120, H=64, E=8, k=2, I=48, S=32, dtype=dtype, w_std=0.1, seed=41, bias=bias)
    dev = torch.device("cuda:0")
    layer = _layer_from_case(case, dev)
    # parameter identity and order (src/model.rs:1887-1897, names :4890-4910)
    names = [n for n, _ in layer.trainable_parameters()]
    want = ["router.gate.weight", "router.gate.bias"]
    for e in range(8):
        want += [f"experts.{e}.{n}_proj.weight" for n in ("gate", "up", "down")]
    want += [f"shared_expert.{n}_proj.weight" for n in ("gate", "up", "down")]
    assert names == want
    assert all(a is b for (_, a), b in zip(layer.trainable_parameters(),
                                          [layer.router.gate.weight, layer.router.bias] +
                                          [getattr(ex, f"{n}_proj").weight
                                           for ex in layer.experts for n in ("gate", "up", "down")] +
                                          [getattr(layer.shared_expert, f"{n}_proj").weight
                                           for n in ("gate", "up", "down")]))
    x = torch.tensor(case.p["x"], device=dev).to(case.tdtype).reshape(2, 60, 64).requires_grad_()
    dout = torch.tensor(case.p["dout"], device=dev).to(case.tdtype).reshape(2, 60, 64)
    out, aux, z = layer(x)
    assert out.shape == (2, 60, 64)
    ((out * dout).sum() + 0.01 * aux + 0.001 * z).backward()
    torch.cuda.synchronize()
    logits = gpu_run(case, backward=False)["logits"]
    o = oracle_run(case, logits, d_aux=0.01, d_z=0.001)
    tol = 1e-5 if dtype == "f32" else 1e-2
    errs = {"out": rel(out.detach().float().cpu().numpy().reshape(120, 64), o["out"]),
            "aux": abs(float(aux.detach()) - o["aux"]) / abs(o["aux"]),
            "z": abs(float(z.detach()) - o["z"]) / abs(o["z"]),
            "dx": rel(x.grad.float().cpu().numpy().reshape(120, 64), o["x"]),
            "router": rel(layer.router.gate.weight.grad.float().cpu().numpy(), o["router"]),
            "router_bias": rel(layer.router.bias.grad.float().cpu().numpy(), o["router_bias"])}
    for e, ex in enumerate(layer.experts):
        for n in ("gate", "up", "down"):
            grad = getattr(ex, f"{n}_proj").weight.grad
            if not o["has_grad"][e]:
                assert grad is None, (e, n)
                continue
            errs[f"{n}{e}"] = rel(grad.float().cpu().numpy(), o[n][e])
    for n in ("gate", "up", "down"):
        errs[f"shared_{n}"] = rel(getattr(layer.shared_expert, f"{n}_proj").weight.grad.float()
                                  .cpu().numpy(), o[f"shared_{n}"])
    assert list(o["has_grad"]) == [1, 1, 0, 1, 1, 1, 1, 0]
    bad = {n: e for n, e in errs.items() if not e <= tol}
    assert not bad, f"over tolerance {tol}: {bad} (all: {errs})"


def test_alternating_gradient_buffers_match_oracle():
    # Three backward calls into two alternating sets of gradient buffers (the
    # pointer tables change on every call; they are uploaded through the
    # plan's staging ring, without synchronising the stream): every call's
    # gradients must match the oracle.
    case = Case(T=150, H=64, E=8, k=2, I=48, S=32, dtype="bf16", w_std=0.1, seed=43)
    dev = torch.device("cuda:0")
    t = {n: torch.tensor(v, device=dev).to(torch.bfloat16) for n, v in case.p.items()}
    plan = Plan(case.cfg, torch.bfloat16, dev)
    gate, up, down = (list(t[n].unbind(0)) for n in ("gate", "up", "down"))
    shared = (t["shared_gate"], t["shared_up"], t["shared_down"])
    w, _kw = plan.weights_struct(t["router"], gate, up, down, None, shared)
    out, aux, z, saved = plan.forward(t["x"], w)
    sets = []
    for _ in range(2):
        gr = {n: torch.full_like(t[n], float("nan")) for n in ("router", "gate", "up", "down")}
        gsh = [torch.full_like(a, float("nan")) for a in shared]
        g, keep = plan.grads_struct(gr["router"], list(gr["gate"].unbind(0)),
                                    list(gr["up"].unbind(0)), list(gr["down"].unbind(0)), None, gsh)
        sets.append((gr, gsh, g, keep))
    dxs = []
    for call in range(3):
        gr, gsh, g, _keep = sets[call % 2]
        dxs.append(plan.backward(t["x"], t["dout"], w, g, saved,
                                 d_aux=torch.tensor(0.01, device=dev)).float().cpu().numpy())
        torch.cuda.synchronize()
        got = {"dx": dxs[-1], "router": gr["router"].float().cpu().numpy()}
        for n in ("gate", "up", "down"):
            got[n] = gr[n].float().cpu().numpy()
        for n, a in zip(("shared_gate", "shared_up", "shared_down"), gsh):
            got[n] = a.float().cpu().numpy()
        if call == 0:
            logits = plan.saved_field(saved, 150, "logits").cpu().numpy()
            o = oracle_run(case, logits, d_aux=0.01)
        hg = o["has_grad"].astype(bool)
        errs = {"dx": rel(got["dx"], o["x"]), "router": rel(got["router"], o["router"])}
        for n in ("gate", "up", "down"):
            errs[n] = rel(got[n][hg], o[n][hg])
            assert np.isnan(got[n][~hg]).all(), (call, n)
        for n in ("shared_gate", "shared_up", "shared_down"):
            errs[n] = rel(got[n], o[n])
        assert max(errs.values()) <= 1e-2, (call, errs)
        for gt in (gr["router"], gr["gate"], gr["up"], gr["down"], *gsh):
            gt.fill_(float("nan"))  # the next call into this set must rewrite it
    np.testing.assert_array_equal(dxs[0], dxs[2])


def test_refused_table_leaves_the_plan_usable():
    # A call refused for a bad expert pointer must not leave the plan's cached
    # tables half-updated: the next good call with changed tables uploads them.
    case = Case(T=64, H=64, E=4, k=2, I=32, S=0, dtype="f32", w_std=0.1, seed=45)
    dev = torch.device("cuda:0")
    t = {n: torch.tensor(v, device=dev) for n, v in case.p.items()}
    plan = Plan(case.cfg, torch.float32, dev)
    gate, up, down = (list(t[n].unbind(0)) for n in ("gate", "up", "down"))
    w, _k = plan.weights_struct(t["router"], gate, up, down)
    first, _a, _b, _s = plan.forward(t["x"], w, need_grad=False)
    gate2 = [g.clone() * 2.0 for g in gate]
    bad = _lib.MoeWeightsC()
    bad.router = t["router"].data_ptr()
    tabs = [_lib.ptr_array([a.data_ptr() for a in gate2]),
            _lib.ptr_array([a.data_ptr() for a in up]),
            _lib.ptr_array([a.data_ptr() for a in down[:-1]] + [0])]  # NULL down pointer
    bad.gate, bad.up, bad.down = (ctypes.cast(a, ctypes.c_void_p) for a in tabs)
    with pytest.raises(_lib.MoeError, match="NULL"):
        plan.forward(t["x"], bad, need_grad=False)
    w2, _k2 = plan.weights_struct(t["router"], gate2, up, down)
    second, _a, _b, _s = plan.forward(t["x"], w2, need_grad=False)
    torch.cuda.synchronize()
    case2 = Case(T=64, H=64, E=4, k=2, I=32, S=0, dtype="f32", w_std=0.1, seed=45)
    case2.p["gate"] = case.p["gate"] * 2.0
    g2 = gpu_run(case2, backward=False)
    np.testing.assert_array_equal(second.cpu().numpy(), g2["out"])
    assert not np.array_equal(first.cpu().numpy(), second.cpu().numpy())
