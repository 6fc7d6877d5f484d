"""Pins the CPU oracle (oracle/moe_oracle.cpp) before anything is checked
against it.

The reference's MoE arithmetic lives in boostr 0.10.0, which is absent, and the
reference holds no golden vectors for it (its MoE tests are structural:
src/model.rs:7497-7529, :8499-8534, tests/shared_expert.rs:66-120). The oracle
is therefore pinned by checks that a plausible mistake would fail:
  * routing: brute-force ordering with adversarial ties, softmax/logsumexp
    from scipy, the k == E special case (src/model.rs:7219-7222);
  * dispatch: integer invariants and numpy's stable argsort;
  * forward: a dense-gate torch restatement (tests/dense_ref.py) that never
    permutes tokens, plus closed forms of the aux and z losses;
  * backward: torch autograd of the dense restatement and central finite
    differences of the oracle's own forward;
  * unrouted experts: has_grad == 0 and untouched gradient buffers
    (src/trainer.rs:556-566).
"""
import numpy as np
import pytest
import torch
from scipy.special import logsumexp, softmax

from oracle import moe_oracle as mo
from oxidizr_amd.synth import host_problem, zipf_bias
from tests.dense_ref import dense_block, dense_moe

pytestmark = pytest.mark.filterwarnings("ignore::RuntimeWarning")


def _rel(a, b):
    a = np.asarray(a, np.float64); b = np.asarray(b, np.float64)
    return np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300)


def _problem(cfg, seed=0, bias=None):
    return host_problem(cfg.T, cfg.H, cfg.E, cfg.k, cfg.I, cfg.S, w_std=0.3, seed=seed, bias=bias)


def _run(cfg, p, precision=64):
    o = mo.MoeOracle(cfg, precision)
    out, aux, z = o.forward(p["x"], p["router"], p["gate"], p["up"], p["down"],
                            p.get("router_bias"), p.get("shared_gate"), p.get("shared_up"),
                            p.get("shared_down"))
    return o, out, aux, z


# ---------------------------------------------------------------- routing

@pytest.mark.parametrize("E,k", [(4, 1), (4, 2), (8, 3), (16, 8), (5, 5)])
def test_route_brute_force_with_ties(E, k):
    rng = np.random.default_rng(E * 10 + k)
    T = 200
    logits = rng.integers(-2, 3, size=(T, E)).astype(np.float64)  # many exact ties
    cfg = mo.make_cfg(T, 4, E, k, 4)
    probs, lse, idx, w = mo.route(cfg, logits)
    for t in range(T):
        # order by (-logit, index): largest first, lowest index wins ties
        want = sorted(range(E), key=lambda e: (-logits[t, e], e))[:k]
        assert list(idx[t]) == want
    np.testing.assert_allclose(probs, softmax(logits, axis=1), rtol=1e-13, atol=0)
    np.testing.assert_allclose(lse, logsumexp(logits, axis=1), rtol=1e-13)
    np.testing.assert_allclose(w, np.take_along_axis(probs, idx, 1), rtol=0, atol=0)


def test_route_k_equals_e_selects_all_in_descending_order():
    rng = np.random.default_rng(3)
    T, E = 50, 6
    logits = rng.normal(size=(T, E))
    cfg = mo.make_cfg(T, 4, E, E, 4)
    _, _, idx, w = mo.route(cfg, logits)
    np.testing.assert_array_equal(idx, np.argsort(-logits, axis=1, kind="stable"))
    np.testing.assert_allclose(w.sum(1), 1.0, rtol=1e-13)


def test_route_temperature_and_renormalisation():
    rng = np.random.default_rng(4)
    T, E, k = 40, 8, 3
    logits = rng.normal(size=(T, E)) * 3
    cfg = mo.make_cfg(T, 4, E, k, 4, tau=2.5, norm_topk=True)
    probs, lse, idx, w = mo.route(cfg, logits)
    np.testing.assert_allclose(probs, softmax(logits / 2.5, axis=1), rtol=1e-13)
    np.testing.assert_allclose(lse, logsumexp(logits / 2.5, axis=1), rtol=1e-13)
    sel = np.take_along_axis(probs, idx, 1)
    np.testing.assert_allclose(w, sel / sel.sum(1, keepdims=True), rtol=1e-13)


# ---------------------------------------------------------------- dispatch

@pytest.mark.parametrize("T,E,k", [(1, 4, 2), (37, 8, 2), (300, 64, 6), (64, 128, 8), (0, 4, 2)])
def test_dispatch_invariants(T, E, k):
    rng = np.random.default_rng(T + E)
    idx = np.array([rng.permutation(E)[:k] for _ in range(T)], np.int32).reshape(T, k)
    counts, offsets, perm, inv = mo.dispatch(idx, E)
    flat = idx.reshape(-1)
    assert counts.sum() == T * k
    np.testing.assert_array_equal(counts, np.bincount(flat, minlength=E))
    np.testing.assert_array_equal(offsets, np.concatenate([[0], np.cumsum(counts)]))
    assert sorted(perm.tolist()) == list(range(T * k))          # bijection
    np.testing.assert_array_equal(inv[perm], np.arange(T * k))  # inv_perm o perm = id
    np.testing.assert_array_equal(perm, np.argsort(flat, kind="stable"))  # expert, then token
    for e in range(E):
        seg = perm[offsets[e]:offsets[e + 1]]
        assert np.all(flat[seg] == e)
        assert np.all(np.diff(seg // k) > 0)  # token ascending inside a segment


def test_dispatch_rejects_out_of_range():
    with pytest.raises(ValueError):
        mo.dispatch(np.array([[0, 4]], np.int32), 4)


# ---------------------------------------------------------------- forward

CASES = [
    dict(T=24, H=8, E=4, k=2, I=16, S=0),
    dict(T=20, H=12, E=5, k=3, I=8, S=16),
    dict(T=16, H=8, E=3, k=3, I=8, S=8, norm_topk=True, tau=1.7, shared_scale=0.5),
    dict(T=30, H=8, E=6, k=2, I=8, S=0, has_bias=True, aux_switch=0.3, aux_sqprob=2.0),
]


@pytest.mark.parametrize("case", CASES)
def test_forward_matches_dense_restatement(case):
    cfg = mo.make_cfg(**case)
    bias = zipf_bias(cfg.E, beta=0.8) if cfg.has_bias else None
    p = _problem(cfg, bias=bias)
    o, out, aux, z = _run(cfg, p)
    dout_, daux_, dz_, _, routing = dense_moe(p, cfg, need_grad=False)
    np.testing.assert_array_equal(o.get("topk_idx"), routing["idx"])
    np.testing.assert_array_equal(o.get("counts"), routing["counts"])
    assert _rel(out, dout_) < 1e-12
    assert abs(aux - daux_) < 1e-12 * max(1, abs(daux_))
    assert abs(z - dz_) < 1e-12 * max(1, abs(dz_))


def test_aux_and_z_closed_forms_on_equal_logits():
    # equal logits: probs are 1/E for every token, so P_e = 1/E and both aux
    # terms equal 1 whatever the routing; lse = log E gives z = (log E)^2.
    cfg = mo.make_cfg(T=32, H=8, E=8, k=2, I=8)
    p = _problem(cfg)
    p["router"] = np.zeros_like(p["router"])
    o, out, aux, z = _run(cfg, p)
    assert abs(aux - 2.0) < 1e-14
    assert abs(z - np.log(8) ** 2) < 1e-13
    np.testing.assert_array_equal(o.get("topk_idx"), np.tile([0, 1], (32, 1)))  # ties -> low index
    np.testing.assert_array_equal(o.get("counts"), [32, 32, 0, 0, 0, 0, 0, 0])


def test_single_expert_reduces_to_dense_swiglu():
    cfg = mo.make_cfg(T=10, H=6, E=1, k=1, I=12)
    p = _problem(cfg)
    o, out, _, _ = _run(cfg, p)
    x, g, u, d = p["x"].astype(np.float64), p["gate"][0], p["up"][0], p["down"][0]
    G = x @ g.T.astype(np.float64)
    want = ((G / (1 + np.exp(-G))) * (x @ u.T.astype(np.float64))) @ d.T.astype(np.float64)
    assert _rel(out, want) < 1e-13


def test_two_shared_experts_equal_one_concatenated():
    # The workloads with "2 shared experts" run one shared SwiGLU of the summed
    # width; summing two SwiGLU experts equals concatenating gate/up rows and
    # down columns.
    cfg = mo.make_cfg(T=12, H=8, E=2, k=1, I=8, S=16)
    p = _problem(cfg)
    _, out, _, _ = _run(cfg, p)
    cfg0 = mo.make_cfg(T=12, H=8, E=2, k=1, I=8, S=0)
    _, out_routed, _, _ = _run(cfg0, p)
    x = p["x"].astype(np.float64)
    sh = 0
    for h in (slice(0, 8), slice(8, 16)):
        G = x @ p["shared_gate"][h].T
        sh = sh + ((G / (1 + np.exp(-G))) * (x @ p["shared_up"][h].T)) @ p["shared_down"][:, h].T
    assert _rel(out, out_routed + sh) < 1e-13


# ---------------------------------------------------------------- backward

@pytest.mark.parametrize("case", CASES)
def test_backward_matches_autograd(case):
    cfg = mo.make_cfg(**case)
    bias = zipf_bias(cfg.E, beta=0.8) if cfg.has_bias else None
    p = _problem(cfg, seed=1, bias=bias)
    o, *_ = _run(cfg, p)
    g = o.backward(p["dout"], d_aux=0.37, d_z=0.11)
    *_, want, _ = dense_moe(p, cfg, need_grad=True, d_aux=0.37, d_z=0.11)
    assert _rel(g["x"], want["x"]) < 1e-11
    assert _rel(g["router"], want["router"]) < 1e-11
    if cfg.has_bias:
        assert _rel(g["router_bias"], want["router_bias"]) < 1e-11
    for e in range(cfg.E):
        if g["has_grad"][e]:
            for n in ("gate", "up", "down"):
                assert _rel(g[n][e], want[n][e]) < 1e-11, (n, e)
        else:
            assert np.isnan(g["gate"][e]).all() and np.isnan(g["down"][e]).all()
            assert not np.any(want["gate"][e]) and not np.any(want["down"][e])
    if cfg.S:
        for n in ("shared_gate", "shared_up", "shared_down"):
            assert _rel(g[n], want[n]) < 1e-11, n


def test_backward_finite_differences():
    cfg = mo.make_cfg(T=6, H=8, E=4, k=2, I=16, S=16, has_bias=True, norm_topk=True, tau=1.3)
    p = _problem(cfg, seed=2, bias=np.array([0.1, -0.2, 0.3, 0.0], np.float32))
    d_aux, d_z = 0.7, 0.3

    def loss(pp):
        _, out, aux, z = _run(cfg, pp)
        return float((out * pp["dout"].astype(np.float64)).sum() + d_aux * aux + d_z * z)

    o, *_ = _run(cfg, {n: v.astype(np.float64) for n, v in p.items()})
    idx0 = o.get("topk_idx")
    g = o.backward(p["dout"], d_aux=d_aux, d_z=d_z)
    rng = np.random.default_rng(7)
    names = {"x": "x", "router": "router", "router_bias": "router_bias", "gate": "gate",
             "up": "up", "down": "down", "shared_gate": "shared_gate",
             "shared_up": "shared_up", "shared_down": "shared_down"}
    eps = 1e-6
    for n, gn in names.items():
        base = {m: v.astype(np.float64) for m, v in p.items()}
        V = rng.normal(size=base[n].shape)
        if n in ("gate", "up", "down"):
            V[~g["has_grad"].astype(bool)] = 0  # unrouted experts carry NaN sentinels
        plus = dict(base); plus[n] = base[n] + eps * V
        minus = dict(base); minus[n] = base[n] - eps * V
        fd = (loss(plus) - loss(minus)) / (2 * eps)
        gv = np.nan_to_num(g[gn])
        an = float((gv * V).sum())
        assert abs(fd - an) <= 1e-6 * max(1.0, abs(an)), (n, fd, an)
    o2, *_ = _run(cfg, p)
    np.testing.assert_array_equal(o2.get("topk_idx"), idx0)


def test_unrouted_expert_has_no_gradient_entry():
    cfg = mo.make_cfg(T=16, H=8, E=4, k=1, I=8, has_bias=True)
    p = _problem(cfg, bias=np.array([0.0, 0.0, -1e6, 0.0], np.float32))  # expert 2 never chosen
    o, *_ = _run(cfg, p)
    assert o.get("counts")[2] == 0
    g = o.backward(p["dout"], d_aux=0.01)
    assert g["has_grad"][2] == 0 and g["has_grad"][[0, 1, 3]].all()
    assert np.isnan(g["gate"][2]).all() and np.isnan(g["up"][2]).all() and np.isnan(g["down"][2]).all()
    assert np.isfinite(g["x"]).all() and np.isfinite(g["router"]).all()


def test_oracle_fp32_matches_fp64():
    cfg = mo.make_cfg(T=64, H=32, E=8, k=2, I=48, S=32)
    p = _problem(cfg, seed=3)
    o64, out64, aux64, z64 = _run(cfg, p, 64)
    o32, out32, aux32, z32 = _run(cfg, p, 32)
    np.testing.assert_array_equal(o64.get("topk_idx"), o32.get("topk_idx"))
    assert _rel(out32, out64) < 1e-5
    g64 = o64.backward(p["dout"], 0.1, 0.1)
    g32 = o32.backward(p["dout"], 0.1, 0.1)
    for n in ("x", "router", "gate", "up", "down", "shared_gate", "shared_down"):
        assert _rel(np.nan_to_num(g32[n]), np.nan_to_num(g64[n])) < 1e-5, n


def test_oracle_is_deterministic():
    cfg = mo.make_cfg(T=128, H=32, E=8, k=2, I=32, S=16)
    p = _problem(cfg, seed=4)
    a, out_a, *_ = _run(cfg, p, 32)
    b, out_b, *_ = _run(cfg, p, 32)
    np.testing.assert_array_equal(out_a, out_b)
    ga, gb = a.backward(p["dout"], 0.1, 0.1), b.backward(p["dout"], 0.1, 0.1)
    for n in ("x", "router", "gate", "shared_down"):
        np.testing.assert_array_equal(ga[n], gb[n])


# ---------------------------------------------------------------- block path

def test_rmsnorm_matches_torch_rms_norm_and_closed_forms():
    rng = np.random.default_rng(5)
    h = rng.standard_normal((7, 24))
    w = rng.standard_normal(24)
    x, rstd = mo.rmsnorm_forward(h, w, 1e-6)
    want = torch.nn.functional.rms_norm(torch.tensor(h), (24,), torch.tensor(w), 1e-6).numpy()
    assert _rel(x, want) < 1e-14
    # a constant row c normalises to sign(c) * w (up to eps); scaling a row
    # leaves the result unchanged; eps enters under the square root
    c = np.full((1, 24), -3.0)
    xc, rc = mo.rmsnorm_forward(c, w, 0.0)
    assert _rel(xc[0], -w) < 1e-15 and abs(rc[0] - 1 / 3.0) < 1e-15
    x5, _ = mo.rmsnorm_forward(5.0 * h, w, 0.0)
    x1, _ = mo.rmsnorm_forward(h, w, 0.0)
    assert _rel(x5, x1) < 1e-14
    _, r_eps = mo.rmsnorm_forward(c, w, 7.0)
    assert abs(r_eps[0] - 1 / 4.0) < 1e-15


@pytest.mark.parametrize("case", CASES[:2])
def test_block_forward_backward_match_autograd(case):
    cfg = mo.make_cfg(**case)
    p = _problem(cfg, seed=3)
    rng = np.random.default_rng(9)
    pb = dict(p)
    pb["h"] = pb.pop("x") * 3.0
    pb["norm_weight"] = 1.0 + 0.3 * rng.standard_normal(cfg.H)
    eps = 1e-5
    o = mo.MoeBlockOracle(cfg, eps)
    out, aux, z = o.forward(pb["h"], pb["norm_weight"], pb["router"], pb["gate"], pb["up"],
                            pb["down"], None, pb.get("shared_gate"), pb.get("shared_up"),
                            pb.get("shared_down"))
    g = o.backward(pb["dout"], d_aux=0.37, d_z=0.11)
    want_out, want_aux, want_z, want, _ = dense_block(pb, cfg, eps, d_aux=0.37, d_z=0.11)
    assert _rel(out, want_out) < 1e-12
    assert abs(aux - want_aux) < 1e-12 and abs(z - want_z) < 1e-12
    assert _rel(g["h"], want["h"]) < 1e-11
    assert _rel(g["norm_weight"], want["norm_weight"]) < 1e-11
    assert _rel(g["router"], want["router"]) < 1e-11
