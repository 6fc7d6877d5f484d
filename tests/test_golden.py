"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py
from the dense fp64 torch restatement): the CPU oracle must reproduce them to
fp64 accuracy, the HIP path (fp32) to the 1e-5 relative bar, with routing
(top-k indices, expert counts) bit-exact."""
import ast
import glob
import os

import numpy as np
import pytest

from oracle import moe_oracle as mo

HERE = os.path.dirname(os.path.abspath(__file__))
FILES = sorted(glob.glob(os.path.join(HERE, "golden", "*.npz")))
GRADS = ("x", "router", "router_bias", "gate", "up", "down", "shared_gate", "shared_up",
         "shared_down")


def _load(path):
    z = np.load(path)  # allow_pickle stays False: plain arrays only
    meta = dict(ast.literal_eval(str(z["meta"])))
    ins = {k[3:]: z[k] for k in z.files if k.startswith("in_")}
    return z, meta, ins


def _rel(a, b):
    a = np.asarray(a, np.float64); b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def _cfg(meta):
    return mo.make_cfg(meta["T"], meta["H"], meta["E"], meta["k"], meta["I"], meta["S"],
                       norm_topk=meta.get("norm_topk", False), has_bias=meta["bias"],
                       tau=meta.get("tau", 1.0), shared_scale=meta.get("shared_scale", 1.0),
                       aux_switch=meta.get("aux_switch", 1.0),
                       aux_sqprob=meta.get("aux_sqprob", 1.0))


def test_fixtures_present():
    assert len(FILES) >= 4


@pytest.mark.parametrize("path", FILES, ids=lambda p: os.path.basename(p)[:-4])
def test_oracle_reproduces_golden(path):
    z, meta, p = _load(path)
    o = mo.MoeOracle(_cfg(meta), 64)
    out, aux, zl = o.forward(p["x"], p["router"], p["gate"], p["up"], p["down"],
                             p.get("router_bias"), p.get("shared_gate"), p.get("shared_up"),
                             p.get("shared_down"))
    np.testing.assert_array_equal(o.get("topk_idx"), z["topk_idx"])
    np.testing.assert_array_equal(o.get("counts"), z["counts"])
    assert _rel(out, z["out"]) < 1e-11
    assert abs(aux - float(z["aux"])) < 1e-12 * max(1.0, abs(float(z["aux"])))
    assert abs(zl - float(z["z"])) < 1e-12 * max(1.0, abs(float(z["z"])))
    g = o.backward(p["dout"], d_aux=float(z["d_aux"]), d_z=float(z["d_z"]))
    for n in GRADS:
        if f"grad_{n}" in z.files and g.get(n) is not None:
            want = z[f"grad_{n}"]
            if n in ("gate", "up", "down"):
                hg = g["has_grad"].astype(bool)
                assert not np.any(want[~hg])
                assert _rel(g[n][hg], want[hg]) < 1e-10, n
            else:
                assert _rel(g[n], want) < 1e-10, n


@pytest.mark.gpu
@pytest.mark.parametrize("path", FILES, ids=lambda p: os.path.basename(p)[:-4])
def test_hip_reproduces_golden(path):
    from tests.gpu_helpers import Case, gpu_run
    z, meta, p = _load(path)
    case = Case(meta["T"], meta["H"], meta["E"], meta["k"], meta["I"], meta["S"], dtype="f32",
                bias=p.get("router_bias"), norm_topk=meta.get("norm_topk", False),
                tau=meta.get("tau", 1.0), shared_scale=meta.get("shared_scale", 1.0),
                aux_switch=meta.get("aux_switch", 1.0), aux_sqprob=meta.get("aux_sqprob", 1.0))
    case.p = {n: v.astype(np.float32) for n, v in p.items()}
    g = gpu_run(case, d_aux=float(z["d_aux"]), d_z=float(z["d_z"]))
    np.testing.assert_array_equal(g["topk_idx"], z["topk_idx"])
    np.testing.assert_array_equal(g["counts"], z["counts"])
    errs = {"out": _rel(g["out"], z["out"]), "dx": _rel(g["dx"], z["grad_x"]),
            "router": _rel(g["router"], z["grad_router"])}
    errs["aux"] = abs(float(g["aux"]) - float(z["aux"])) / max(abs(float(z["aux"])), 1e-30)
    errs["z"] = abs(float(g["z"]) - float(z["z"])) / max(abs(float(z["z"])), 1e-30)
    hg = g["has_grad"].astype(bool)
    for n in ("gate", "up", "down"):
        errs[n] = _rel(g[n][hg], z[f"grad_{n}"][hg])
    for n in ("router_bias", "shared_gate", "shared_up", "shared_down"):
        if f"grad_{n}" in z.files and g.get(n) is not None:
            errs[n] = _rel(g[n], z[f"grad_{n}"])
    bad = {n: e for n, e in errs.items() if not e <= 1e-5}
    assert not bad, (bad, errs)
