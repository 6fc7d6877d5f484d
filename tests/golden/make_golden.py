"""Writes the MoE golden fixtures (tests/golden/*.npz) -- test infrastructure.

The reference's MoE arithmetic (boostr 0.10.0, boostr::nn::moe) is absent from
the reference tree and its tests hold no MoE vectors, so the expected values
come from tests/dense_ref.py: an fp64 torch restatement that runs every expert
on every token and mixes them with a dense top-k gate matrix (no histogram,
permutation or gather), with gradients from torch autograd.  The fixtures pin
the oracle and the HIP path to that independent computation.

Shapes follow the reference's own MoE test fixtures: src/model/recompute/
fixtures.rs:36-64 (H=16, E=4, top-2, shared expert), src/model.rs:7219-7222
(experts_per_tok == num_experts) and tests/serving_parity.rs:48-90 (E=3,
k=2).  Every case keeps a margin between the k-th and (k+1)-th logit so that
fp32 routing cannot flip a selection.

Run from the repository root:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle.moe_oracle import make_cfg  # noqa: E402  (config struct only)
from oxidizr_amd.synth import host_problem  # noqa: E402
from tests.dense_ref import dense_moe  # noqa: E402

CASES = {
    "recompute_fixture_shape": dict(T=32, H=16, E=4, k=2, I=16, S=16, seed=11),
    "k_equals_e_renorm_temp_bias": dict(T=24, H=24, E=3, k=3, I=8, S=0, seed=12, norm_topk=True,
                                        tau=1.7, bias=True),
    "serving_parity_shape_coefs": dict(T=40, H=16, E=3, k=2, I=16, S=8, seed=13, aux_switch=0.3,
                                       aux_sqprob=2.0, shared_scale=0.5),
    "eight_experts_top2": dict(T=48, H=32, E=8, k=2, I=24, S=0, seed=14),
}
D_AUX, D_Z = 0.01, 0.001
MARGIN = 1e-3


def build(name, spec):
    spec = dict(spec)
    seed = spec.pop("seed")
    bias = spec.pop("bias", False)
    for attempt in range(100):
        s = seed * 1000 + attempt
        b = np.linspace(0.3, -0.3, spec["E"]).astype(np.float32) if bias else None
        p = host_problem(spec["T"], spec["H"], spec["E"], spec["k"], spec["I"], spec["S"],
                         w_std=0.2, seed=s, bias=b)
        cfg = make_cfg(spec["T"], spec["H"], spec["E"], spec["k"], spec["I"], spec["S"],
                       norm_topk=spec.get("norm_topk", False), has_bias=bias,
                       tau=spec.get("tau", 1.0), shared_scale=spec.get("shared_scale", 1.0),
                       aux_switch=spec.get("aux_switch", 1.0),
                       aux_sqprob=spec.get("aux_sqprob", 1.0))
        lg = p["x"].astype(np.float64) @ p["router"].astype(np.float64).T
        if bias:
            lg = lg + b
        srt = -np.sort(-lg, axis=1)
        if spec["k"] < spec["E"] and (srt[:, spec["k"] - 1] - srt[:, spec["k"]]).min() < MARGIN:
            continue
        out, aux, z, grads, routing = dense_moe(p, cfg, need_grad=True, d_aux=D_AUX, d_z=D_Z)
        arrays = {f"in_{n}": v for n, v in p.items()}
        arrays.update({"out": out, "aux": np.float64(aux), "z": np.float64(z),
                       "topk_idx": routing["idx"], "counts": routing["counts"],
                       "logits": routing["logits"], "d_aux": np.float64(D_AUX),
                       "d_z": np.float64(D_Z)})
        arrays.update({f"grad_{n}": v for n, v in grads.items()})
        meta = dict(spec, bias=bias, seed=s)
        arrays["meta"] = np.array(repr(sorted(meta.items())))
        np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **arrays)
        return s
    raise RuntimeError(f"{name}: no seed with routing margin {MARGIN}")


if __name__ == "__main__":
    for n, sp in CASES.items():
        print(n, "seed", build(n, sp))
