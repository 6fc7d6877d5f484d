"""Seeded synthetic MoE-layer inputs shared by the tests, smoke() and bench.py.

Host generation is a counter-based SplitMix64 stream per tensor name, turned
into N(0, 1) by Box-Muller, so the same bytes can feed the GPU path and the CPU
oracle. Large benchmark shapes are generated on the device with torch's seeded
generator instead (bench.py), where host generation would take minutes.

The five workload shapes are the BASELINE configurations of the MoE layer
(oxidizr's config keys: num_experts, experts_per_tok, intermediate_size,
shared_expert_enabled; src/config.rs:125-131 in the reference).
"""
from dataclasses import dataclass, field

import numpy as np

_M64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def _fnv1a(name: str) -> int:
    h = 0xCBF29CE484222325
    for b in name.encode():
        h ^= b
        h = (h * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def _splitmix64(seed: int, n: int) -> np.ndarray:
    with np.errstate(over="ignore"):
        i = np.arange(1, n + 1, dtype=np.uint64)
        z = np.uint64(seed) + i * np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def normal(name: str, shape, std=1.0, seed=0) -> np.ndarray:
    """N(0, std^2) float32 array from the named stream."""
    n = int(np.prod(shape))
    m = (n + 1) // 2
    z = _splitmix64(_fnv1a(name) ^ (seed * 0x9E3779B97F4A7C15 & 0xFFFFFFFFFFFFFFFF), 2 * m)
    u = ((z >> np.uint64(11)).astype(np.float64) + 1.0) * (1.0 / 9007199254740992.0)
    u1, u2 = u[0::2], u[1::2]
    r = np.sqrt(-2.0 * np.log(u1))
    out = np.empty(2 * m)
    out[0::2] = r * np.cos(2 * np.pi * u2)
    out[1::2] = r * np.sin(2 * np.pi * u2)
    return (out[:n] * std).astype(np.float32).reshape(shape)


def bf16_round(a: np.ndarray) -> np.ndarray:
    """Round float32 values to bfloat16 (nearest-even) and return them as float32."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    lsb = (u >> np.uint64(16)) & np.uint64(1)
    r = ((u + np.uint64(0x7FFF) + lsb) >> np.uint64(16)) << np.uint64(16)
    out = (r & np.uint64(0xFFFFFFFF)).astype(np.uint32).view(np.float32)
    nan = np.isnan(a)
    if nan.any():
        out = out.copy()
        out[nan] = np.nan
    return out


@dataclass
class Workload:
    name: str
    T: int
    H: int
    E: int
    k: int
    I: int
    S: int = 0             # total shared-expert width (0: no shared expert)
    dtype: str = "bf16"    # "f32" or "bf16"
    w_std: float = 0.02
    backward: bool = True
    alpha: float = 0.01    # trainer load_balance_alpha
    skew: str = "none"     # "none" | "zipf" | "lognormal"
    batch: tuple = field(default=())


WORKLOADS = {
    1: Workload("cfg1_fp32_T1024_H384_E8_k2", 1024, 384, 8, 2, 1024, 0, "f32", batch=(2, 512)),
    2: Workload("cfg2_bf16_T8192_H2048_E16_k2_shared2816", 8192, 2048, 16, 2, 1408, 2816,
                batch=(4, 2048)),
    3: Workload("cfg3_bf16_T16384_H2048_E64_k6_shared2x1408_zipf", 16384, 2048, 64, 6, 1408,
                2 * 1408, alpha=0.0, skew="zipf"),
    4: Workload("cfg4_bf16_T64_H4096_E128_k8_fwd", 64, 4096, 128, 8, 1536, 0, backward=False,
                alpha=0.0),
    5: Workload("cfg5_bf16_T8192_H7168_E256_k8_shared2048_lognormal", 8192, 7168, 256, 8, 2048,
                2048, w_std=0.006, alpha=0.0, skew="lognormal"),
}


def host_problem(T, H, E, k, I, S=0, w_std=0.02, seed=0, bias=None, dtype="f32"):
    """Seeded float32 inputs (bf16-representable when dtype == 'bf16').
    Weights are packed per expert: gate/up [E, I, H], down [E, H, I]."""
    f = bf16_round if dtype == "bf16" else (lambda a: a)
    p = {
        "x": f(normal("x", (T, H), 1.0, seed)),
        "router": f(normal("router.gate.weight", (E, H), w_std, seed)),
        "gate": f(normal("experts.gate_proj.weight", (E, I, H), w_std, seed)),
        "up": f(normal("experts.up_proj.weight", (E, I, H), w_std, seed)),
        "down": f(normal("experts.down_proj.weight", (E, H, I), w_std, seed)),
        "dout": f(normal("d_out", (T, H), 1.0, seed)),
    }
    if S:
        p["shared_gate"] = f(normal("shared_expert.gate_proj.weight", (S, H), w_std, seed))
        p["shared_up"] = f(normal("shared_expert.up_proj.weight", (S, H), w_std, seed))
        p["shared_down"] = f(normal("shared_expert.down_proj.weight", (H, S), w_std, seed))
    if bias is not None:
        p["router_bias"] = np.asarray(bias, np.float32)
    return p


def zipf_bias(E, s=1.2, beta=1.0, seed=0):
    """Per-expert logit bias beta*log(rank^-s) over a seeded permutation of experts."""
    rng = np.random.default_rng(seed + 12345)
    ranks = rng.permutation(E) + 1
    return (beta * np.log(ranks.astype(np.float64) ** (-s))).astype(np.float32)


def lognormal_bias(E, sigma=0.5, seed=0):
    """Per-expert logit bias log(load) with load ~ lognormal(0, sigma)."""
    rng = np.random.default_rng(seed + 54321)
    return rng.normal(0.0, sigma, size=E).astype(np.float32)


def skew_bias(T, k, E, skew, x, router):
    """Per-expert fp32 router-logit bias on the device that shapes the expert
    loads of a BASELINE workload, and a dict describing the realised skew.

    "zipf" (config 3): b_e = beta * log(rank_e^-1.2) over a seeded permutation,
    beta bisected so the busiest expert gets about 8x the mean load; if no
    expert is then empty, the least likely one is pushed to -1e4 (it gets no
    token). "lognormal" (config 5): b_e fitted so the realised top-k loads
    follow lognormal(0, 0.5) shares. "none": (None, {}).
    x [T, H] and router [E, H] are device tensors; the bias depends on their
    logits, so the same inputs always give the same bias."""
    import torch
    if skew not in ("zipf", "lognormal"):
        return None, {}
    dev = x.device
    base = x.float() @ router.float().t()
    if skew == "lognormal":
        target = np.exp(lognormal_bias(E, 0.5).astype(np.float64))
        target = target / target.sum() * (T * k)
        tgt = torch.tensor(target, dtype=torch.float32, device=dev)
        b = torch.log(tgt / tgt.mean()) * 0.1
        for _ in range(60):
            idx = torch.topk(base + b, k, dim=1).indices
            c = torch.bincount(idx.flatten(), minlength=E).float()
            b = b + 0.3 * torch.log((tgt + 1.0) / (c + 1.0))
        idx = torch.topk(base + b, k, dim=1).indices
        c = torch.bincount(idx.flatten(), minlength=E).float()
        lc = torch.log(c.clamp(min=1.0))
        return b, {"load_log_std": round(float(lc.std()), 3),
                   "load_max_over_mean": round(float(c.max() / c.mean()), 2)}
    mean = T * k / E

    def counts(beta):
        b = torch.tensor(zipf_bias(E, 1.2, beta), device=dev)
        idx = torch.topk(base + b, k, dim=1).indices
        return torch.bincount(idx.flatten(), minlength=E), b

    lo, hi = 0.0, 20.0
    for _ in range(30):  # busiest expert at ~8x the mean load
        mid = 0.5 * (lo + hi)
        c, _ = counts(mid)
        if c.max().item() < 8 * mean:
            lo = mid
        else:
            hi = mid
    c, b = counts(lo)
    b = b.clone()
    if (c == 0).sum().item() == 0:  # push the tail: the least likely expert gets no token
        b[int(np.argmin(b.cpu().numpy()))] = -1e4
    return b, {"zipf_beta": round(lo, 4)}
