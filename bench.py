#!/usr/bin/env python3
"""MoE layer forward + backward throughput on one MI355X.

One step = one forward and one backward pass of the MoE layer over one batch of
synthetic tokens (every gradient written). Default workload
(T=8192, H=2048, E=16, top-2, I=1408, shared 2816, bf16, alpha 0.01).
Prints ONE JSON line. Other BASELINE configs: --config {1,3,4,5}.

Inputs live in HBM before timing starts; random-init weights and N(0,1)
activations/upstream gradients are generated on the device with a seeded
generator. Configs 3 and 5 skew routing with a fixed per-expert logit bias.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_FP32_TFLOPS = 157.3    # MI355X fp32 matrix
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def gen_weights(torch, shape, std, gen, dtype, dev):
    t = torch.empty(shape, dtype=dtype, device=dev)
    t.normal_(0.0, std, generator=gen)
    return t


def measured_traffic(workload):
    """Bytes per launch recorded in profiles/*.md ("traffic_bytes_per_launch
    <workload>: <bytes>"), or None."""
    pdir = os.path.join(ROOT, "profiles")
    if not os.path.isdir(pdir):
        return None
    key = f"traffic_bytes_per_launch {workload}:"
    for name in sorted(os.listdir(pdir)):
        if not name.endswith((".md", ".txt")):
            continue
        with open(os.path.join(pdir, name)) as f:
            for line in f:
                if line.startswith(key):
                    return int(line[len(key):].strip())
    return None


def cpu_baseline(wl, seconds, threads):
    """The oracle (fp32, OpenMP) on a bounded sample of the same workload."""
    import numpy as np
    from oracle import moe_oracle as mo
    mo.set_threads(threads)
    E = wl.E if wl.E <= 16 else 16   # per-token cost depends on k, H, I, S, not E
    k = min(wl.k, E)
    rng = np.random.default_rng(1)

    def normal(shape, std):
        return (rng.standard_normal(shape, dtype=np.float32) * std)

    W = {"router": normal((E, wl.H), wl.w_std), "gate": normal((E, wl.I, wl.H), wl.w_std),
         "up": normal((E, wl.I, wl.H), wl.w_std), "down": normal((E, wl.H, wl.I), wl.w_std)}
    if wl.S:
        W.update(shared_gate=normal((wl.S, wl.H), wl.w_std), shared_up=normal((wl.S, wl.H), wl.w_std),
                 shared_down=normal((wl.H, wl.S), wl.w_std))

    grads = None

    def run(T):
        nonlocal grads
        cfg = mo.make_cfg(T, wl.H, E, k, wl.I, wl.S)
        o = mo.MoeOracle(cfg, 32)
        x = normal((T, wl.H), 1.0)
        dout = normal((T, wl.H), 1.0)
        o.T = T
        if grads is None:
            grads = o.grad_buffers(0.0)   # weight-sized outputs, allocated outside the timing
        grads["x"] = np.empty((T, wl.H), np.float32)
        t0 = time.perf_counter()
        o.forward(x, W["router"], W["gate"], W["up"], W["down"], None, W.get("shared_gate"),
                  W.get("shared_up"), W.get("shared_down"))
        if wl.backward:
            o.backward(dout, d_aux=wl.alpha, d_z=0.0, out=grads)
        return time.perf_counter() - t0

    run(32)                        # warm-up: first touch of weights and thread pool
    t_small = run(64)
    T = int(max(64, min(wl.T, 64 * seconds / max(t_small, 1e-6))))
    t = run(T)
    sample = (f"{T} tokens of the workload shape (H={wl.H}, k={k}, I={wl.I}, S={wl.S}) over "
              f"{E} experts, oracle fp32 {'fwd+bwd' if wl.backward else 'fwd'}, {threads} threads")
    return {"value": round(T / t, 2), "unit": "tokens/s", "cores": threads,
            "kind": "port", "sample": sample, "seconds": round(t, 3)}


def achievable_peaks():
    """Library bf16 GEMMs (hipBLASLt through torch.matmul) at a square shape and
    at the expert / shared-expert shapes of configs 2 and 5, and a plain 1 GiB
    device copy: the achievable ceilings the roofline fractions are read
    against, next to the datasheet peaks."""
    import torch
    dev = torch.device("cuda:0")
    res = {"gemm_bf16_tflops": {}, "peak_bf16_tflops": PEAK_BF16_TFLOPS,
           "peak_hbm_gbs": PEAK_HBM_GBS}
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    shapes = [(8192, 8192, 8192), (16384, 2816, 2048), (16384, 2048, 1408),
              (8192, 5632, 2048), (8192, 2048, 2816), (2048, 4096, 7168)]
    for M, N, K in shapes:
        a = torch.randn(M, K, device=dev, dtype=torch.bfloat16)
        b = torch.randn(N, K, device=dev, dtype=torch.bfloat16)
        for _ in range(3):
            c = a @ b.t()
        torch.cuda.synchronize()
        e0.record()
        for _ in range(20):
            c = a @ b.t()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / 20
        res["gemm_bf16_tflops"][f"{M}x{N}x{K}"] = round(2 * M * N * K / ms / 1e9, 1)
        del a, b, c
    x = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    y = torch.empty_like(x)
    for _ in range(3):
        y.copy_(x)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(10):
        y.copy_(x)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / 10
    res["copy_1GiB_read_plus_write_gbs"] = round(2 * (1 << 30) / ms / 1e6, 1)
    print(json.dumps(res), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", type=int, default=2, choices=[1, 2, 3, 4, 5])
    ap.add_argument("--cpu-baseline", choices=["on", "off"], default="on")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB (5 launches) and exit: the "
                         "reference kernel that scales rocprofv3 FETCH_SIZE / WRITE_SIZE to bytes")
    ap.add_argument("--achievable-peaks", action="store_true",
                    help="only measure this box's achievable peaks (library bf16 GEMMs through "
                         "torch.matmul = hipBLASLt, and a 1 GiB device copy) and exit")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--block", action="store_true",
                    help="time the block's whole MoE sub-block (post_attention_layernorm "
                         "RMSNorm + MoE layer + residual add) through moe_block_forward / "
                         "moe_block_backward")
    ap.add_argument("--recompute", action="store_true",
                    help="keep only the routing state between forward and backward and "
                         "recompute the expert activations in the backward (the plan's "
                         "recompute_activations; activation checkpointing)")
    args = ap.parse_args()
    if args.achievable_peaks:
        achievable_peaks()
        return
    if args.copy_calibration:
        import torch
        n = args.copy_calibration * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes_read": n * 4, "bytes_written": n * 4,
                          "launches": 5}), flush=True)
        return
    if args.gpus != 1:
        print("bench.py measures one MI355X: this build runs the MoE layer on a single GPU "
              "(no expert parallelism); --gpus must be 1", file=sys.stderr)
        sys.exit(2)

    import torch
    from oxidizr_amd.moe import MoeConfig, Plan
    from oxidizr_amd.synth import WORKLOADS, skew_bias

    wl = WORKLOADS[args.config]
    dev = torch.device("cuda:0")
    dtype = torch.float32 if wl.dtype == "f32" else torch.bfloat16
    T, H, E, k, I, S = wl.T, wl.H, wl.E, wl.k, wl.I, wl.S
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    x = gen_weights(torch, (T, H), 1.0, gen, dtype, dev)
    dout = gen_weights(torch, (T, H), 1.0, gen, dtype, dev)
    router = gen_weights(torch, (E, H), wl.w_std, gen, dtype, dev)
    gate = gen_weights(torch, (E, I, H), wl.w_std, gen, dtype, dev)
    up = gen_weights(torch, (E, I, H), wl.w_std, gen, dtype, dev)
    down = gen_weights(torch, (E, H, I), wl.w_std, gen, dtype, dev)
    shared = None
    if S:
        shared = (gen_weights(torch, (S, H), wl.w_std, gen, dtype, dev),
                  gen_weights(torch, (S, H), wl.w_std, gen, dtype, dev),
                  gen_weights(torch, (H, S), wl.w_std, gen, dtype, dev))
    bias, skew_info = skew_bias(wl.T, wl.k, wl.E, wl.skew, x, router)

    cfg = MoeConfig(hidden_size=H, num_experts=E, experts_per_tok=k, intermediate_size=I,
                    shared_expert_enabled=S > 0, shared_intermediate_size=S or None,
                    load_balance_alpha=wl.alpha, router_bias=bias is not None,
                    recompute_activations=bool(args.recompute), fused_block=bool(args.block))
    plan = Plan(cfg, dtype, dev)
    norm_w = (1.0 + 0.1 * torch.randn(H, generator=gen, device=dev)).to(dtype) if args.block else None
    w, _keep_w = plan.weights_struct(router, list(gate.unbind(0)), list(up.unbind(0)),
                                     list(down.unbind(0)), bias, shared)
    out = torch.empty_like(x)
    aux = torch.empty((), dtype=torch.float32, device=dev)
    z = torch.empty((), dtype=torch.float32, device=dev)
    saved = plan.new_saved(T)
    if wl.backward:
        dx = torch.empty_like(x)
        g_router = torch.empty_like(router)
        g_gate, g_up, g_down = torch.empty_like(gate), torch.empty_like(up), torch.empty_like(down)
        g_shared = tuple(torch.empty_like(t) for t in shared) if shared else None
        g, _keep_g = plan.grads_struct(g_router, list(g_gate.unbind(0)), list(g_up.unbind(0)),
                                       list(g_down.unbind(0)), None, g_shared)
        d_aux = torch.tensor(float(wl.alpha), device=dev)   # dL/d aux = load_balance_alpha
        d_z = torch.tensor(0.0, device=dev)                  # z-loss weight 0 in the timed runs
        has_grad = torch.empty(E, dtype=torch.uint8, device=dev)

    if args.block:
        d_norm_w = torch.empty_like(norm_w)

    def fwd(need_grad=True):
        if args.block:  # x is the block input h; out = MoE(RMSNorm(h)) + h
            plan.block_forward(x, norm_w, w, out=out, saved=saved if need_grad else None, aux=aux,
                               z=z, need_grad=need_grad)
        else:
            plan.forward(x, w, out=out, saved=saved if need_grad else None, aux=aux, z=z,
                         need_grad=need_grad)

    def step():
        if wl.backward:
            fwd()
            if args.block:
                plan.block_backward(x, norm_w, dout, w, g, saved, dh=dx, d_norm_w=d_norm_w,
                                    d_aux=d_aux, d_z=d_z, has_grad=has_grad)
            else:
                plan.backward(x, dout, w, g, saved, dx=dx, d_aux=d_aux, d_z=d_z, has_grad=has_grad)
        else:  # forward-only call: no saved state, no gate / up pre-activations
            fwd(need_grad=False)

    dominant = "gateup_fwd"
    fwd()  # realized routing (untimed)
    counts = plan.saved_field(saved, T, "counts").cpu()
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    plan.stage_times(reset=True)
    plan.set_profiling([dominant])
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    dom_ms, dom_calls = plan.stage_times(reset=True)[dominant]
    # per-stage breakdown from a few extra (untimed) steps with every stage
    # evented and the shared expert in serial order (in the timed steps it runs
    # concurrently on the plan's second stream, so stage times there overlap)
    plan.set_shared_overlap(False)
    plan.set_profiling(None)
    for _ in range(3):
        step()
    stages = {n: ms / c for n, (ms, c) in plan.stage_times(reset=True).items() if c}
    plan.set_profiling([])
    plan.set_shared_overlap(True)

    ms_per_step = elapsed * 1e3 / args.steps
    tok_s = T / (elapsed / args.steps)
    TK = T * k
    fwd_flops = 2 * T * H * E + 6 * TK * H * I + 6 * T * H * S
    total_flops = fwd_flops * (3 if wl.backward else 1)
    dom_avg_ms = dom_ms / max(dom_calls, 1)
    n_touched = int((counts > 0).sum())
    if wl.dtype == "f32":
        peak, bound = PEAK_FP32_TFLOPS, "mfma"
    else:
        peak, bound = PEAK_BF16_TFLOPS, "mfma"
    dom_flops = 4 * TK * H * I
    if not wl.backward:  # small-token forward: HBM bound on the expert weights touched
        b = 2
        dom_bytes = n_touched * 2 * H * I * b + TK * H * b + TK * I * b
        roof = {"bound": "hbm", "achieved": round(dom_bytes / (dom_avg_ms * 1e-3) / 1e9, 1),
                "peak": PEAK_HBM_GBS, "unit": "GB/s"}
        roof["frac"] = round(roof["achieved"] / PEAK_HBM_GBS, 4)
        layer_bytes = (n_touched * 3 * H * I * b + E * H * b + 2 * T * H * b + T * E * 4 + TK * 8)
        extra = {"layer_hbm_GBs": round(layer_bytes / (elapsed / args.steps) / 1e9, 1),
                 "layer_hbm_frac": round(layer_bytes / (elapsed / args.steps) / 1e9 / PEAK_HBM_GBS, 4)}
    else:
        ach = dom_flops / (dom_avg_ms * 1e-3) / 1e12
        roof = {"bound": bound, "achieved": round(ach, 1), "peak": peak, "unit": "TFLOP/s",
                "frac": round(ach / peak, 4)}
        iso = dom_flops / (stages[dominant] * 1e-3) / 1e12
        extra = {"dominant_kernel_serial": {"achieved": round(iso, 1), "frac": round(iso / peak, 4),
                                            "ms": round(stages[dominant], 4)}}
    # HBM-side bytes per launch of this kernel and workload, as measured by the
    # rocprofv3 FETCH_SIZE / WRITE_SIZE passes (scaled by a copy kernel) that
    # are summarised under profiles/; null when no such measurement exists.
    roof["traffic"] = measured_traffic(wl.name)
    if wl.dtype == "bf16" and T <= 64:   # small-token path: weight-streaming kernels
        roof["kernel"] = (f"k_skinny_fwd<true, false> (gate/up weight stream + SwiGLU), "
                          f"{dom_avg_ms:.4f} ms/launch")
    else:
        roof["kernel"] = (f"k_gateup_fwd<{'bf16' if wl.dtype == 'bf16' else 'f32'}, true> "
                          f"(grouped gate/up GEMM + SwiGLU), {dom_avg_ms:.4f} ms/launch")

    # memory-bound stages against the HBM roofline: algorithmic bytes per call
    # (b = element size) over the serial stage time of the profiling steps
    b = 2 if wl.dtype == "bf16" else 4
    stage_bytes = {
        "router_gemm": T * H * b + E * H * b + T * E * 4,
        "route": 3 * T * E * 4 + T * 4 + TK * 8,
        "dispatch": 2 * TK * 4 + TK * 8 + 2 * E * 4,
        "gather": T * H * b + TK * H * b + TK * 4,
        "combine_fwd": TK * H * b + (T * H * b if S else 0) + TK * 8 + T * H * b,
    }
    if wl.backward:
        stage_bytes["combine_bwd"] = T * H * b + 2 * TK * H * b + TK * 8 + TK * 4
    hbm_stages = {}
    for name, nbytes in stage_bytes.items():
        if stages.get(name):
            gbs = nbytes / (stages[name] * 1e-3) / 1e9
            hbm_stages[name] = {"GB/s": round(gbs, 1), "frac": round(gbs / PEAK_HBM_GBS, 4)}

    gemm_stages = ("gateup_fwd", "down_fwd", "shared_fwd", "down_dgrad", "down_wgrad",
                   "gateup_dgrad", "gateup_wgrad", "shared_bwd", "router_gemm", "dx")
    gemm_ms = sum(stages.get(s, 0.0) for s in gemm_stages)
    res = {
        "metric": "MoE layer fwd+bwd tokens/sec on 1 MI355X; % bf16 MFMA peak; % HBM peak"
                  if wl.backward else "MoE layer fwd tokens/sec on 1 MI355X; % HBM peak",
        "value": round(tok_s, 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16" if wl.dtype == "bf16" else "f32",
        "data": "synthetic (seeded N(0,1) tokens, N(0,std) random-init weights)",
        "config": {"workload": wl.name, "tokens": T, "hidden": H, "num_experts": E,
                   "experts_per_tok": k, "intermediate": I, "shared_intermediate": S,
                   "load_balance_alpha": wl.alpha, "pass": "fwd+bwd" if wl.backward else "fwd",
                   "parallelism": "single GPU", "routing": wl.skew, **skew_info,
                   "max_expert_tokens": int(counts.max()), "empty_experts": int((counts == 0).sum()),
                   "activations": "recomputed in backward" if args.recompute else "kept",
                   "scope": ("block MoE sub-block: RMSNorm + layer + residual" if args.block
                             else "MoE layer"),
                   "saved_MB_per_layer": round(plan.saved_bytes(T) / 1e6, 1),
                   "workspace_MB": round(plan.workspace_bytes(T) / 1e6, 1)},
        "roofline": roof,
        "layer_tflops": round(total_flops / (elapsed / args.steps) / 1e12, 1),
        "layer_mfma_frac": round(total_flops / (elapsed / args.steps) / 1e12 / peak, 4),
        "gemm_tflops": round(total_flops / (gemm_ms * 1e-3) / 1e12, 1) if gemm_ms else None,
        "stages_ms": {n: round(v, 4) for n, v in stages.items()},
        "hbm_stages": hbm_stages,
        **extra,
    }
    if args.cpu_baseline == "on":
        try:
            threads = min(16, len(os.sched_getaffinity(0)))
        except AttributeError:
            threads = min(16, os.cpu_count() or 1)
        res["cpu_baseline"] = cpu_baseline(wl, args.cpu_seconds, threads)
    else:
        res["cpu_baseline"] = None
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
