#!/usr/bin/env python3
"""MoE layer forward + backward throughput on one MI355X.

One step = one forward and one backward pass of the MoE layer over one batch of
synthetic tokens (every gradient written). Default workload: BASELINE config 5,
the largest configuration (T=8192, H=7168, E=256, top-8, I=2048, shared 2048,
bf16, lognormal expert loads). Prints ONE JSON line. Other BASELINE configs:
--config {1,2,3,4}.

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


def measured_traffic(workload, stage):
    """HBM-side bytes per launch of one stage's kernel recorded in
    profiles/*.md ("traffic_bytes_per_launch <workload> <stage>: <bytes>"), or
    None."""
    pdir = os.path.join(ROOT, "profiles")
    if not os.path.isdir(pdir):
        return None
    key = f"traffic_bytes_per_launch {workload} {stage}:"
    for name in sorted(os.listdir(pdir)):
        if not name.endswith((".md", ".txt")):
            continue
        with open(os.path.join(pdir, name)) as f:
            for line in f:
                if line.startswith(key):
                    return int(line[len(key):].strip())
    return None


def cpu_baseline(wl, seconds, threads):
    """The oracle (fp32, OpenMP) on a bounded sample of the same workload: the
    workload's H, E, k, I and S, its weight-gradient writes included, over a
    token sample sized to take about `seconds`. With more than 16 experts the
    expert weights are 16 distinct random sets repeated over the E experts (the
    arithmetic and memory traffic are those of E separate experts; generating
    E distinct sets would take minutes); if the host cannot hold the E
    experts' weights and gradients, the sample falls back to 16 experts."""
    import numpy as np
    from oracle import moe_oracle as mo
    mo.set_threads(threads)
    E = wl.E
    need = 2 * 3 * E * wl.I * wl.H * 4 + (2 * 3 * wl.S * wl.H * 4 if wl.S else 0)
    try:
        import psutil
        avail = psutil.virtual_memory().available
    except Exception:  # noqa: BLE001 - psutil missing: assume the small sample
        avail = 0
    if E > 16 and avail < 1.5 * need:
        E = 16
    k = min(wl.k, E)
    rng = np.random.default_rng(1)

    def normal(shape, std):
        return (rng.standard_normal(shape, dtype=np.float32) * std)

    def experts(shape):
        base = normal((min(E, 16),) + shape, wl.w_std)
        return base if E <= 16 else np.tile(base, (E // 16 + 1, 1, 1))[:E].copy()

    W = {"router": normal((E, wl.H), wl.w_std), "gate": experts((wl.I, wl.H)),
         "up": experts((wl.I, wl.H)), "down": experts((wl.H, wl.I))}
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
    # a call costs a fixed part (weight gradients written once) plus a part per
    # token: fit both from two small calls, then size the sample
    t1, t2 = run(64), run(256)
    per_tok = max((t2 - t1) / 192, 1e-7)
    fixed = max(t1 - 64 * per_tok, 0.0)
    T = int(max(256, min(wl.T, (seconds - fixed) / per_tok)))
    t = run(T)
    sample = (f"{T} tokens of the workload shape (H={wl.H}, E={E}, k={k}, I={wl.I}, S={wl.S}"
              f"{'; 16 distinct weight sets over the experts' if E > 16 else ''}), oracle fp32 "
              f"{'fwd+bwd with every weight gradient written' if wl.backward else 'fwd'}, "
              f"{threads} threads")
    return {"value": round(T / t, 2), "unit": "tokens/s", "cores": threads,
            "kind": "port", "sample": sample, "seconds": round(t, 3)}


def dropin_step(torch, cfg, dtype, dev, x, dout, router, gate, up, down, bias, shared, d_aux,
                steps):
    """The same forward + backward through the drop-in autograd module
    (oxidizr_amd.moe.MoeLayer: torch autograd, fresh gradient tensors on every
    call, parameters as separate tensors) on copies of the same weights and
    inputs.  Reported beside the direct C-ABI step, which reuses its buffers."""
    from oxidizr_amd.moe import MoeLayer
    layer = MoeLayer(cfg, dtype=dtype, device=dev)
    with torch.no_grad():
        layer.router.gate.weight.copy_(router)
        if bias is not None:
            layer.router.bias.copy_(bias)
        for e, ex in enumerate(layer.experts):
            ex.gate_proj.weight.copy_(gate[e])
            ex.up_proj.weight.copy_(up[e])
            ex.down_proj.weight.copy_(down[e])
        if shared:
            for mod, t in zip((layer.shared_expert.gate_proj, layer.shared_expert.up_proj,
                               layer.shared_expert.down_proj), shared):
                mod.weight.copy_(t)
    params = [prm for _, prm in layer.trainable_parameters()]
    x3 = x.detach().reshape(1, *x.shape).clone().requires_grad_()
    dout3 = dout.reshape(1, *dout.shape)
    da = torch.tensor(float(d_aux), device=dev)
    dz = torch.tensor(0.0, device=dev)

    def one():
        for prm in params:
            prm.grad = None
        x3.grad = None
        out, aux, z = layer(x3)
        torch.autograd.backward([out, aux, z], [dout3, da, dz])

    for _ in range(2):
        one()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        one()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    del layer, params, x3
    torch.cuda.empty_cache()
    return {"ms_per_step": round(ms, 4), "tokens_per_s": round(x.shape[0] / (ms * 1e-3), 1),
            "steps": steps, "path": "oxidizr_amd.moe.MoeLayer forward + torch.autograd.backward"}


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


def measure(args, config, steps, warmup, extras=True):
    """One workload: warm-up steps, then `steps` timed steps, plus the
    per-stage breakdown; returns the result dict (without cpu_baseline).
    extras: also the drop-in autograd timing."""
    import torch
    from oxidizr_amd.moe import MoeConfig, Plan
    from oxidizr_amd.synth import WORKLOADS, skew_bias

    wl = WORKLOADS[config]
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

    fwd()  # realized routing (untimed)
    counts = plan.saved_field(saved, T, "counts").cpu()
    n_touched = int((counts > 0).sum())
    b = 2 if wl.dtype == "bf16" else 4
    TK = T * k
    # Algorithmic work of the single-kernel GEMM stages: flops, and HBM bytes
    # (operands read once, outputs written once; weights of the experts that
    # received tokens).
    gemm_work = {
        # the token operands of the gate/up forward and of the down input
        # gradient are x and d_out read through the permutation: T rows
        "gateup_fwd": (4 * TK * H * I, T * H * b + 2 * n_touched * I * H * b + 3 * TK * I * b),
        "down_fwd": (2 * TK * I * H, TK * I * b + n_touched * H * I * b + TK * H * b),
        "down_dgrad": (2 * TK * H * I, T * H * b + n_touched * H * I * b + 4 * TK * I * b),
        "gateup_dgrad": (4 * TK * I * H, 2 * TK * I * b + 2 * n_touched * I * H * b + TK * H * b),
        "down_wgrad": (2 * TK * H * I, TK * H * b + TK * I * b + n_touched * H * I * b),
        "gateup_wgrad": (4 * TK * H * I, 2 * TK * I * b + TK * H * b + 2 * n_touched * I * H * b),
    }
    kernel_of = {
        "gateup_fwd": f"k_gateup_fwd<{wl.dtype}, true> (grouped gate/up GEMM + SwiGLU)",
        "down_fwd": f"k_down_fwd<{wl.dtype}, true> (grouped down projection)",
        "down_dgrad": f"k_down_dgrad<{wl.dtype}, true> (grouped input gradient of down + SwiGLU backward)",
        "gateup_dgrad": f"k_gateup_dgrad<{wl.dtype}, true> (grouped input gradient of gate/up)",
        "down_wgrad": f"k_wgrad<{wl.dtype}, 1, true> (grouped down weight gradient)",
        "gateup_wgrad": f"k_wgrad<{wl.dtype}, 2, true> (grouped gate/up weight gradient)",
    }
    peak_mfma = PEAK_FP32_TFLOPS if wl.dtype == "f32" else PEAK_BF16_TFLOPS
    ridge = peak_mfma * 1e12 / (PEAK_HBM_GBS * 1e9)   # flop per HBM byte
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    if wl.backward:
        # The dominant kernel is the one with the largest share of the step's
        # GPU work: the longest stage when every stage runs alone (serial
        # order, every stage evented, three untimed steps). In the overlapped
        # steps a kernel's duration also holds the time other streams' kernels
        # share the CUs with it (per-kernel durations summed over streams count
        # that time twice), so those in-situ times are reported beside it.
        plan.set_shared_overlap(False)
        plan.stage_times(reset=True)
        plan.set_profiling(list(gemm_work))
        for _ in range(3):
            step()
        # per step: a stage may be recorded more than once per step (the
        # dispatch: k_scan and the scatter)
        alone = {n: ms / 3 for n, (ms, c) in plan.stage_times(reset=True).items() if c}
        plan.set_shared_overlap(True)
        for _ in range(2):
            step()
        insitu = {n: ms / 2 for n, (ms, c) in plan.stage_times(reset=True).items() if c}
        dominant = max((n for n in gemm_work if n in alone), key=lambda n: alone[n])
    else:  # forward-only small-token path: the gate/up weight stream
        dominant = "gateup_fwd"
    plan.set_profiling([])
    torch.cuda.synchronize()
    plan.stage_times(reset=True)
    plan.set_profiling([dominant])
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
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
    stages = {n: ms / 3 for n, (ms, c) in plan.stage_times(reset=True).items() if c}
    plan.set_profiling([])
    plan.set_shared_overlap(True)

    ms_per_step = elapsed * 1e3 / steps
    tok_s = T / (elapsed / steps)
    fwd_flops = 2 * T * H * E + 6 * TK * H * I + 6 * T * H * S
    total_flops = fwd_flops * (3 if wl.backward else 1)
    dom_avg_ms = dom_ms / max(dom_calls, 1)
    peak = peak_mfma
    extra = {}
    if not wl.backward:  # small-token forward: HBM bound on the expert weights touched
        dom_bytes = n_touched * 2 * H * I * b + TK * H * b + TK * I * b
        roof = {"bound": "hbm", "achieved": round(dom_bytes / (dom_avg_ms * 1e-3) / 1e9, 1),
                "peak": PEAK_HBM_GBS, "unit": "GB/s"}
        roof["frac"] = round(roof["achieved"] / PEAK_HBM_GBS, 4)
        layer_bytes = (n_touched * 3 * H * I * b + E * H * b + 2 * T * H * b + T * E * 4 + TK * 8)
        extra = {"layer_hbm_GBs": round(layer_bytes / (elapsed / steps) / 1e9, 1),
                 "layer_hbm_frac": round(layer_bytes / (elapsed / steps) / 1e9 / PEAK_HBM_GBS, 4)}
        roof["kernel"] = (f"k_skinny_fwd<true, false> (gate/up weight stream + SwiGLU), "
                          f"{dom_avg_ms:.4f} ms/launch")
    else:
        flops, nbytes = gemm_work[dominant]
        tflops = flops / (dom_avg_ms * 1e-3) / 1e12
        gbs = nbytes / (dom_avg_ms * 1e-3) / 1e9
        mfma_side = {"achieved": round(tflops, 1), "peak": peak, "unit": "TFLOP/s",
                     "frac": round(tflops / peak, 4)}
        hbm_side = {"achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                    "frac": round(gbs / PEAK_HBM_GBS, 4)}
        # the roof that binds: HBM below the ridge intensity, MFMA above it
        intensity = flops / nbytes
        if intensity < ridge:
            roof = {"bound": "hbm", **hbm_side}
            extra["roofline_mfma_side"] = mfma_side
        else:
            roof = {"bound": "mfma", **mfma_side}
            extra["roofline_hbm_side"] = hbm_side
        roof["kernel"] = (f"{kernel_of[dominant]}, {dom_avg_ms:.4f} ms/launch in the timed "
                          f"(overlapped) steps")
        roof["stage"] = dominant
        roof["flop_per_launch"] = flops
        roof["bytes_per_launch"] = nbytes
        roof["intensity_flop_per_byte"] = round(intensity, 1)
        iso_ms = stages[dominant]
        extra["dominant_kernel_serial"] = {"ms": round(iso_ms, 4),
                                           "TFLOP/s": round(flops / (iso_ms * 1e-3) / 1e12, 1),
                                           "GB/s": round(nbytes / (iso_ms * 1e-3) / 1e9, 1)}
        extra["insitu_stage_ms"] = {n: round(v, 4) for n, v in insitu.items()}
        extra["alone_stage_ms"] = {n: round(v, 4) for n, v in alone.items()}
    # HBM-side bytes per launch of this kernel and workload, as measured by the
    # rocprofv3 FETCH_SIZE / WRITE_SIZE passes (scaled by a copy kernel) that
    # are summarised under profiles/; null when no such measurement exists.
    roof["traffic"] = measured_traffic(wl.name, dominant)

    # memory-bound stages against the HBM roofline: algorithmic bytes per call
    # (b = element size) over the serial stage time of the profiling steps
    stage_bytes = {
        "router_gemm": T * H * b + E * H * b + T * E * 4,
        "route": 3 * T * E * 4 + T * 4 + TK * 8,
        "dispatch": 2 * TK * 4 + TK * 8 + 2 * E * 4,
        "combine_fwd": TK * H * b + (T * H * b if S else 0) + TK * 8 + T * H * b,
    }
    if wl.backward:
        # the backward's weighted token rows (x read once, T*k rows written,
        # inv_perm and weights read); the forward keeps no permuted copy
        stage_bytes["gather"] = T * H * b + TK * H * b + TK * 8
        # weighted d_out rows for the down weight gradient
        stage_bytes["combine_bwd"] = T * H * b + TK * H * b + TK * 8
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
        "value": round(tok_s, 1), "unit": "tokens/s", "n_gpus": 1, "steps": steps,
        "warmup": warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True,
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
        "layer_tflops": round(total_flops / (elapsed / steps) / 1e12, 1),
        "layer_mfma_frac": round(total_flops / (elapsed / steps) / 1e12 / peak, 4),
        "gemm_tflops": round(total_flops / (gemm_ms * 1e-3) / 1e12, 1) if gemm_ms else None,
        "stages_ms": {n: round(v, 4) for n, v in stages.items()},
        "hbm_stages": hbm_stages,
        **extra,
    }
    if extras and wl.backward and not args.block and not args.recompute and args.dropin == "on":
        res["dropin_autograd"] = dropin_step(torch, cfg, dtype, dev, x, dout, router, gate, up,
                                             down, bias, shared, wl.alpha, min(steps, 10))
    del plan, saved
    return res, wl


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", type=int, default=5, choices=[1, 2, 3, 4, 5])
    ap.add_argument("--cpu-baseline", choices=["on", "off"], default="on")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB (5 launches) and exit: the "
                         "reference kernel that scales rocprofv3 FETCH_SIZE / WRITE_SIZE to bytes")
    ap.add_argument("--achievable-peaks", action="store_true",
                    help="only measure this box's achievable peaks (library bf16 GEMMs through "
                         "torch.matmul = hipBLASLt, and a 1 GiB device copy) and exit")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--block", action="store_true",
                    help="time the block's whole MoE sub-block (post_attention_layernorm "
                         "RMSNorm + MoE layer + residual add) through moe_block_forward / "
                         "moe_block_backward")
    ap.add_argument("--dropin", choices=["on", "off"], default="on",
                    help="also time the step through the drop-in autograd module "
                         "(MoeLayer) on the same weights; reported as dropin_autograd")
    ap.add_argument("--per-config", choices=["on", "off"], default="on",
                    help="after the config-5 line, also run configs 2, 3 and 4 for 10 steps "
                         "each and report them under per_config")
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

    res, wl = measure(args, args.config, args.steps, args.warmup)
    if args.per_config == "on" and args.config == 5 and not args.block and not args.recompute:
        # the other north-star targets (configs 2, 3: layer MFMA fraction; 4:
        # small-token forward against HBM), a few steps each, after the headline
        import torch
        torch.cuda.empty_cache()
        res["per_config"] = {}
        for c in (2, 3, 4):
            sub, swl = measure(args, c, 10, 3, extras=False)
            torch.cuda.empty_cache()
            entry = {"ms_per_step": sub["ms_per_step"], "tokens_per_s": sub["value"],
                     "steps": sub["steps"], "roofline": sub["roofline"]}
            if swl.backward:
                entry.update(layer_tflops=sub["layer_tflops"],
                             layer_mfma_frac=sub["layer_mfma_frac"],
                             alone_stage_ms=sub.get("alone_stage_ms"))
            else:
                entry.update(layer_hbm_GBs=sub["layer_hbm_GBs"],
                             layer_hbm_frac=sub["layer_hbm_frac"])
            res["per_config"][swl.name] = entry
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
