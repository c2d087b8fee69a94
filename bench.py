"""Benchmark: one MoE FFN layer on one MI355X, BASELINE.json's headline config.

Default workload = configs[1]: GLM-class decode layer, Q2_K routed experts
(H=6144, E=256, I=2048, top-8 sigmoid + bias, x2.5), Q8_0 shared expert,
T=1 bf16 token. A step = one full layer forward (router logits -> top-k ->
dispatch -> routed gate/up/down -> shared expert -> combine + residual) for
one token. Several independent layers are resident in HBM and the steps
cycle through them with a fresh token each, like a decode pass through a
model, so the 256 MB Infinity Cache cannot hold the experts a step reads.

The roofline leg times the dominant kernel (routed gate/up dequant-GEMV)
alone with HIP events on the stream it runs on; its algorithmic bytes are
the quantised gate+up bytes of the selected (unique) experts.

The cpu_baseline leg times the CPU oracle (test infrastructure, C++,
multithreaded) on a bounded sample of the same decode workload.
"""
import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="c2")
    ap.add_argument("--tokens", type=int, default=0, help="T (default: the config's first)")
    ap.add_argument("--layers", type=int, default=8, help="resident layer copies")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 "
                                   "(multi-GPU expert parallelism is design-only)"}))
        sys.exit(2)

    import numpy as np
    import torch

    from inferno_amd import configs as cf
    from inferno_amd import lib, ops

    lib()
    dev = torch.device("cuda:0")
    cfg = cf.CONFIGS[args.config]
    T = args.tokens or cfg.tokens[0]
    L = max(1, args.layers)
    H, E, I, k = cfg.hidden, cfg.experts, cfg.intermediate, cfg.top_k

    t0 = time.time()
    layers = []
    for l in range(L):
        c = cf.Config(**{**cfg.__dict__, "index": cfg.index + 100 * l}) if l else cfg
        layers.append(cf.build_layer(c, 0, dev, max_tokens=T))
        log(f"[bench] built layer {l + 1}/{L} ({time.time() - t0:.1f}s)")
    n_inputs = 64
    xs = [cf.make_input(cfg, T, variant=v, device=dev) for v in range(n_inputs)]
    residual = torch.randn(T, H, device=dev)
    out = torch.empty(T, H, device=dev)
    ids_buf = [torch.empty(T * k, dtype=torch.int32, device=dev) for _ in range(L)]
    w_buf = [torch.empty(T * k, device=dev) for _ in range(L)]
    torch.cuda.synchronize()

    def step(i):
        l = i % L
        layers[l].layer.forward(xs[i % n_inputs], residual, out=out, ids=ids_buf[l],
                                weights=w_buf[l])

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    t_start = time.perf_counter()
    for i in range(args.steps):
        step(args.warmup + i)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t_start
    ms_per_step = 1e3 * elapsed / args.steps
    tokens_per_s = T * args.steps / elapsed

    # ---- dominant kernel alone: routed gate/up dequant-GEMV -------------
    q = cfg.quants[0]
    bb = ops.block_bytes(q)
    gu_bytes_per_expert = 2 * I * (H // 256) * bb
    expert_bytes = gu_bytes_per_expert + H * (I // 256) * bb
    plans = []
    for j in range(n_inputs):
        l = j % L
        lt = layers[l]
        logits = ops.router_logits(xs[j], lt.router)
        ids, w, _ = ops.router_topk(logits, lt.bias, k, cfg.score_fn, cfg.norm, cfg.scale)
        off, srt, act = ops.dispatch(ids, T, k, E)
        plans.append((lt, xs[j], off, srt, act, w, int(torch.unique(ids).numel())))
    h_out = torch.empty(T * k, I, device=dev)
    gws = ops.gemv_workspace(T, H, dev)
    reps = max(args.steps, 64)
    for j in range(8):
        lt, x, off, srt, act, w, _ = plans[j]
        ops.expert_gate_up_swiglu(q, lt.gate, lt.up, x, off, srt, act, w, k, E, I, out=h_out,
                                  ws=gws)
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    uniq = 0
    for j in range(reps):
        lt, x, off, srt, act, w, nu = plans[j % n_inputs]
        ops.expert_gate_up_swiglu(q, lt.gate, lt.up, x, off, srt, act, w, k, E, I, out=h_out,
                                  ws=gws)
        uniq += nu
    ev1.record()
    torch.cuda.synchronize()
    gu_us = 1e3 * ev0.elapsed_time(ev1) / reps
    gu_bytes = gu_bytes_per_expert * uniq / reps
    gu_gbs = gu_bytes / (gu_us * 1e-6) / 1e9

    # whole-layer algorithmic bytes (routed experts of the step's unique experts)
    uniq_layer = np.mean([p[6] for p in plans])
    layer_routed_bytes = expert_bytes * uniq_layer
    layer_us = ms_per_step * 1e3

    # ---- CPU baseline: oracle on the host cores -------------------------
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(cfg, layers, xs, residual, T, args.cpu_seconds)

    result = {
        "metric": "MoE-layer decode us/token + HBM GB/s (% of 8 TB/s); prefill tokens/s, MFMA %",
        "value": round(tokens_per_s, 3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded N(0,1) activations, N(0,0.02) weights quantised on device)",
        "config": {"workload": cfg.name, "tokens": T, "hidden": H, "experts": E,
                   "intermediate": I, "top_k": k, "quant": "Q2_K" if q == 10 else str(q),
                   "shared_intermediate": cfg.shared_intermediate, "layers_resident": L},
        "us_per_token": round(layer_us / T, 3),
        "layer_routed_bytes": int(layer_routed_bytes),
        "layer_routed_GBps": round(layer_routed_bytes / (layer_us * 1e-6) / 1e9, 1),
        "roofline": {"bound": "hbm", "kernel": "gemv_kernel<gate_up routed>",
                     "achieved": round(gu_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gu_gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "launch_us": round(gu_us, 3), "bytes_per_launch": int(gu_bytes)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)


def cpu_baseline(cfg, layers, xs, residual, T, seconds):
    """Times the C++ oracle on a bounded sample of decode tokens (one layer
    each, cycling layers). Only the oracle calls are timed; copying the
    selected experts' bytes to the host is not."""
    import numpy as np
    import torch

    sys.path.insert(0, str(ROOT / "tests"))
    import oracle_lib as orc  # test-infrastructure checker, used here only as the CPU baseline

    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count() or 1
    cores = max(1, min(cores, 16))
    orc.THREADS = cores
    k, E = cfg.top_k, cfg.experts
    busy, n = 0.0, 0
    while busy < seconds and n < 256:
        lt = layers[n % len(layers)]
        x = xs[n % len(xs)][:1].float().cpu().numpy()
        router = lt.router.cpu().numpy()
        bias = None if lt.bias is None else lt.bias.cpu().numpy()
        t0 = time.perf_counter()
        logits = orc.linear(x, router)
        ids, w = orc.router_topk(logits, bias, k, cfg.score_fn, cfg.norm, cfg.scale)
        busy += time.perf_counter() - t0
        experts = np.unique(ids)
        sel = torch.as_tensor(experts.astype(np.int64), device=lt.gate.device)
        g = lt.gate.view(E, -1)[sel].cpu().numpy().reshape(-1)
        u = lt.up.view(E, -1)[sel].cpu().numpy().reshape(-1)
        d = lt.down.view(E, -1)[sel].cpu().numpy().reshape(-1)
        remap = {int(e): i for i, e in enumerate(experts)}
        ids_c = np.array([remap[int(e)] for e in ids], np.uint32)
        shared = [s.cpu().numpy() for s in lt.shared] if lt.shared else None
        res = residual[:1].cpu().numpy()
        t0 = time.perf_counter()
        routed = orc.moe_routed(lt.quant, lt.quant, g, u, d, x, ids_c, w, len(experts), k,
                                cfg.intermediate)
        if shared:
            orc.shared_q8_0(*shared, x, cfg.shared_intermediate, routed=routed, residual=res)
        busy += time.perf_counter() - t0
        n += 1
    return {"value": round(n / busy, 4), "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"{n} decode tokens (T=1 layer forwards incl. router, routed experts and "
                      f"shared expert) in {busy:.1f}s of oracle time"}


if __name__ == "__main__":
    main()
