"""Benchmark: one MoE FFN layer on one MI355X, BASELINE.json's headline config.

Default workload = configs[1]: GLM-class decode layer, Q2_K routed experts
(H=6144, E=256, I=2048, top-8 sigmoid + bias, x2.5), Q8_0 shared expert,
T=1 bf16 token. A step = one full layer forward (router logits -> top-k ->
dispatch -> routed gate/up/down -> shared expert -> combine + residual) for
one token. Several independent layers are resident in HBM and the steps
cycle through them with a fresh token each, like a decode pass through a
model, so the 256 MB Infinity Cache cannot hold the experts a step reads.

The roofline leg re-runs the same layer steps with the library's event hook
on: HIP events on the layer's stream bracket the dominant kernel (the routed
gate/up dequant-GEMV of the fused decode path) and the routed down kernel.
Algorithmic bytes per gate/up launch = quantised gate+up bytes of the step's
unique selected experts. `traffic` (HBM bytes per launch) comes from the
committed rocprofv3 FETCH_SIZE/WRITE_SIZE summary, scaled by the same
counters read for a plain device copy of known size (--calibrate-copy).

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
QUANT_NAMES = {8: "Q8_0", 10: "Q2_K", 11: "Q3_K", 12: "Q4_K", 14: "Q6_K"}
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
    ap.add_argument("--layers", type=int, default=0,
                    help="resident layer copies (default 8 for decode, 2 for prefill)")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run 10 device copies of 256 MiB (counter calibration)")
    args = ap.parse_args()
    if args.calibrate_copy:
        calibrate_copy()
        return
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
    L = args.layers or (2 if T > 64 or cfg.layers > 1 else 8)
    H, E, I, k = cfg.hidden, cfg.experts, cfg.intermediate, cfg.top_k

    prefill = T > 64
    stacked = cfg.layers > 1
    n_sub = cfg.layers  # MoE layers per step (a stack runs all of the config's layers)
    t0 = time.time()
    units = []  # resident copies: one layer, or one whole stack
    for l in range(L):
        c = cf.Config(**{**cfg.__dict__, "index": cfg.index + 100 * l}) if l else cfg
        if stacked:
            units.append(cf.build_stack(c, dev, max_tokens=T))
        else:
            lt = cf.build_layer(c, 0, dev, max_tokens=T)
            units.append(([lt], None))
        log(f"[bench] built {'stack' if stacked else 'layer'} {l + 1}/{L} ({time.time() - t0:.1f}s)")
    n_inputs = 4 if prefill else 64
    xs = [cf.make_input(cfg, T, variant=v, device=dev) for v in range(n_inputs)]
    hiddens = [x.float() for x in xs] if stacked else None
    if cfg.zipf or cfg.balanced:
        # correction bias fitted so that the top-k load of the first input
        # follows Zipf(s) (s = 0 for the near-uniform workload); written in
        # place (the layer holds its pointer)
        for lts, _ in units:
            lt = lts[0]
            logits = ops.router_logits(xs[0], lt.router)
            lt.bias.copy_(torch.from_numpy(cf.zipf_bias(cfg, logits.cpu().numpy())).to(dev))
        log(f"[bench] Zipf({cfg.zipf}) load bias fitted ({time.time() - t0:.1f}s)")
    residual = torch.randn(T, H, device=dev)
    out = torch.empty(T, H, device=dev)
    ids_buf = [torch.empty(n_sub * T * k, dtype=torch.int32, device=dev) for _ in range(L)]
    w_buf = [torch.empty(T * k, device=dev) for _ in range(L)]
    torch.cuda.synchronize()

    def step(i):
        u = i % L
        lts, stack = units[u]
        if stacked:
            stack.forward(hiddens[i % n_inputs], out=out, ids=ids_buf[u])
        else:
            lts[0].layer.forward(xs[i % n_inputs], residual, out=out, ids=ids_buf[u],
                                 weights=w_buf[u])

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

    # ---- per-kernel times and the dominant kernel ----------------------------
    # Same steps again with the event hook on: the C library brackets each
    # launch of a layer with HIP events on the layer's stream and labels what
    # the launch covered (a stack step makes one launch per layer and timer).
    # Decode: the routed gate/up launch streams the gate+up bytes of the
    # layer's unique selected experts, plus the Q8_0 shared expert's gate+up
    # when the label kind is "tiles"/"ring" (on the "mfma" path the shared
    # gate/up runs in the route launch instead, label kind "route+shared");
    # the down launch streams the routed down bytes plus the shared down when
    # the kind is "down8". Prefill: flops per launch = 2 * (2 * H * I) *
    # assignments (routed only).
    quants = list(cfg.quants)
    gu_per_expert = [2 * I * (H // 256) * ops.block_bytes(q) for q in quants]
    dn_per_expert = [H * (I // 256) * ops.block_bytes(cfg.down_quant or q) for q in quants]
    # shared expert bytes per layer: gate + up, down (Q8_0, or the Laguna XS
    # formats: the shared gate/up format and the routed down format)
    Is = cfg.shared_intermediate
    sq = cfg.shared_quant
    sdq = cfg.shared_down_quant or (sq if sq == cf.Q8_0 else (cfg.down_quant or quants[0]))
    shared_gu = 2 * Is * H // ops.block_values(sq) * ops.block_bytes(sq) if Is else 0
    shared_dn = H * Is // ops.block_values(sdq) * ops.block_bytes(sdq) if Is else 0
    reps = max(args.steps, 64) if not prefill else max(args.steps, 10)
    timers = [ops.TIMER_GATE_UP, ops.TIMER_DOWN, ops.TIMER_ROUTE, ops.TIMER_SELECT]
    uniq = [0] * n_sub
    ops.kernel_timing(True)
    try:
        for tm in timers:
            ops.kernel_timing_read(tm)
        loads = []
        for i in range(reps):
            step(i)
            u = i % L
            for j in range(n_sub):
                uniq[j] += int(torch.unique(ids_buf[u][j * T * k:(j + 1) * T * k]).numel())
            if i < L:
                loads.append(torch.bincount(ids_buf[u][:T * k].long(), minlength=E).cpu())
        torch.cuda.synchronize()
        timed = {tm: ops.kernel_timing_read(tm) for tm in timers}
        labels = {tm: ops.kernel_timing_label(tm) for tm in timers}
    finally:
        ops.kernel_timing(False)
    launches = reps * n_sub
    # the library takes the grouped-GEMM path from 66 assignments on (48 without
    # a shared expert; several
    # tokens per expert), the fused decode launches below; the label says which
    prefill = labels[ops.TIMER_GATE_UP].startswith("prefill")
    if prefill:
        timers = [ops.TIMER_GATE_UP, ops.TIMER_DOWN]
    # one token on the fp8 x fp4 gate/up: the selection (and the shared down)
    # run in the gate/up launch, so there is no select launch
    sel_in_gu = labels[ops.TIMER_GATE_UP].split(":")[0].endswith("+select")
    if sel_in_gu:
        timers = [ops.TIMER_GATE_UP, ops.TIMER_DOWN, ops.TIMER_ROUTE]
    for tm in timers:
        if timed[tm][1] != launches:
            raise RuntimeError(f"kernel timer {tm} saw {timed[tm][1]} launches for {launches}")
    us = {tm: 1e3 * timed[tm][0] / timed[tm][1] for tm in timers}  # per launch
    gu_us, dn_us = us[ops.TIMER_GATE_UP], us[ops.TIMER_DOWN]
    uniq_sub = [u / reps for u in uniq]  # unique experts per step, per layer of the step
    layer_us = ms_per_step * 1e3
    gu_routed = sum(g * u for g, u in zip(gu_per_expert, uniq_sub)) / n_sub  # per launch
    dn_routed = sum(d * u for d, u in zip(dn_per_expert, uniq_sub)) / n_sub
    layer_routed_bytes = (gu_routed + dn_routed) * n_sub
    shared_bytes = n_sub * (shared_gu + shared_dn)
    router_bytes = n_sub * E * H * 4
    extra = {}
    if not prefill:
        kinds = {tm: labels[tm].split(":")[0] for tm in timers}
        # a stack mixes formats: the label is the last layer's, so the shared
        # bytes follow the kind of each layer's launch, read per layer below
        gu_kind, dn_kind = kinds[ops.TIMER_GATE_UP], kinds[ops.TIMER_DOWN]
        rt_kind = kinds[ops.TIMER_ROUTE]
        sl_kind = kinds.get(ops.TIMER_SELECT)
        kernels = {
            "route": {"label": labels[ops.TIMER_ROUTE], "launch_us": us[ops.TIMER_ROUTE],
                      "bytes_per_launch": E * H * 4 + (shared_gu if rt_kind == "route+shared" else 0)},
            "gate_up": {"label": labels[ops.TIMER_GATE_UP], "launch_us": gu_us,
                        "bytes_per_launch": gu_routed
                        + (shared_gu if gu_kind in ("tiles", "ring", "runs+shared+select") else 0)
                        + (shared_dn if gu_kind == "mfma+select" else 0),
                        "routed_bytes_per_launch": gu_routed,
                        "traffic_file": {"mfma": "gate_up_fp4_q2k_c2_decode_traffic.txt",
                                         "mfma+select": "gate_up_sel_fp4_q2k_c2_decode_traffic.txt",
                                         "tiles": "gate_up_q2k_c2_decode_traffic.txt"}.get(gu_kind)},
            "down": {"label": labels[ops.TIMER_DOWN], "launch_us": dn_us,
                     "bytes_per_launch": dn_routed
                     + (shared_dn if dn_kind in ("down8", "runs-down+shared") else 0),
                     "routed_bytes_per_launch": dn_routed,
                     "traffic_file": {"down8": "down8_q2k_c2_decode_traffic.txt",
                                      "mfma-down": "down_mfma_q2k_c2_decode_traffic.txt"}.get(dn_kind)},
        }
        if not sel_in_gu:
            kernels["select"] = {"label": labels[ops.TIMER_SELECT], "launch_us": us[ops.TIMER_SELECT],
                                 "bytes_per_launch": shared_dn if sl_kind == "select+shared-down" else None}
        if stacked:
            for kd in kernels.values():
                kd["label"] = f"{kd['label']} [last of {n_sub} layers; times and bytes averaged per launch]"
        for kd in kernels.values():
            b = kd["bytes_per_launch"]
            kd["launch_us"] = round(kd["launch_us"], 3)
            kd["GBps"] = round(b / (kd["launch_us"] * 1e-6) / 1e9, 1) if b else None
            if b:
                kd["bytes_per_launch"] = int(b)
            if "routed_bytes_per_launch" in kd:
                kd["routed_bytes_per_launch"] = int(kd["routed_bytes_per_launch"])
        # the dominant kernel: the longer of the two expert-streaming launches
        dom = max(("gate_up", "down"), key=lambda n: kernels[n]["launch_us"])
        kd = kernels[dom]
        tf = kd.pop("traffic_file", None)
        for other in kernels.values():
            other.pop("traffic_file", None)
        traffic = read_traffic(ROOT / "profiles" / tf, kd["label"].split(":")[1].split("(")[0].strip()) \
            if tf and cfg.name.startswith("c2_") else None
        # achieved and frac count the routed expert bytes only (the north
        # star's roofline is on the selected experts' quantized bytes); the
        # launch's other bytes (shared expert) are reported beside them
        routed_gbps = round(kd["routed_bytes_per_launch"] / (kd["launch_us"] * 1e-6) / 1e9, 1)
        roofline = {"bound": "hbm", "kernel": kd["label"], "achieved": routed_gbps,
                    "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(routed_gbps / HBM_PEAK_GBS, 4), "traffic": traffic,
                    "launch_us": kd["launch_us"],
                    "routed_bytes_per_launch": kd["routed_bytes_per_launch"],
                    "shared_bytes_per_launch": int(kd["bytes_per_launch"] - kd["routed_bytes_per_launch"]),
                    "all_bytes_per_launch": kd["bytes_per_launch"],
                    "all_bytes_GBps": kd["GBps"]}
        extra["kernels"] = kernels
        if stacked:
            extra["unique_experts_per_layer"] = [round(u, 3) for u in uniq_sub]
    else:
        A = T * k
        gu_flops = 4.0 * H * I * A
        gu_tfs = gu_flops / (gu_us * 1e-6) / 1e12
        dn_tfs = 2.0 * H * I * A / (dn_us * 1e-6) / 1e12
        # the gate/up launch's bound by its arithmetic intensity (flops per
        # algorithmic byte, the expert weights each read once) against the
        # ridge point of the two peaks: c5 (~900 flop/B) is MFMA-bound; c3
        # (~75), c4 at T = 32 and c1 at T = 16 stream their weights (HBM)
        gu_gbps = gu_routed / (gu_us * 1e-6) / 1e9
        intensity = gu_flops / max(gu_routed, 1.0)
        ridge = MFMA_BF16_PEAK_TFLOPS * 1e12 / (HBM_PEAK_GBS * 1e9)
        mfma_frac = round(gu_tfs / MFMA_BF16_PEAK_TFLOPS, 4)
        hbm_frac = round(gu_gbps / HBM_PEAK_GBS, 4)
        if intensity >= ridge:
            roofline = {"bound": "mfma", "achieved": round(gu_tfs, 2), "peak": MFMA_BF16_PEAK_TFLOPS,
                        "unit": "TFLOP/s", "frac": mfma_frac}
        else:
            roofline = {"bound": "hbm", "achieved": round(gu_gbps, 1), "peak": HBM_PEAK_GBS,
                        "unit": "GB/s", "frac": hbm_frac}
        roofline.update({"kernel": labels[ops.TIMER_GATE_UP], "traffic": None,
                         "launch_us": round(gu_us, 3), "flops_per_launch": gu_flops,
                         "routed_bytes_per_launch": int(gu_routed),
                         "flops_per_byte": round(intensity, 1), "ridge_flops_per_byte": round(ridge, 1),
                         "mfma_frac": mfma_frac, "hbm_frac": hbm_frac})
        extra["down_launch"] = {"launch_us": round(dn_us, 3), "TFLOPs": round(dn_tfs, 2)}
        extra["layer_mfma_frac"] = round(6.0 * H * I * A * n_sub / (layer_us * 1e-6) / 1e12
                                         / MFMA_BF16_PEAK_TFLOPS, 4)
        load = torch.stack(loads).float().mean(0)
        extra["expert_load"] = {"active": int((load > 0).sum()), "hottest_share":
                                round(float(load.max() / A), 4),
                                "empty": int((load == 0).sum())}

    # ---- CPU baseline: oracle on the host cores -------------------------
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(cfg, units, xs, residual, T, args.cpu_seconds)

    # arithmetic of the gate/up kernel that ran (decode MFMA: x as two e4m3
    # terms times Q2_K fields as e2m1, down on f16 MFMA; prefill: f16 MFMA;
    # packed-f16 tile kernels otherwise), always fp32 accumulation
    gu_label = labels[ops.TIMER_GATE_UP]
    dn_label = labels[ops.TIMER_DOWN]
    dn_mfma = dn_label.startswith(("mfma-down", "runs-down", "runs-multi-down", "prefill"))
    down_t = "f16 MFMA down" if dn_mfma else "f16-dot2 down"
    if gu_label.startswith("mfma"):
        dtype = f"e4m3x2*e2m1 MFMA gate/up, {down_t}, f32 acc"
    elif gu_label.startswith("runs") and cfg.x_dtype == torch.float32:
        dtype = f"f16x2-term MFMA gate/up (fp32 x), {down_t}, f32 acc"
    elif gu_label.startswith("runs"):
        dtype = f"f16 MFMA gate/up, {down_t}, f32 acc"
    elif gu_label.startswith("prefill"):
        dtype = "f16 MFMA, f32 acc"
    else:
        dtype = "f16-dot2/f32-acc"

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
        "dtype": dtype,
        "data": "synthetic (seeded N(0,1) activations, N(0,0.02) weights quantised on device)",
        "config": {"workload": cfg.name, "tokens": T, "hidden": H, "experts": E,
                   "intermediate": I, "top_k": k, "quant": QUANT_NAMES.get(quants[0], str(quants[0])),
                   "shared_intermediate": cfg.shared_intermediate,
                   "layers_per_step": n_sub, "quants": [QUANT_NAMES.get(x, str(x)) for x in quants],
                   "rms_norm_eps": cfg.rms_eps if stacked else None,
                   "copies_resident": L},
        "us_per_token": round(layer_us / T, 3),
        "us_per_token_per_layer": round(layer_us / T / n_sub, 3),
        "layer_routed_bytes": int(layer_routed_bytes),
        "layer_routed_GBps": round(layer_routed_bytes / (layer_us * 1e-6) / 1e9, 1),
        "layer_total_bytes": int(layer_routed_bytes + shared_bytes + router_bytes),
        "layer_total_GBps": round((layer_routed_bytes + shared_bytes + router_bytes)
                                  / (layer_us * 1e-6) / 1e9, 1),
        "roofline": roofline,
        **extra,
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)


def calibrate_copy():
    """10 plain device-to-device copies of 256 MiB: the HBM counters of a
    copy kernel of known size (256 MiB read + 256 MiB written per launch)."""
    import torch
    n = 256 << 20
    src = torch.empty(n, dtype=torch.uint8, device="cuda:0").fill_(7)
    dst = torch.empty_like(src)
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calibrate_copy_bytes": n, "launches": 10}), flush=True)


def read_traffic(path, kernel):
    """HBM bytes per launch of the roofline kernel, from the committed
    rocprofv3 FETCH_SIZE/WRITE_SIZE summary; null when the file is absent or
    was measured on another kernel (its "kernel:" line must name `kernel`)."""
    try:
        text = Path(path).read_text().splitlines()
    except OSError:
        return None
    named = [l.split(":", 1)[1].strip() for l in text if l.startswith("kernel:")]
    if not named or named[0] != kernel:
        return None
    for line in text:
        if line.startswith("traffic_bytes_per_launch:"):
            return int(float(line.split(":", 1)[1]))
    return None


def cpu_baseline(cfg, units, xs, residual, T, seconds):
    """Times the C++ oracle on a bounded sample of the workload's tokens:
    decode one token per step, prefill chunks of 4 consecutive tokens of the
    batch, cycling the resident copies; a stack step runs every layer (RMSNorm,
    bf16 rounding, router, routed and shared experts). Only the oracle calls
    are timed; copying the selected experts' bytes to the host is not."""
    import numpy as np
    import torch

    sys.path.insert(0, str(ROOT / "tests"))
    import oracle_lib as orc  # test-infrastructure checker, used here only as the CPU baseline
    import parity_helpers as ph

    try:
        host_cores = len(os.sched_getaffinity(0))
    except AttributeError:
        host_cores = os.cpu_count() or 1
    threads = max(1, min(host_cores, 16))
    orc.THREADS = threads
    k, E = cfg.top_k, cfg.experts
    chunk = 1 if T <= 64 else 4
    stacked = cfg.layers > 1
    busy, n = 0.0, 0
    while busy < seconds and n < 2048:
        lts, _ = units[n % len(units)]
        j = (n * chunk) % T
        x = xs[n % len(xs)][j:j + chunk].float().cpu().numpy()
        r = x.copy() if stacked else residual[j:j + chunk].cpu().numpy()
        for lt in lts:
            router = lt.router.cpu().numpy()
            bias = None if lt.bias is None else lt.bias.cpu().numpy()
            t0 = time.perf_counter()
            if stacked:
                x = orc.rms_norm(r, lt.norm_w.cpu().numpy(), cfg.rms_eps)
                if cfg.x_dtype == torch.bfloat16:
                    x = ph.bf16_round(x)
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
            t0 = time.perf_counter()
            routed = orc.moe_routed(lt.quant, lt.down_quant or lt.quant, g, u, d, x, ids_c, w,
                                    len(experts), k, cfg.intermediate)
            if shared:
                r = orc.shared_ffn(lt.shared_quant, lt.shared_down_quant, *shared, x,
                                   cfg.shared_intermediate, routed=routed, residual=r)
            else:
                r = routed + r
            busy += time.perf_counter() - t0
        n += 1
    what = ("decode tokens (T=1 forwards" if chunk == 1 else
            f"prefill tokens (forwards over chunks of {chunk} tokens")
    what += f" of all {cfg.layers} layers with RMSNorm" if stacked else " of the layer"
    return {"value": round(n * chunk / busy, 4), "unit": "tokens/s", "cores": threads,
            "host_cores": host_cores, "kind": "port",
            "threads_note": "oracle worker threads = min(host cores in this process's "
                            "affinity, 16); threads are spawned per oracle call",
            "sample": f"{n * chunk} {what}, incl. router, routed experts and shared expert) "
                      f"in {busy:.1f}s of oracle time"}


if __name__ == "__main__":
    main()
