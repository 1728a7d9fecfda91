"""Benchmark of the MI355X MoE FFN block (one GPU).

Default workload: BASELINE.json config 2. That is a decode batch of 16 independent tokens
through one sparse-MoE block of LFM2.5-8B-A1B's shape (hidden 2048, expert FFN 1792, 32
experts, top-4, Q4_K experts with Q8 activations). A step is one pass of the hot path over one
batch: router, gating, dispatch, gate/up + SwiGLU, down + combine.

The 256 MB Infinity Cache would hold one layer's 198 MB of experts, so step i runs layer
i mod L of L independently generated layers (L = 12 by default, 2.4 GB), as successive layers
of a real model would. Inputs are resident in HBM before the timed region.

The output is one JSON line with `value` in tok/s. It also carries:
  roofline      the dominant kernel's algorithmic bytes per launch divided by its mean launch
                time, measured with HIP events on the stream it runs on
  cpu_baseline  the reference path (its C++ restatement, OpenMP over output rows as the
                reference's rayon does) timed on this host on a bounded sample
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0
BF16_PEAK_TFLOPS = 2500.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", type=int, default=2, choices=[1, 2, 3, 4, 5])
    ap.add_argument("--layers", type=int, default=12, help="distinct weight sets rotated across steps")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="bound on the CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    return ap.parse_args()


def algorithmic_bytes(w, counts, T):
    """Per-kernel and per-step algorithmic bytes for one MoE layer (no intermediates/re-reads)."""
    from bebelm_amd import synth

    H, F, K = w.hidden, w.moe_ff, w.n_used
    u_hit = int(np.count_nonzero(counts))
    gu = synth.byte_size(w.gate_dtype, H * F) + synth.byte_size(w.up_dtype, H * F)
    dn = synth.byte_size(w.down_dtype, F * H)
    q8 = lambda n: n + n // 256 * 4 + n // 32 * 4  # noqa: E731
    gateup = u_hit * gu + T * q8(H) + T * K * (F * 4 + q8(F))      # weights + x_q8 in, act (+q8) out
    down = u_hit * dn + T * K * q8(F) + T * H * 4 + T * K * H * 4  # weights + act_q8 in, out + slots
    route = w.router.nbytes + T * H * 4 + T * q8(H)
    step = u_hit * (gu + dn) + w.router.nbytes + T * H * 4 * 2      # SURVEY 8(d) block figure
    return {"gateup_swiglu": gateup, "down_combine": down, "route_small": route, "step": step, "u_hit": u_hit}


def cpu_baseline(layers, x, T, seconds):
    from oracle import bbo

    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count() or 1
    cores = min(cores, int(os.environ.get("OMP_NUM_THREADS", cores)))
    bbo.set_threads(cores)
    xs = x.reshape(-1)
    calls = 0
    t0 = time.perf_counter()
    while True:
        w = layers[calls % len(layers)]
        if T == 1:
            bbo.moe_ffn(w, xs)
        else:
            bbo.moe_ffn_batch(w, xs, T)
        calls += 1
        el = time.perf_counter() - t0
        if el >= seconds or calls >= 1000:
            break
    return {"value": calls * T / el, "unit": "tok/s", "cores": cores, "kind": "port",
            "sample": f"{calls} calls of the C++ restatement of moe_ffn{'_batch' if T > 1 else ''} "
                      f"(T={T}, {len(layers)} rotated layers) in {el:.1f} s, OpenMP over output rows"}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only; --gpus {args.gpus} is not supported by this build", file=sys.stderr)
        sys.exit(2)
    import torch

    from bebelm_amd import synth
    from bebelm_amd.model import Context, MoeLayer, RouteTrace

    cfg = synth.CONFIGS[args.config]
    if args.config == 5:
        print("config 5 is measured by bench_stack in DESIGN notes; use --config 1..4 here", file=sys.stderr)
        sys.exit(2)
    T = cfg.tokens
    L = max(1, args.layers)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    ctx = Context(0)
    ctx.set_stream(torch.cuda.current_stream().cuda_stream)

    t_gen = time.perf_counter()
    weights = [synth.config_layer(args.config, seed=args.seed, layer=l) for l in range(L)]
    layers = [MoeLayer(ctx, w) for w in weights]
    x_host = synth.hidden_states(args.seed, T)
    x = torch.from_numpy(x_host).to(dev)
    out = torch.empty_like(x)
    t_gen = time.perf_counter() - t_gen

    # data-dependent hit counts per layer (for the algorithmic byte counts)
    per_layer = []
    for w, layer in zip(weights, layers):
        tr = RouteTrace(T, w.n_experts, w.n_used)
        layer.forward(np.ascontiguousarray(x_host.reshape(-1)), T, np.empty(T * w.hidden, np.float32), tr)
        per_layer.append(algorithmic_bytes(w, tr.counts, T))

    for i in range(args.warmup):
        layers[i % L].forward(x, T, out)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        layers[i % L].forward(x, T, out)
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    ms = el * 1e3 / args.steps

    # second pass with HIP events around every launch, for per-kernel mean durations
    ctx.profile(True)
    ctx.reset_stats()
    for i in range(args.steps):
        layers[i % L].forward(x, T, out)
    stats = ctx.kernel_stats()
    ctx.profile(False)

    used = [per_layer[i % L] for i in range(args.steps)]
    avg = {k: float(np.mean([u[k] for u in used])) for k in used[0]}
    kern_us = {n: v[0] * 1e3 / v[1] for n, v in stats.items()}
    dominant = max(("gateup_swiglu", "down_combine"), key=lambda n: stats.get(n, (0, 1))[0])
    dom_us = kern_us[dominant]
    achieved = avg[dominant] / (dom_us * 1e-6) / 1e9
    traffic = None
    tfile = os.path.join(ROOT, "profiles", f"traffic_{dominant}_{cfg.name}.json")
    if os.path.exists(tfile):
        traffic = json.load(open(tfile)).get("hbm_bytes_per_launch")

    result = {
        "metric": "MoE-block decode tok/s (config 2: 16 tokens, one MoE FFN block)",
        "value": T / (ms * 1e-3),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded Q4_K experts, N(0,1) hidden states; no GGUF offline)",
        "config": {"workload": f"config {args.config}: {cfg.description}", "tokens": T, "hidden": 2048,
                   "moe_ff": 1792, "experts": 32, "top_k": 4, "down": "Q6_K" if cfg.down_dtype == 14 else "Q4_K",
                   "weight_sets_rotated": L, "weight_bytes_resident": int(sum(w.nbytes for w in weights))},
        "block_hbm_gbps": avg["step"] / (ms * 1e-3) / 1e9,
        "block_frac_of_8tbs": avg["step"] / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS,
        "mean_hit_experts": avg["u_hit"],
        "kernel_us": {k: round(v, 3) for k, v in kern_us.items()},
        "roofline": {"kernel": dominant, "bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBPS, "traffic": traffic,
                     "algorithmic_bytes_per_launch": avg[dominant]},
        "cpu_baseline": None,
        "setup_s": round(t_gen, 1),
    }
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(weights[: min(L, 4)], x_host, T, args.cpu_seconds)
    for l in layers:
        l.close()
    ctx.close()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
