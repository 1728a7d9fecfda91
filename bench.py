"""Benchmark of the MI355X MoE FFN block (one GPU).

Default workload: BASELINE.json config 2. That is a decode batch of 16 independent tokens
through one sparse-MoE block of LFM2.5-8B-A1B's shape (hidden 2048, expert FFN 1792, 32
experts, top-4, Q4_K experts with Q8 activations). A step is one pass of the hot path over one
batch: router, gating, dispatch, gate/up + SwiGLU, down, combine. `--config 1|3|4` runs the
other single-block configurations (3 and 4 take the batched path: dispatch and grouped int8-MFMA
GEMMs), `--config 5` the 24-layer FFN stack at one token.

The 256 MB Infinity Cache would hold one layer's 198-228 MB of experts, so for configs 1-4 step
i runs layer i mod L of L independently generated layers (L = 12 by default, 2.4-2.7 GB), as
successive layers of a real model would; config 5 holds its ~5 GB of layers resident. Inputs are
resident in HBM before the timed region.

The output is one JSON line with `value` in tok/s. It also carries:
  roofline      the dominant kernel's algorithmic bytes (decode, config 3) or operations
                (config 4) per launch divided by its mean launch time, measured with HIP events
                on the stream the kernels run on, against MI355X's 8 TB/s or int8 MFMA peak
  cpu_baseline  the reference path (its C++ restatement, OpenMP over output rows as the
                reference's rayon does) timed on this host: the median of 20 timed repetitions
                on all cores, the same on one core, and the CPU model
  prefill       (default run only) config 4 measured in the same process the same way: tok/s,
                ms per step, the grouped GEMMs' µs and their int8 / bf16 MFMA fractions
  decode_t1     (default run only) config 1, one token through one MoE block
  prefill_t512  (default run only) config 3, 512 tokens through one MoE block (unbiased router)
  ffn_stack     (default run only) config 5, the 24-layer FFN stack at one token
  decoder       (default run only) the whole decoder at LFM2.5-8B-A1B's full shape (24 layers:
                short conv / GQA attention operators, 2 dense + 22 MoE FFNs, the 128000-row
                logits head): a 512-token prompt absorbed as one prefill chunk, then one-token
                forward_steps at that context, and at 4,096 and 16,384 positions; per-kernel
                times of a decode step; the C++ restatement's forward_step timed on this host
                at the same 512-token context
Each object carries its own ms_per_step, kernel_us, roofline and cpu_baseline.
"""
import argparse
import json
import os
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0
INT8_PEAK_TOPS = 5000.0   # MI355X dense int8 MFMA
BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA (the north-star prefill target's yardstick)

DECODE_KERNELS = ("gateup_swiglu", "down_combine")
GEMM_KERNELS = ("gemm_gateup", "gemm_down")
BATCHED_MIN_ENTRIES = 64  # the library's default T*k from which the grouped int8-MFMA path runs
ROUTE_IN_GATEUP_MAX_T = 4  # up to this many tokens the gate/up GEMV routes them itself


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--config", type=int, default=2, choices=[1, 2, 3, 4, 5])
    ap.add_argument("--layers", type=int, default=12, help="distinct weight sets rotated across steps")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="bound on the CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-prefill", action="store_true", help="skip the config-4 prefill object of the default run")
    ap.add_argument("--no-decoder", action="store_true", help="skip the whole-decoder object of the default run")
    ap.add_argument("--no-others", action="store_true",
                    help="skip the config 1, 3 and 5 objects (decode_t1, prefill_t512, ffn_stack) of the default run")
    ap.add_argument("--cpu-reps", type=int, default=20, help="timed repetitions of the CPU baseline")
    ap.add_argument("--logits-head", action="store_true",
                    help="time bb_logits_from_hidden (rmsnorm + Q6_K 2048 -> 128000 matvec) instead of a config")
    return ap.parse_args()


def logits_head(args):
    """One decode token's logits (model.rs:380-388) on the device: the token_embd matvec of
    2048 -> 128000 Q6_K rows (215 MB) after the final rmsnorm. Prints one JSON line."""
    import torch

    from bebelm_amd import kernels as kops
    from bebelm_amd import synth
    from bebelm_amd.model import Context, Tensor

    H, V = 2048, 128000
    steps = args.steps if args.steps is not None else 200
    warmup = args.warmup if args.warmup is not None else 20
    ctx = Context(0)
    ctx.set_stream(torch.cuda.current_stream().cuda_stream)
    w = synth.quant_tensor(synth.rng(args.seed, synth.Q6_K, V), synth.Q6_K, H, V)
    emb = Tensor(ctx, synth.Q6_K, w, (H, V))
    h = torch.from_numpy(synth.hidden_states(args.seed, 1).reshape(-1)).cuda()
    gain = torch.ones(H, dtype=torch.float32, device="cuda")
    y = torch.empty(V, dtype=torch.float32, device="cuda")
    for _ in range(warmup):
        kops.logits_from_hidden(ctx, emb, gain, 1e-5, h, y)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        kops.logits_from_hidden(ctx, emb, gain, 1e-5, h, y)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    ctx.profile(True)
    ctx.reset_stats()
    for _ in range(steps):
        kops.logits_from_hidden(ctx, emb, gain, 1e-5, h, y)
    stats = ctx.kernel_stats()
    ctx.profile(False)
    kern_us = {n: v[0] * 1e3 / v[1] for n, v in stats.items()}
    nbytes = synth.byte_size(synth.Q6_K, H * V) + q8_bytes(H) + V * 4
    achieved = nbytes / (kern_us["rows_q8"] * 1e-6) / 1e9
    print(json.dumps({
        "metric": "logits head tok/s (rmsnorm + Q6_K token_embd matvec 2048 -> 128000)",
        "value": 1e3 / ms, "unit": "tok/s", "n_gpus": 1, "steps": steps, "warmup": warmup, "ms_per_step": ms,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic (seeded Q6_K rows)", "config": {"workload": "logits_head_q6k_2048x128000"},
        "kernel_us": kern_us,
        "roofline": {"kernel": "rows_q8", "bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBPS, "traffic": None, "algorithmic_bytes_per_launch": nbytes},
    }), flush=True)


def q8_bytes(n):
    return n + n // 256 * 4


def kernel_names(T, K, E, batched):
    """The two expert kernels a call runs: per-expert GEMVs below BATCHED_MIN_ENTRIES entries,
    grouped int8-MFMA GEMMs from there."""
    return GEMM_KERNELS if batched else DECODE_KERNELS


def layer_work(w, counts, T, batched, prerouted=False):
    """Algorithmic bytes and int8 operations per kernel launch of one MoE layer.

    Bytes: weights of the hit experts (each read once), activations in, results out; no
    intermediates re-read. Operations: 2 per multiply-add of the expert GEMMs. prerouted: the
    router logits and the XQ records come from the stack's layer boundary (the gate/up GEMV
    reads them instead of the router and the f32 rows)."""
    from bebelm_amd import synth

    H, F, K = w.hidden, w.moe_ff, w.n_used
    n_ent = T * K
    u_hit = int(np.count_nonzero(counts))
    gu = synth.byte_size(w.gate_dtype, H * F) + synth.byte_size(w.up_dtype, H * F)
    dn = synth.byte_size(w.down_dtype, F * H)
    if not batched and T <= ROUTE_IN_GATEUP_MAX_T and prerouted:
        gate_b = u_hit * gu + T * (q8_bytes(H) + H // 256 * 48) + T * w.n_experts * 4 + n_ent * F * 4
    elif not batched and T <= ROUTE_IN_GATEUP_MAX_T:
        # the kernel also routes: the router and the f32 rows are its inputs
        gate_b = u_hit * gu + w.router.nbytes + T * H * 4 + n_ent * F * 4
    else:
        gate_b = u_hit * gu + T * q8_bytes(H) + n_ent * F * 4
        if T <= 16 and n_ent <= 64 and w.gate_dtype == synth.Q4_K and w.n_experts <= 32:
            gate_b += n_ent * q8_bytes(F)  # k_gateup16 also writes the act rows' Q8
    # one token on its own (not in the stack): the down GEMV also combines, writing H outputs
    # instead of K slot rows
    combine_in_down = not batched and T == 1 and K <= 4 and not prerouted
    down_b = u_hit * dn + n_ent * (F * 4 if not batched else q8_bytes(F)) + (T if combine_in_down else n_ent) * H * 4
    gate_ops = 2.0 * n_ent * 2 * F * H
    down_ops = 2.0 * n_ent * F * H
    names = kernel_names(T, K, w.n_experts, batched)
    return {
        names[0]: (gate_b, gate_ops),
        names[1]: (down_b, down_ops),
        "step_bytes": u_hit * (gu + dn) + w.router.nbytes + T * H * 4 * 2,
        "u_hit": u_hit,
        "ops": gate_ops + down_ops,
    }


def cpu_baseline(run_one, T, seconds, what, reps=20, one_core=True, reps_1core=None):
    """The reference path's C++ restatement on this host's cores: `reps` timed repetitions of
    about seconds / reps each (whole calls, at least one), tok/s as their median; then the same
    on one core (reps_1core repetitions, default `reps`). run_one(i) runs call i (callers rotate
    weight sets by i)."""
    from oracle import bbo

    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count() or 1
    cores = min(cores, int(os.environ.get("OMP_NUM_THREADS", cores)))

    def median_rate(threads, budget, n_reps):
        bbo.set_threads(threads)
        run_one(0)  # warm-up: pages in weights, starts the thread pool
        rates, calls = [], 1
        per_rep = budget / n_reps
        for _ in range(n_reps):
            n = 0
            t0 = time.perf_counter()
            while True:
                run_one(calls)
                calls += 1
                n += 1
                el = time.perf_counter() - t0
                if el >= per_rep:
                    break
            rates.append(n * T / el)
        return float(np.median(rates)), calls - 1

    value, n_all = median_rate(cores, seconds, reps)
    out = {"value": value, "unit": "tok/s", "cores": cores, "kind": "port", "cpu_model": bbo.cpu_model(),
           "oracle_build": os.path.basename(bbo.lib_path())}
    each = "one call each" if seconds / reps < 0.01 else f"about {seconds / reps:.2f} s each"
    sample = (f"median of {reps} repetitions ({n_all} calls, {each}) of the C++ "
              f"restatement of {what}, OpenMP over output rows")
    if one_core and cores > 1:
        r1 = reps_1core or reps
        v1, n1 = median_rate(1, seconds * r1 / reps, r1)
        out["value_1core"] = v1
        sample += f"; 1 core: {n1} calls in {r1} repetitions"
    bbo.set_threads(cores)
    out["sample"] = sample
    return out


def run_config(args, ctx, config, steps, warmup, with_cpu, cpu_share=1.0):
    """Times `steps` steps of one configuration (after `warmup`), then the same steps again with
    per-kernel HIP events; returns the bench fields of that configuration. cpu_share scales the
    CPU baseline's time budget (--cpu-seconds) for the secondary configurations."""
    import torch

    from bebelm_amd import synth
    from bebelm_amd.model import DenseLayer, FfnStack, MoeLayer, RouteTrace

    cfg = synth.CONFIGS[config]
    T = cfg.tokens
    prefill = config in (3, 4)
    dev = torch.device("cuda:0")
    batched = T * 4 >= BATCHED_MIN_ENTRIES

    t_gen = time.perf_counter()
    x_host = synth.hidden_states(args.seed, T)
    x = torch.from_numpy(x_host).to(dev)
    out = torch.empty_like(x)
    if config == 5:
        spec = synth.stack_layers(seed=args.seed)
        built = [(g, MoeLayer(ctx, w) if isinstance(w, synth.MoeWeights) else DenseLayer(ctx, w)) for g, w in spec]
        stack = FfnStack(ctx, built)
        dense_w = [w for _, w in spec if not isinstance(w, synth.MoeWeights)]
        units = [stack]
        weight_bytes = int(sum(w.nbytes for _, w in spec))
        L = 1
    else:
        L = max(1, args.layers)
        weights = synth._par_map(lambda l: synth.config_layer(config, seed=args.seed, layer=l), range(L))
        units = [MoeLayer(ctx, w) for w in weights]
        weight_bytes = int(sum(w.nbytes for w in weights))
    t_gen = time.perf_counter() - t_gen

    # data-dependent hit counts (for the algorithmic byte counts)
    if config == 5:
        from bebelm_amd import kernels as kops
        # routing of every MoE layer of the stack for this token, from the library's own route
        # trace, layer by layer on the host-side residual stream (run_layers, model.rs:105-130)
        layers_work = []
        h = x_host.reshape(-1).copy()
        for (g, w), (_, layer) in zip(spec, built):
            normed = np.empty_like(h)
            kops.rmsnorm(ctx, h, g, 1e-5, normed)
            y = np.empty_like(h)
            if isinstance(w, synth.MoeWeights):
                tr = RouteTrace(1, w.n_experts, w.n_used)
                layer.forward(normed, 1, y, tr)
                # (every MoE layer follows a layer boundary that computes its logits)
                layers_work.append(layer_work(w, tr.counts, 1, False, prerouted=True))
            else:
                layer.forward(normed, 1, y)
            h = (h + y).astype(np.float32)
        dense_bytes = sum(synth.byte_size(w.gate_dtype, w.hidden * w.ff) * 3 for w in dense_w)
        step_bytes = sum(l["step_bytes"] for l in layers_work) + dense_bytes
    else:
        per_layer = []
        for w, layer in zip(weights, units):
            tr = RouteTrace(T, w.n_experts, w.n_used)
            layer.forward(np.ascontiguousarray(x_host.reshape(-1)), T, np.empty(T * w.hidden, np.float32), tr)
            per_layer.append(layer_work(w, tr.counts, T, batched))

    def step(i):
        units[i % len(units)].forward(x, T, out)

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        step(i)
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    ms = el * 1e3 / steps

    # second pass with HIP events around every launch on the same stream: mean kernel durations
    ctx.profile(True)
    ctx.reset_stats()
    for i in range(steps):
        step(i)
    stats = ctx.kernel_stats()
    ctx.profile(False)
    kern_us = {n: v[0] * 1e3 / v[1] for n, v in stats.items()}

    if config == 5:
        names = DECODE_KERNELS
        avg = {n: float(np.mean([lw[n][0] for lw in layers_work])) for n in names}
        avg_ops = {n: float(np.mean([lw[n][1] for lw in layers_work])) for n in names}
        u_hit = float(np.mean([lw["u_hit"] for lw in layers_work]))
    else:
        names = kernel_names(T, 4, 32, batched)
        used = [per_layer[i % L] for i in range(steps)]
        avg = {n: float(np.mean([u[n][0] for u in used])) for n in names}
        avg_ops = {n: float(np.mean([u[n][1] for u in used])) for n in names}
        step_bytes = float(np.mean([u["step_bytes"] for u in used]))
        u_hit = float(np.mean([u["u_hit"] for u in used]))
    dominant = max(names, key=lambda n: stats.get(n, (0, 1))[0])
    dom_us = kern_us[dominant]
    traffic = None
    tfile = os.path.join(ROOT, "profiles", f"traffic_{dominant}_{cfg.name}.json")
    if os.path.exists(tfile):
        traffic = json.load(open(tfile)).get("hbm_bytes_per_launch")
    if config == 4:
        achieved = avg_ops[dominant] / (dom_us * 1e-6) / 1e12
        roofline = {"kernel": dominant, "bound": "mfma", "achieved": achieved, "peak": INT8_PEAK_TOPS,
                    "unit": "TFLOP/s", "frac": achieved / INT8_PEAK_TOPS, "traffic": traffic,
                    "ops_per_launch": avg_ops[dominant], "op_type": "int8 multiply-adds x2",
                    "frac_of_bf16_peak": achieved / BF16_PEAK_TFLOPS}
    else:
        achieved = avg[dominant] / (dom_us * 1e-6) / 1e9
        roofline = {"kernel": dominant, "bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                    "frac": achieved / HBM_PEAK_GBPS, "traffic": traffic,
                    "algorithmic_bytes_per_launch": avg[dominant]}

    kind = "prefill" if prefill else ("FFN-stack decode" if config == 5 else "decode")
    result = {
        "metric": f"MoE-block {kind} tok/s (config {config}: {T} token{'s' if T > 1 else ''}"
                  f"{', 24-layer FFN stack' if config == 5 else ', one MoE FFN block'})",
        "value": T / (ms * 1e-3),
        "unit": "tok/s",
        "ms_per_step": ms,
        "config": {"workload": f"config {config}: {cfg.description}", "tokens": T, "hidden": 2048,
                   "moe_ff": 1792, "experts": 32, "top_k": 4,
                   "down": "Q4_K/Q6_K alternating" if config == 5 else
                           ("Q6_K" if cfg.down_dtype == 14 else "Q4_K"),
                   "path": "grouped int8-MFMA GEMMs" if batched else "per-expert GEMV",
                   "weight_sets_rotated": L, "weight_bytes_resident": weight_bytes},
        "block_hbm_gbps": step_bytes / (ms * 1e-3) / 1e9,
        "block_frac_of_8tbs": step_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS,
        "mean_hit_experts": u_hit,
        "kernel_us": {k: round(v, 3) for k, v in kern_us.items()},
        "roofline": roofline,
        "cpu_baseline": None,
        "setup_s": round(t_gen, 1),
    }
    if prefill:
        ops = float(np.mean([per_layer[i % L]["ops"] for i in range(steps)]))
        gemm_us = sum(kern_us.get(n, 0.0) for n in GEMM_KERNELS)
        gemm_tops = ops / (gemm_us * 1e-6) / 1e12
        result["block_tflops"] = ops / (ms * 1e-3) / 1e12
        result["block_frac_of_bf16_peak"] = result["block_tflops"] / BF16_PEAK_TFLOPS
        result["gemms"] = {"gateup_us": kern_us.get("gemm_gateup"), "down_us": kern_us.get("gemm_down"),
                           "us": gemm_us, "ops": ops, "tops": gemm_tops,
                           "frac_of_int8_peak": gemm_tops / INT8_PEAK_TOPS,
                           "frac_of_bf16_peak": gemm_tops / BF16_PEAK_TFLOPS}
    if with_cpu:
        from oracle import bbo

        secs = args.cpu_seconds * cpu_share
        if config == 5:
            layers_o = [(g, w) for g, w in spec]
            result["cpu_baseline"] = cpu_baseline(lambda i: bbo.ffn_stack(layers_o, x_host.reshape(-1), 1, 1e-5), T,
                                                  secs, "the 24-layer FFN stack (T=1)", args.cpu_reps)
        elif prefill:
            # one call takes about 0.3 s (T = 512) or 2-4 s (T = 4096) on all cores: repetitions
            # of one call each. Config 3: 20 of them, then 3 on one core (about 1.2 s each);
            # config 4: 5 on all cores, then one call on one core (about 13 s)
            sample = weights[: min(L, 4)]
            xs = x_host.reshape(-1)
            reps = 20 if config == 3 else 5
            result["cpu_baseline"] = cpu_baseline(lambda i: bbo.moe_ffn_batch(sample[i % len(sample)], xs, T), T,
                                                  1e-3 * reps, f"moe_ffn_batch (T={T}, {len(sample)} rotated layers)",
                                                  reps, reps_1core=3 if config == 3 else 1)
        else:
            sample = weights[: min(L, 4)]
            xs = x_host.reshape(-1)
            fn = (lambda i: bbo.moe_ffn(sample[i % len(sample)], xs)) if T == 1 else \
                (lambda i: bbo.moe_ffn_batch(sample[i % len(sample)], xs, T))
            result["cpu_baseline"] = cpu_baseline(fn, T, secs,
                                                  f"moe_ffn{'_batch' if T > 1 else ''} (T={T}, {len(sample)} rotated layers)",
                                                  args.cpu_reps)
    if config == 5:
        stack.close()
        for _, l in built:
            l.close()
    else:
        for l in units:
            l.close()
    return result, steps, warmup


def decoder_bench(args, ctx, with_cpu):
    """The whole decoder (Model::forward_step, Agent::absorb) at full size on the GPU."""
    import torch

    from bebelm_amd import gguf, synth
    from bebelm_amd.model import Model

    mw = synth.model_weights(seed=args.seed)
    # the decoder is loaded the way Model::load does it (model.rs:36-50): from a GGUF file, every
    # tensor copied from the file's mapping into HBM; the file is written first (page-cache warm)
    upload = None
    tmpdir = tempfile.mkdtemp(prefix="bb_gguf_")
    path = os.path.join(tmpdir, "model.gguf")
    try:
        synth.model_gguf(mw).save(path)
        nbytes = os.path.getsize(path)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        with gguf.GgufFile.open(path) as g:
            g.validate()
            m = Model.load(ctx, g)
        up = time.perf_counter() - t0
        upload = {"file_gb": round(nbytes / 1e9, 3), "load_s": round(up, 3), "gb_s": round(nbytes / up / 1e9, 2),
                  "what": "bb_gguf_open + validate + bb_model_load (tensor table check, every tensor "
                          "copied from the mapping into HBM, MoE weights repacked on the GPU); file in page cache"}
    except OSError as e:  # no room for the file: build the same decoder from the arrays
        upload = {"skipped": f"could not write the GGUF file: {e}"}
        m = Model(ctx, mw)
    finally:
        if os.path.exists(path):
            os.remove(path)
        os.rmdir(tmpdir)
    prompt = np.random.default_rng(args.seed + 1).integers(0, mw.vocab, 512).astype(np.uint32)
    cache = m.new_cache(4096)

    def prefill_once():
        cache.reset()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        m.absorb(cache, prompt, 4096)  # one chunk of 512 (agent.rs:31); returns after the stream drained
        return time.perf_counter() - t0

    prefill_once()
    pre = sorted(prefill_once() for _ in range(3))[1]
    rng_dec = np.random.default_rng(args.seed + 2)

    def decode_rate(n_dec):
        """The one-token step with its logits back on the host at the cache's context."""
        toks = rng_dec.integers(0, mw.vocab, n_dec + 4)
        for t in toks[:4]:
            m.forward_step(int(t), cache)
        t0 = time.perf_counter()
        for t in toks[4:]:
            m.forward_step(int(t), cache)
        return (time.perf_counter() - t0) / n_dec

    # decode at a 512-token context: the median of three runs of 32 steps (the host's share of a
    # step varies from run to run)
    dec = sorted(decode_rate(32) for _ in range(3))[1]
    # per-kernel times of decode steps (events stamped by each dispatch)
    ctx.reset_stats()
    ctx.profile(True)
    for t in rng_dec.integers(0, mw.vocab, 8):
        m.forward_step(int(t), cache)
    stats = ctx.kernel_stats()
    ctx.profile(False)
    total = sum(v[0] for v in stats.values()) or 1.0
    per_step = {k: round(v[0] / 8 * 1e3, 1) for k, v in sorted(stats.items(), key=lambda kv: -kv[1][0]) if v[1]}
    # long contexts (the reference's agent window is 32,768 positions, agent.rs:25-26): the
    # prompt grows by chunks of 512 to 4,096 and then 16,384 positions, and the decode step is
    # timed at each
    long_ctx = {}
    for n_ctx in (4096, 16384):
        more = n_ctx - cache.kv_len()
        t0 = time.perf_counter()
        m.absorb(cache, rng_dec.integers(0, mw.vocab, more).astype(np.uint32), 32768)
        ab = time.perf_counter() - t0
        d = sorted(decode_rate(16) for _ in range(3))[1]
        ctx.reset_stats()
        ctx.profile(True)
        for t in rng_dec.integers(0, mw.vocab, 4):
            m.forward_step(int(t), cache)
        st = ctx.kernel_stats()
        ctx.profile(False)
        long_ctx[f"ctx{n_ctx}"] = {"ms_per_token": round(d * 1e3, 3), "tok_s": round(1.0 / d, 1),
                                   "absorb_ms": round(ab * 1e3, 1), "absorbed_tokens": int(more),
                                   "kernel_ms_per_step": round(sum(v[0] for v in st.values()) / 4, 3),
                                   "attention_kernel_us_per_step": {
                                       k: round(v[0] / 4 * 1e3, 1) for k, v in st.items()
                                       if k.startswith("attn") and v[1]}}
    out = {
        "workload": "LFM2.5-8B-A1B shape: 24 layers (6 GQA attention, 18 short conv), 2 dense + 22 MoE FFNs, "
                    "vocab 128000, Q4_K/Q6_K synthetic weights",
        "prefill_512": {"ms": round(pre * 1e3, 2), "tok_s": round(512 / pre, 1)},
        "decode_t1_ctx512": {"ms_per_token": round(dec * 1e3, 3), "tok_s": round(1.0 / dec, 1),
                             "includes": "host call, logits copied back to the host"},
        "decode_long_context": long_ctx,
        "decode_kernel_us_per_step": per_step,
        "decode_kernel_ms_per_step": round(total / 8, 3),
        "gguf_upload": upload,
    }
    cache.close()
    m.close()
    if with_cpu:
        from oracle import bbo

        # the restatement at the GPU figure's context: the same 512-token prompt absorbed
        # (batched, as Agent::absorb does), then forward_steps at 512+ positions
        om = bbo.Model(mw, 600)
        t0 = time.perf_counter()
        om.absorb(list(prompt), 4096)
        cpu_pre = time.perf_counter() - t0
        toks = np.random.default_rng(args.seed + 3).integers(0, mw.vocab, 3)
        t0 = time.perf_counter()
        for t in toks:
            om.forward_step(int(t))
        cpu = (time.perf_counter() - t0) / len(toks)
        out["cpu_baseline"] = {"value": round(1.0 / cpu, 2), "unit": "tok/s", "cores": bbo.get_threads(),
                               "kind": "port", "prefill_512_tok_s": round(512 / cpu_pre, 1),
                               "sample": f"the 512-token prompt absorbed in one chunk, then {len(toks)} forward_steps "
                               "of the C++ restatement (Python composition of its operators) at a 512-token context"}
    return out


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only; --gpus {args.gpus} is not supported by this build", file=sys.stderr)
        sys.exit(2)
    if args.logits_head:
        logits_head(args)
        return
    import torch

    from bebelm_amd.model import Context

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    ctx = Context(0)
    ctx.set_stream(torch.cuda.current_stream().cuda_stream)

    def defaults(config):
        # timed steps: 0.04-0.11 s of GPU work each, so that the fixed cost of a timed region (the
        # launch queue filling behind the first step, the final synchronisation) is a small share
        # of a step (config 2: 53.3 µs a step over 200 steps, 49.5-49.7 µs over 2000)
        steps = args.steps if args.steps is not None else {1: 2000, 2: 2000, 3: 500, 4: 100, 5: 200}[config]
        warmup = args.warmup if args.warmup is not None else {1: 200, 2: 200, 3: 50, 4: 10, 5: 20}[config]
        return steps, warmup

    steps, warmup = defaults(args.config)
    res, steps, warmup = run_config(args, ctx, args.config, steps, warmup, not args.no_cpu)
    result = {
        "metric": res.pop("metric"),
        "value": res.pop("value"),
        "unit": res.pop("unit"),
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": res.pop("ms_per_step"),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded Q4_K/Q6_K experts, N(0,1) hidden states; no GGUF offline)",
        "config": res.pop("config"),
        **res,
    }
    def sub(config, share):
        """Another BASELINE configuration measured in the same process the same way, as an
        object of the line."""
        ps, pw = defaults(config)
        if args.steps is not None:
            ps = min(ps, args.steps)
        if args.warmup is not None:
            pw = min(pw, args.warmup)
        p, ps, pw = run_config(args, ctx, config, ps, pw, not args.no_cpu, share)
        o = {"metric": p["metric"], "value": p["value"], "unit": "tok/s", "steps": ps, "warmup": pw,
             "ms_per_step": p["ms_per_step"], "config": p["config"]}
        for k in ("gemms", "block_tflops", "block_frac_of_bf16_peak", "block_hbm_gbps", "block_frac_of_8tbs"):
            if k in p:
                o[k] = p[k]
        o.update({"kernel_us": p["kernel_us"], "roofline": p["roofline"], "cpu_baseline": p["cpu_baseline"],
                  "mean_hit_experts": p["mean_hit_experts"]})
        return o

    if args.config == 2 and not args.no_others:
        # the metric's other configurations: one token (config 1), 512-token prefill (config 3),
        # the 24-layer FFN stack at one token (config 5)
        result["decode_t1"] = sub(1, 0.4)
        result["prefill_t512"] = sub(3, 1.0)
    if args.config == 2 and not args.no_prefill:
        # the metric's prefill half: config 4 in the same process, measured the same way
        result["prefill"] = sub(4, 1.0)
    if args.config == 2 and not args.no_others:
        result["ffn_stack"] = sub(5, 0.5)
    if args.config == 2 and not args.no_decoder:
        result["decoder"] = decoder_bench(args, ctx, not args.no_cpu)
    ctx.close()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
