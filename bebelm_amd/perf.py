"""Profiling driver and counter post-processing for the MoE kernels (not part of the product path).

Four subcommands:

  python3 -m bebelm_amd.perf drive --decoder [--steps 16]
      The whole decoder at full size: a 512-token prompt absorbed, then `steps` forward_steps.

  python3 -m bebelm_amd.perf drive --config 2 [--steps 50] [--layers 12]
      Runs the config's MoE layer `steps` times on cuda:0 (rotating `layers` weight sets, as
      bench.py does), then a device-to-device copy of CAL_BYTES with a known byte count. Meant
      to run under `rocprofv3 --pmc FETCH_SIZE` and `rocprofv3 --pmc WRITE_SIZE`; the copy is
      the calibration reference for those counters.

  python3 -m bebelm_amd.perf traffic --fetch F.csv --write W.csv --kernel SUBSTR --config 2
      Reads the two counter-collection CSVs, calibrates FETCH_SIZE and WRITE_SIZE against the
      copy kernel (read = written = CAL_BYTES), and writes
      profiles/traffic_<name>_<workload>.json with the HBM bytes per launch of the kernels whose
      name contains SUBSTR.

  python3 -m bebelm_amd.perf stats --csv S.csv --command CMD --bench B.json --bench-command BCMD
      Writes profiles/kernel_stats_<workload>.md: the per-kernel table of S, the
      *_kernel_stats.csv of the `rocprofv3 --kernel-trace --stats` run CMD of bench.py, and the
      bench line B of the unprofiled run BCMD (the profiler's own completion signals slow the
      bench's event-timed pass, so its line comes from a run without it).

  python3 -m bebelm_amd.perf pmc --csv P1.csv P2.csv ... --commands C1 C2 ... --config 4
      Writes profiles/pmc_<workload>.md: per kernel whose name contains one of --kernels, the
      mean per dispatch of every counter of the `rocprofv3 --pmc` passes (one CSV per pass;
      the commands that made them are quoted), with instruction counts per wave and the
      VALU : MFMA instruction ratio.
"""
import argparse
import collections
import csv
import json
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CAL_BYTES = 512 << 20
COPY_KERNEL = "copyBuffer"


def drive_decoder(args):
    """The whole decoder at full size: a 512-token prompt absorbed, then `steps` forward_steps."""
    import numpy as np
    import torch

    sys.path.insert(0, ROOT)
    from bebelm_amd import synth
    from bebelm_amd.model import Context, Model

    ctx = Context(0)
    ctx.set_stream(torch.cuda.current_stream().cuda_stream)
    mw = synth.model_weights(seed=0)
    m = Model(ctx, mw)
    cache = m.new_cache(4096)
    g = np.random.default_rng(1)
    m.absorb(cache, g.integers(0, mw.vocab, 512).astype(np.uint32), 4096)
    for t in g.integers(0, mw.vocab, args.steps):
        m.forward_step(int(t), cache)
    torch.cuda.synchronize()
    cache.close()
    m.close()
    ctx.close()


def drive(args):
    import torch

    if args.decoder:
        drive_decoder(args)
        return
    sys.path.insert(0, ROOT)
    from bebelm_amd import synth
    from bebelm_amd.model import Context, MoeLayer

    cfg = synth.CONFIGS[args.config]
    T = cfg.tokens
    ctx = Context(0)
    ctx.set_stream(torch.cuda.current_stream().cuda_stream)
    if args.config == 5:
        # the 24-layer FFN stack (bench.py's config 5): all layers resident, one token per step
        from bebelm_amd.model import DenseLayer, FfnStack

        spec = synth.stack_layers(seed=0)
        built = [(g, MoeLayer(ctx, w) if isinstance(w, synth.MoeWeights) else DenseLayer(ctx, w)) for g, w in spec]
        layers = [FfnStack(ctx, built)]
    else:
        built = []
        weights = synth._par_map(lambda l: synth.config_layer(args.config, seed=0, layer=l), range(args.layers))
        layers = [MoeLayer(ctx, w) for w in weights]
    x = torch.from_numpy(synth.hidden_states(0, T)).cuda()
    out = torch.empty_like(x)
    for i in range(args.steps):
        layers[i % len(layers)].forward(x, T, out)
    torch.cuda.synchronize()
    src = torch.empty(CAL_BYTES // 4, dtype=torch.float32, device="cuda").fill_(1.0)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    for l in layers:
        l.close()
    for _, l in built:
        l.close()
    ctx.close()
    print("perf drive done", flush=True)


def _per_kernel(path, counter):
    vals = collections.defaultdict(list)
    with open(path) as f:
        for row in csv.DictReader(f):
            if row.get("Counter_Name") != counter:
                continue
            vals[row["Kernel_Name"]].append(float(row["Counter_Value"]))
    return vals


def traffic(args):
    sys.path.insert(0, ROOT)
    from bebelm_amd import synth

    cfg = synth.CONFIGS[args.config]
    fetch = _per_kernel(args.fetch, "FETCH_SIZE")
    write = _per_kernel(args.write, "WRITE_SIZE")

    def mean_of(d, sub):
        xs = [v for k, vs in d.items() if sub in k for v in vs]
        if not xs:
            raise SystemExit(f"no dispatches of a kernel containing {sub!r}")
        return sum(xs) / len(xs), len(xs)

    # counters are in KiB per dispatch; the calibration copies are the large copy dispatches
    # (smaller ones are the uploads of weights and constants)
    def cal_of(d):
        xs = [v for k, vs in d.items() if COPY_KERNEL in k for v in vs if v * 1024.0 > CAL_BYTES / 8]
        if not xs:
            raise SystemExit("no calibration copy found")
        return sum(xs) / len(xs)

    cal_f, cal_w = cal_of(fetch), cal_of(write)
    f_factor = CAL_BYTES / (cal_f * 1024.0)
    w_factor = CAL_BYTES / (cal_w * 1024.0)
    kf, n = mean_of(fetch, args.kernel)
    kw, _ = mean_of(write, args.kernel)
    res = {
        "kernel": args.kernel,
        "workload": cfg.name,
        "dispatches": n,
        "fetch_kib_per_launch": kf,
        "write_kib_per_launch": kw,
        "copy_calibration": {"bytes_read": CAL_BYTES, "bytes_written": CAL_BYTES, "fetch_kib": cal_f,
                             "write_kib": cal_w, "fetch_factor": f_factor, "write_factor": w_factor},
        "hbm_read_bytes_per_launch": kf * 1024.0 * f_factor,
        "hbm_write_bytes_per_launch": kw * 1024.0 * w_factor,
    }
    res["hbm_bytes_per_launch"] = res["hbm_read_bytes_per_launch"] + res["hbm_write_bytes_per_launch"]
    if args.command_fetch:
        res["command_fetch"] = args.command_fetch
    if args.command_write:
        res["command_write"] = args.command_write
    name = args.name or args.kernel
    out = os.path.join(ROOT, "profiles", f"traffic_{name}_{cfg.name}.json")
    with open(out, "w") as f:
        json.dump(res, f, indent=1)
    print(json.dumps(res, indent=1))


def stats(args):
    sys.path.insert(0, ROOT)
    from bebelm_amd import synth

    if args.decoder:
        wname, title = "decoder_full", ("the whole decoder at LFM2.5-8B-A1B's shape (24 layers, 128000-row "
                                       "logits head): a 512-token prompt absorbed, then one-token forward_steps")
    else:
        cfg = synth.CONFIGS[args.config]
        wname, title = cfg.name, f"config {args.config} ({cfg.name}): {cfg.description}"
    rows = []
    with open(args.csv) as f:
        for row in csv.DictReader(f):
            name = row["Name"].split("(")[0]
            rows.append((name, int(row["Calls"]), float(row["AverageNs"]) / 1e3, float(row["MinNs"]) / 1e3,
                         float(row["MaxNs"]) / 1e3, float(row["Percentage"])))
    bench = None
    if args.bench:
        with open(args.bench) as f:
            for line in f:
                line = line.strip()
                if line.startswith("{"):
                    bench = json.loads(line)
    keep = ("value", "unit", "ms_per_step", "kernel_us", "roofline")
    out = [f"# Kernel statistics — {title}", "",
           "Command (from the repository root on one MI355X; `cd /tmp && export TMPDIR=/tmp` first for "
           "rocprofv3's scratch files):", "", "```", args.command, "```", "",
           "Per-kernel durations over every launch of that run:", "",
           "| kernel | calls | mean µs | min µs | max µs | share |", "|---|---|---|---|---|---|"]
    for name, calls, avg, mn, mx, pct in rows:
        out.append(f"| `{name}` | {calls} | {avg:.2f} | {mn:.2f} | {mx:.2f} | {pct:.1f}% |")
    if bench is not None:
        out += ["", "The bench line (HIP events stamped by each kernel's dispatch, mean µs per launch) of the "
                "same workload without the profiler:", "", "```", args.bench_command, "```", "", "```",
                json.dumps({k: bench[k] for k in keep if k in bench}), "```"]
    if args.note:
        out += ["", args.note]
    path = os.path.join(ROOT, "profiles", f"kernel_stats_{wname}.md")
    with open(path, "w") as f:
        f.write("\n".join(out) + "\n")
    print(path)


def pmc(args):
    sys.path.insert(0, ROOT)
    from bebelm_amd import synth

    cfg = synth.CONFIGS[args.config]
    # kernel -> counter -> per-dispatch totals (a dispatch's rows, one per XCD / SE instance,
    # are summed)
    per = collections.defaultdict(lambda: collections.defaultdict(lambda: collections.defaultdict(float)))
    names = {}
    for path in args.csv:
        with open(path) as f:
            for row in csv.DictReader(f):
                k = row["Kernel_Name"]
                if not any(s in k for s in args.kernels):
                    continue
                short = k.split("(")[0]
                names[short] = k
                per[short][row["Counter_Name"]][row.get("Dispatch_Id", "?")] += float(row["Counter_Value"])
    lines = [f"# PMC counters — config {args.config} ({cfg.name}): {cfg.description}", "",
             "Commands (from the repository root on one MI355X; `cd /tmp && export TMPDIR=/tmp` first), one "
             "`rocprofv3 --pmc` pass each:", "", "```"] + list(args.commands) + ["```", "",
             "Mean per dispatch (each dispatch's rows summed over the counter's hardware instances):", ""]
    for short, counters in sorted(per.items()):
        mean = {c: sum(v.values()) / max(1, len(v)) for c, v in counters.items()}
        n = max(len(v) for v in counters.values())
        lines += [f"## `{short}` ({n} dispatches)", "", "| counter | per dispatch |", "|---|---|"]
        for c in sorted(mean):
            lines.append(f"| {c} | {mean[c]:,.0f} |")
        waves = mean.get("SQ_WAVES")
        derived = []
        if "SQ_INSTS_VALU" in mean and "SQ_INSTS_MFMA" in mean and mean["SQ_INSTS_MFMA"]:
            derived.append(f"VALU : MFMA instructions = {mean['SQ_INSTS_VALU'] / mean['SQ_INSTS_MFMA']:.2f}")
        if waves:
            for c in ("SQ_INSTS_VALU", "SQ_INSTS_MFMA", "SQ_INSTS_LDS", "SQ_INSTS_SALU"):
                if c in mean:
                    derived.append(f"{c} per wave = {mean[c] / waves:,.0f}")
        if "SQ_VALU_MFMA_BUSY_CYCLES" in mean and "SQ_BUSY_CYCLES" in mean and mean["SQ_BUSY_CYCLES"]:
            derived.append(f"SQ_VALU_MFMA_BUSY_CYCLES / SQ_BUSY_CYCLES = "
                           f"{mean['SQ_VALU_MFMA_BUSY_CYCLES'] / mean['SQ_BUSY_CYCLES']:.2f}")
        if derived:
            lines += [""] + [f"* {d}" for d in derived]
        lines.append("")
    if args.note:
        lines += [args.note, ""]
    path = os.path.join(ROOT, "profiles", f"pmc_{cfg.name}.md")
    with open(path, "w") as f:
        f.write("\n".join(lines))
    print(path)


def main():
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    d = sub.add_parser("drive")
    d.add_argument("--config", type=int, default=2)
    d.add_argument("--steps", type=int, default=48)
    d.add_argument("--layers", type=int, default=12)
    d.add_argument("--decoder", action="store_true", help="the whole decoder at full size instead of one MoE block")
    t = sub.add_parser("traffic")
    t.add_argument("--fetch", required=True)
    t.add_argument("--write", required=True)
    t.add_argument("--kernel", required=True, help="substring of the kernel name")
    t.add_argument("--name", default=None, help="name used in the output file (default: --kernel)")
    t.add_argument("--config", type=int, default=2)
    t.add_argument("--command-fetch", default=None)
    t.add_argument("--command-write", default=None)
    st = sub.add_parser("stats")
    st.add_argument("--csv", required=True)
    st.add_argument("--bench", default=None)
    st.add_argument("--config", type=int, default=2)
    st.add_argument("--decoder", action="store_true")
    st.add_argument("--command", required=True)
    st.add_argument("--bench-command", default=None)
    st.add_argument("--note", default=None)
    pm = sub.add_parser("pmc")
    pm.add_argument("--csv", nargs="+", required=True)
    pm.add_argument("--commands", nargs="+", required=True)
    pm.add_argument("--kernels", nargs="+", default=["k_gemm"])
    pm.add_argument("--config", type=int, default=4)
    pm.add_argument("--note", default=None)
    args = ap.parse_args()
    {"drive": drive, "traffic": traffic, "stats": stats, "pmc": pmc}[args.cmd](args)


if __name__ == "__main__":
    main()
