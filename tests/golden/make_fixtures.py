"""Writes the golden fixtures of the MoE block for BASELINE.json configs 1-4 (tests/golden/*.json).

The reference holds no golden vectors for this path (its golden prompt needs the GGUF), so the
fixtures pin this build's own generator and CPU restatement: per config the seed, SHA-256 of
the generated inputs (router, bias, expert bytes, hidden states), the restatement's route
trace (selections, weights, counts, offsets, the dispatch permutation's hash) and its block
output (hash of all bytes plus the first and last 16 values).

    python3 tests/golden/make_fixtures.py          # rewrites the four JSON files

tests/test_golden.py regenerates everything and compares (CPU); tests/test_gpu_golden.py checks
the HIP library against the files (GPU).
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from bebelm_amd import synth  # noqa: E402

CONFIGS = (1, 2, 3, 4)
SEED = 0


def sha(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def inputs(cfg_id):
    cfg = synth.CONFIGS[cfg_id]
    w = synth.config_layer(cfg_id, seed=SEED, layer=0)
    x = synth.hidden_states(SEED, cfg.tokens)
    return cfg, w, x


def input_hashes(w, x):
    return {
        "router": sha(w.router),
        "exp_probs_b": sha(w.exp_probs_b),
        "gate_exps": sha(w.gate_exps),
        "up_exps": sha(w.up_exps),
        "down_exps": sha(w.down_exps),
        "x": sha(x),
    }


def route_and_output(oracle, w, x, t):
    if t == 1:
        y, tr = oracle.moe_ffn(w, x.reshape(-1), trace=True)
    else:
        y, tr = oracle.moe_ffn_batch(w, x.reshape(-1), t, trace=True)
    return np.asarray(y, np.float32), tr


def summarize(y, tr, t):
    small = t <= 16
    return {
        "route": {
            "sel": tr.sel.tolist() if small else None,
            "sel_sha256": sha(tr.sel.astype(np.int32)),
            "w_bits": tr.w.view(np.uint32).tolist() if small else None,
            "w_sha256": sha(tr.w.astype(np.float32)),
            "logits_sha256": sha(tr.logits.astype(np.float32)),
            "counts": tr.counts.tolist(),
            "offsets": tr.offsets.tolist(),
            "perm_sha256": sha(tr.perm.astype(np.int32)),
            "ties": int(tr.ties[0]),
        },
        "output": {
            "sha256": sha(y),
            "head_bits": y[:16].view(np.uint32).tolist(),
            "tail_bits": y[-16:].view(np.uint32).tolist(),
            "n": int(y.size),
        },
    }


def fixture(oracle, cfg_id):
    cfg, w, x = inputs(cfg_id)
    y, tr = route_and_output(oracle, w, x, cfg.tokens)
    return {
        "config": cfg_id,
        "workload": cfg.name,
        "seed": SEED,
        "tokens": cfg.tokens,
        "shape": {"hidden": w.hidden, "moe_ff": w.moe_ff, "experts": w.n_experts, "top_k": w.n_used,
                  "gate_dtype": w.gate_dtype, "down_dtype": w.down_dtype},
        "inputs_sha256": input_hashes(w, x),
        **summarize(y, tr, cfg.tokens),
    }


def path(cfg_id):
    return os.path.join(HERE, f"moe_config{cfg_id}.json")


def main():
    from oracle import bbo

    bbo.build()
    bbo.set_threads(os.cpu_count() or 1)
    for c in CONFIGS:
        fx = fixture(bbo, c)
        with open(path(c), "w") as f:
            json.dump(fx, f, indent=1)
        print(f"config {c}: output {fx['output']['sha256'][:16]}… counts {fx['route']['counts'][:8]}…")


if __name__ == "__main__":
    main()
