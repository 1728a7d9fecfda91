"""Writes the golden fixtures of BASELINE.json configs 1-5 (tests/golden/moe_config*.json).

The reference holds no golden vectors for this path (its golden prompt needs the GGUF), so the
fixtures pin this build's own generator and CPU restatement: per config the seed, SHA-256 of
the generated inputs (router, bias, expert bytes, hidden states), the restatement's route
trace (selections, weights, counts, offsets, the dispatch permutation's hash), the smallest
selection margin key[k-1] - key[k] over the tokens, and the block output (hash of all bytes
plus the first and last 16 values). Config 5 (the 24-layer FFN stack at one token) records the
route and margin of each of its 22 MoE layers and the stack's output.

    python3 tests/golden/make_fixtures.py          # rewrites the five JSON files

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

CONFIGS = (1, 2, 3, 4, 5)
SEED = 0


def sha(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def inputs(cfg_id):
    cfg = synth.CONFIGS[cfg_id]
    w = synth.stack_layers(seed=SEED) if cfg_id == 5 else synth.config_layer(cfg_id, seed=SEED, layer=0)
    x = synth.hidden_states(SEED, cfg.tokens)
    return cfg, w, x


def stack_hashes(layers, x):
    """One hash per tensor kind over the stack's layers in order (gains, dense and MoE tensors)."""
    moe = [w for _, w in layers if isinstance(w, synth.MoeWeights)]
    dense = [w for _, w in layers if not isinstance(w, synth.MoeWeights)]
    return {
        "ffn_norm": sha(*[g for g, _ in layers]),
        "dense": sha(*[a for d in dense for a in (d.gate, d.up, d.down)]),
        "router": sha(*[w.router for w in moe]),
        "exp_probs_b": sha(*[w.exp_probs_b for w in moe]),
        "gate_exps": sha(*[w.gate_exps for w in moe]),
        "up_exps": sha(*[w.up_exps for w in moe]),
        "down_exps": sha(*[w.down_exps for w in moe]),
        "x": sha(x),
    }


def stack_routes(oracle, layers, x, t, eps=synth.RMS_EPS):
    """run_layers' FFN path (model.rs:105-130) layer by layer on the CPU restatement: the output
    and, per MoE layer, (layer index, its input rows, its route trace)."""
    H = layers[0][1].hidden
    h = np.ascontiguousarray(x, np.float32).reshape(t, H).copy()
    routes = []
    for li, (g, w) in enumerate(layers):
        normed = np.stack([oracle.rmsnorm(h[i], g, eps) for i in range(t)])
        if isinstance(w, synth.MoeWeights):
            y, tr = route_and_output(oracle, w, normed, t)
            routes.append((li, normed, tr))
        else:
            y = oracle.dense_ffn(w, normed.reshape(-1), t)
        h = h + np.asarray(y, np.float32).reshape(t, H)
    return h.reshape(-1), routes


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


def output_summary(y):
    y = np.asarray(y, np.float32).reshape(-1)
    return {
        "sha256": sha(y),
        "head_bits": y[:16].view(np.uint32).tolist(),
        "tail_bits": y[-16:].view(np.uint32).tolist(),
        "n": int(y.size),
    }


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
        "output": output_summary(y),
    }


def margin_summary(tr):
    m = np.asarray(tr.margin, np.float32)
    i = int(np.argmin(m))
    return {"min": float(m[i]), "min_bits": int(m[i:i + 1].view(np.uint32)[0]), "token": i}


def stack_fixture(oracle, cfg, layers, x):
    t = cfg.tokens
    y, routes = stack_routes(oracle, layers, x, t)
    whole = oracle.ffn_stack(layers, x.reshape(-1), t)
    assert np.array_equal(y.view(np.uint32), whole.view(np.uint32)), "layer-by-layer stack differs from ffn_stack"
    w0 = next(w for _, w in layers if isinstance(w, synth.MoeWeights))
    return {
        "config": 5,
        "workload": cfg.name,
        "seed": SEED,
        "tokens": t,
        "shape": {"hidden": w0.hidden, "moe_ff": w0.moe_ff, "experts": w0.n_experts, "top_k": w0.n_used,
                  "layers": len(layers), "dense_layers": sum(not isinstance(w, synth.MoeWeights) for _, w in layers),
                  "dense_ff": next(w.ff for _, w in layers if not isinstance(w, synth.MoeWeights))},
        "inputs_sha256": stack_hashes(layers, x),
        "layers": [{"layer": li, "sel": tr.sel.tolist(), "w_bits": tr.w.view(np.uint32).tolist(),
                    "logits_sha256": sha(tr.logits.astype(np.float32)), "margin": margin_summary(tr)}
                   for li, _, tr in routes],
        "margin": {"min": min(float(np.min(tr.margin)) for _, _, tr in routes)},
        "output": output_summary(y),
    }


def fixture(oracle, cfg_id):
    cfg, w, x = inputs(cfg_id)
    if cfg_id == 5:
        return stack_fixture(oracle, cfg, w, x)
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
        "margin": margin_summary(tr),
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
        print(f"config {c}: output {fx['output']['sha256'][:16]}… min margin {fx['margin']['min']:.3e}")


if __name__ == "__main__":
    main()
