"""Routing robustness: the selected experts must not depend on the router dot's evaluation order.

The reference's router dot (matmul.rs:36-66) reduces its lanes inside the `wide` 0.7.33 crate,
which /root/reference does not vendor, and its CI also builds for x86-64-v2, where `mul_add`
is a rounded multiply and an add (.github/workflows/ci.yml:28-35). The restatement (and the
GPU) assume FMA chains and the AVX reduce tree; the last bits of a logit are therefore not
pinned by the reference. What must hold is that the routing does not depend on them: for every
token of BASELINE configs 1-5, the gating of model.rs:485-495 applied to the logits of each
plausible evaluation order (oracle.DOT_VARIANTS: FMA or not, each with the AVX tree and the
pairwise fold, lanes left to right, and the once-rounded f64 sum) selects the same experts in the same order.

The test also states the margin this rests on: the smallest selection margin key[k-1] - key[k]
recorded in the golden fixtures, against the largest change of any key between orders.
"""
import json
import os

import numpy as np
import pytest

from bebelm_amd import synth
from golden import make_fixtures as mf

HERE = os.path.dirname(os.path.abspath(__file__))
VARIANTS = (0, 1, 2, 3, 4, 5, 6)


def keys(logits, bias):
    s = (np.float32(1.0) / (np.float32(1.0) + np.exp(-logits.astype(np.float32)))).astype(np.float32)
    return s + bias.astype(np.float32)


def check_orders(oracle, w, x, t, what):
    sel0 = None
    key0 = None
    spread = 0.0
    logit_spread = 0.0
    logits0 = None
    for v in VARIANTS:
        logits = oracle.router_logits_variant(w, x, t, v)
        sel, _, ties, margin = oracle.gate(logits, w.exp_probs_b, w.n_used)
        assert ties == 0, f"{what}: exactly equal keys under order {v}"
        k = keys(logits, w.exp_probs_b)
        if sel0 is None:
            sel0, key0, logits0, margin0 = sel, k, logits, margin
            continue
        bad = np.nonzero(np.any(sel != sel0, axis=1))[0]
        assert bad.size == 0, (f"{what}: order {v} ({oracle.DOT_VARIANTS[v]}) selects other experts for tokens "
                               f"{bad[:8].tolist()} (margins {margin0[bad[:8]].tolist()})")
        spread = max(spread, float(np.max(np.abs(k - key0))))
        logit_spread = max(logit_spread, float(np.max(np.abs(logits - logits0))))
    return float(np.min(margin0)), spread, logit_spread, logits0


def test_variant_zero_is_the_restatement(oracle):
    # order 0 is the dot every other oracle function uses; the other orders do change bits
    w = synth.config_layer(2, seed=0)
    x = synth.hidden_states(0, 16)
    _, tr = oracle.moe_ffn_batch(w, x, 16, trace=True)
    l0 = oracle.router_logits_variant(w, x, 16, 0)
    assert np.array_equal(l0.reshape(-1).view(np.uint32), tr.logits.view(np.uint32))
    for v in VARIANTS[1:]:
        lv = oracle.router_logits_variant(w, x, 16, v)
        assert np.count_nonzero(lv.view(np.uint32) != l0.view(np.uint32)) > 0, f"order {v} equals order 0"
    # and the orders are the dot they claim: the f64 form is within one rounding of the exact sum
    a, b = w.router[3], x[5]
    exact = float(np.dot(a.astype(np.float64), b.astype(np.float64)))
    assert abs(oracle.dot_variant(a, b, 5) - exact) <= abs(exact) * 2.0 ** -24 + 1e-30


@pytest.mark.parametrize("c", [1, 2, 3, pytest.param(4, marks=pytest.mark.slow)])
def test_routing_independent_of_dot_order(oracle, c):
    cfg, w, x = mf.inputs(c)
    m, spread, lspread, _ = check_orders(oracle, w, x, cfg.tokens, f"config {c}")
    with open(os.path.join(HERE, "golden", f"moe_config{c}.json")) as f:
        fx = json.load(f)
    assert np.float32(m) == np.float32(fx["margin"]["min"])
    print(f"config {c}: min margin {m:.3e}, largest key change between orders {spread:.3e} "
          f"(logits {lspread:.3e}), ratio {m / max(spread, 1e-30):.1f}")
    assert spread < m, "a key moved by more than the smallest margin"


@pytest.mark.slow
def test_stack_routing_independent_of_dot_order(oracle):
    cfg, layers, x = mf.inputs(5)
    _, routes = mf.stack_routes(oracle, layers, x, cfg.tokens)
    worst = np.inf
    for li, normed, tr in routes:
        w = layers[li][1]
        m, spread, _, logits0 = check_orders(oracle, w, normed, cfg.tokens, f"config 5 layer {li}")
        assert np.array_equal(logits0.reshape(-1).view(np.uint32), tr.logits.view(np.uint32))
        assert spread < m
        worst = min(worst, m / max(spread, 1e-30))
    print(f"config 5: smallest margin / key change over 22 MoE layers {worst:.1f}")
