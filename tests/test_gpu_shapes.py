"""GPU parity over a seeded sweep of small MoE shapes: hidden and ff widths, 1 to 32 experts,
k from 1 to min(8, E), 1 to 40 tokens, Q4_K/Q6_K gate/up and down, each case on every path
the library chooses between (the per-expert GEMVs with the route inside the gate/up kernel or
in its own kernel, the one-token down GEMV with the combine, the grouped GEMMs). The bar is the
rest of the suite's: routing, weights and block outputs bit-identical to the CPU restatement
of Model::moe_ffn / moe_ffn_batch (model.rs:286-371, 473-556).
"""
import numpy as np
import pytest

from bebelm_amd import synth

from test_gpu_parity import Q4_K, Q6_K, check_moe

pytestmark = pytest.mark.gpu

DEFAULT_MIN_ENTRIES = 64


def _cases(n=16, seed=2024):
    g = np.random.default_rng(seed)
    out = []
    for i in range(n):
        hidden = int(g.choice([256, 512, 768, 1024]))
        ff = int(g.choice([256, 512, 1024, 1792]))
        E = int(g.choice([1, 2, 3, 5, 8, 13, 16, 32]))
        K = int(g.integers(1, min(8, E) + 1))
        T = int(g.choice([1, 2, 3, 4, 5, 9, 16, 17, 40]))
        gdt = int(g.choice([Q4_K, Q6_K]))
        ddt = int(g.choice([Q4_K, Q6_K]))
        out.append((i, hidden, ff, E, K, T, gdt, ddt))
    # one token with k <= 4 (the down GEMV that also combines), the widest rows, k = E
    out += [(n, 768, 512, 8, 4, 1, Q6_K, Q6_K), (n + 1, 512, 1792, 32, 2, 1, Q4_K, Q6_K),
            (n + 2, 2048, 256, 5, 3, 1, Q4_K, Q4_K), (n + 3, 256, 256, 32, 8, 13, Q6_K, Q4_K),
            (n + 4, 2048, 2048, 4, 4, 6, Q4_K, Q6_K)]
    return out


@pytest.mark.parametrize("path", ["gemv", "batched"])
@pytest.mark.parametrize("case", _cases(), ids=lambda c: f"c{c[0]}-H{c[1]}-F{c[2]}-E{c[3]}-k{c[4]}-T{c[5]}")
def test_random_shapes(gpu_ctx, oracle, case, path):
    i, hidden, ff, E, K, T, gdt, ddt = case
    if path == "batched" and E * K < 2:
        pytest.skip("one expert of one slot: the batched path equals the GEMV path here")
    w = synth.moe_weights(300 + i, hidden=hidden, moe_ff=ff, n_experts=E, n_used=K, gate_dtype=gdt, down_dtype=ddt)
    x = synth.hidden_states(400 + i, T, hidden=hidden)
    gpu_ctx.set_batched_min_entries(1 if path == "batched" else 1 << 40)
    try:
        check_moe(gpu_ctx, oracle, w, x, T, f"case {i} {path}")
    finally:
        gpu_ctx.set_batched_min_entries(DEFAULT_MIN_ENTRIES)
