"""Every address the grouped-GEMM launches can touch, checked on the CPU (tests/gemm_address_model.py).

For the shapes the GPU tests run (the seeded sweep of small shapes, the
edge cases of tests/test_gpu_shapes.py, tests/test_gpu_gateup16.py and tests/test_gpu_wide.py,
and the shape at which a since-removed k_gemm_wide variant faulted: T = 400, hidden = ff = 512,
Q6_K down), under uniform, skewed and degenerate routings, the model of launch_gemm's choice and
of each kernel's tile, member-row, copy and store arithmetic must find
  * every weight, activation and scale copy (or buffer-resource range) inside its buffer,
  * every member row inside the quantised input, every store inside the output,
  * every output of a real member written exactly once.
"""
import numpy as np
import pytest

import gemm_address_model as am
from gemm_address_model import DOWN, GATEUP, Q4_K, Q6_K, Shape


def routing(kind, T, E, K, seed):
    g = np.random.default_rng(seed)
    if kind == "uniform":
        return np.stack([g.permutation(E)[:K] for _ in range(T)])
    if kind == "zipf":
        p = np.arange(1, E + 1, dtype=np.float64) ** -1.2
        p /= p.sum()
        return np.stack([g.choice(E, K, replace=False, p=p) for _ in range(T)])
    if kind == "same":  # every token picks experts 0..K-1: one giant group per chosen expert
        return np.tile(np.arange(K), (T, 1))
    if kind == "last":  # only the highest expert ids (the empty experts come first)
        return np.tile(np.arange(E - K, E), (T, 1))
    raise ValueError(kind)


def run(dt_gu, dt_dn, T, H, F, E, K, kinds=("uniform", "zipf", "same", "last"), seed=0):
    seen = set()
    for kind in kinds:
        if kind == "zipf" and E < 2:
            continue
        sel = routing(kind, T, E, K, seed)
        for s in (Shape(dt_gu, GATEUP, T, H, F, E, K), Shape(dt_dn, DOWN, T, F, H, E, K)):
            choice, v = am.check(s, sel)
            seen.add(choice)
            assert not v, (f"{'gate/up' if s.kind == GATEUP else 'down'} {choice} T={T} H={H} F={F} E={E} K={K} "
                           f"routing {kind}: {v[:5]}")
    return seen


@pytest.mark.parametrize("T", [1, 4, 16])
def test_decode_configs(T):
    # configs 1 and 2 and the stack's decode batches: k_gateup16 / member tiles of 16
    assert run(Q4_K, Q4_K, T, 2048, 1792, 32, 4) <= {"gemm", "gateup16"}
    run(Q4_K, Q6_K, T, 2048, 1792, 32, 4)


def test_prefill_config3():
    assert "gemm" in run(Q4_K, Q4_K, 512, 2048, 1792, 32, 4, kinds=("uniform", "same"))


@pytest.mark.slow
def test_prefill_config4():
    # Zipf-skewed 4096 tokens: Q4_K gate/up on member tiles of 80, Q6_K down on k_gemm_wide
    assert "wide" in run(Q4_K, Q6_K, 4096, 2048, 1792, 32, 4, kinds=("zipf", "uniform"))


def test_shape_of_the_removed_wide_variant():
    # T = 400, hidden = ff = 512, Q6_K down (the shape at which the removed variant faulted)
    seen = set()
    for E, K in ((8, 4), (4, 4), (8, 2)):
        seen |= run(Q4_K, Q6_K, 400, 512, 512, E, K)
    assert "wide" in seen


@pytest.mark.parametrize("T,E,K", [(1, 1, 1), (3, 1, 1), (33, 1, 1), (200, 1, 1), (64, 16, 16), (16, 8, 8),
                                   (7, 16, 3), (300, 8, 1), (40, 32, 8), (2, 32, 1)])
def test_edge_shapes(T, E, K):
    for dts in ((Q4_K, Q4_K), (Q4_K, Q6_K), (Q6_K, Q6_K)):
        run(dts[0], dts[1], T, 512, 512, E, K)


def test_seeded_sweep_shapes():
    # the shapes of the GPU sweep: hidden 256-2048, ff 256-2048, 1-32 experts, k <= min(8, E),
    # 1-40 tokens, Q4_K/Q6_K mixes
    g = np.random.default_rng(2024)
    for i in range(40):
        H = int(g.choice([256, 512, 1024, 2048]))
        F = int(g.choice([256, 512, 768, 1792, 2048]))
        E = int(g.integers(1, 33))
        K = int(g.integers(1, min(8, E) + 1))
        T = int(g.integers(1, 41))
        dg, dd = (Q4_K, Q6_K)[int(g.integers(2))], (Q4_K, Q6_K)[int(g.integers(2))]
        run(dg, dd, T, H, F, E, K, kinds=("uniform", "same"), seed=i)


def test_model_catches_a_planted_mistake():
    # the model must notice a launch that reads past its buffer: shrink the packed expert size it
    # checks against (a stride one tile-block short) and every weight range of the last expert fails
    s = Shape(Q4_K, DOWN, 64, 512, 512, 8, 4)
    sel = routing("uniform", 64, 8, 4, 1)
    _, v = am.check(s, sel)
    assert not v
    short = Shape(Q4_K, DOWN, 64, 512, 512, 8, 4)
    short.__class__ = type("ShortShape", (Shape,), {"stride": property(lambda self: Shape.stride.fget(self) - am.TB[Q4_K])})
    _, v = am.check(short, sel)
    assert v and any("weights" in x or "resource" in x for x in v)
