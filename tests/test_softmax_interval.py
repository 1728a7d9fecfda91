"""The rule by which the GPU softmax (wave_softmax in bebelm_amd/csrc/bb_ops.hip) takes the
reference's normaliser inv = (float)(1 / sum) without the one-lane chain of f64 adds
(softmax.rs:14-17), restated in numpy and checked on the CPU: a tree sum S_t of the same
summands (64 lanes, each lane's elements in order, then a butterfly), the interval
[S_t - B, S_t + B] with B = (n + 64)·2^-51·S_t, and inv decided when both ends give the same
float. Wherever the rule decides, its inv must equal the chain's; the row lengths the GPU tests
use to reach the chain (rows of equal scores, whose sum n is exact) must be undecided.
"""
import numpy as np
import pytest

# three of the 17 lengths <= 41,000 at which rows of equal scores reach the chain (one past the
# 40,000 positions a row may take in LDS)
EQUAL_ROW_FALLBACK = (21324, 33825, 40880)


def chain_inv(e):
    s = 0.0
    for v in e.astype(np.float64):
        s += v
    return np.float32(1.0 / s)


def tree_sum(e):
    n = e.size
    lanes = np.zeros(64)
    for l in range(64):
        acc = 0.0
        for v in e[l::64].astype(np.float64):
            acc += v
        lanes[l] = acc
    o = 1
    while o < 64:
        lanes = lanes + lanes[np.arange(64) ^ o]
        o <<= 1
    assert np.all(lanes == lanes[0])  # every lane holds the same sum
    return float(lanes[0])


def decided_inv(e):
    st = tree_sum(e)
    b = float(e.size + 64) * 2.0**-51 * st
    lo, hi = np.float32(1.0 / (st - b)), np.float32(1.0 / (st + b))
    return lo if lo == hi else None


def exps(scores):
    s = scores.astype(np.float32)
    return np.exp((s - s.max()).astype(np.float32)).astype(np.float32)


@pytest.mark.parametrize("n", [1, 2, 63, 64, 65, 300, 1000, 4097])
def test_rule_agrees_with_the_chain(n):
    g = np.random.default_rng(n)
    undecided = 0
    for trial in range(40):
        kind = trial % 4
        if kind == 0:
            x = g.standard_normal(n) * 5
        elif kind == 1:
            x = g.standard_normal(n) * 40  # most exps tiny: the chain rounds often
        elif kind == 2:
            x = np.where(g.random(n) < 0.5, 0.0, -15.0 + g.random(n))
        else:
            x = g.uniform(-1e-3, 1e-3, n)  # exps near 1: sums near n
        e = exps(x)
        inv = decided_inv(e)
        if inv is None:
            undecided += 1
            continue
        assert inv.view(np.uint32) == chain_inv(e).view(np.uint32), (n, trial)
    assert undecided <= 2


def test_equal_rows_reach_the_chain_at_the_listed_lengths():
    found = []
    for n in range(1, 41001):
        st = float(n)  # every exp is 1.0: all sums are exact
        b = float(n + 64) * 2.0**-51 * st
        if np.float32(1.0 / (st - b)) != np.float32(1.0 / (st + b)):
            found.append(n)
    assert set(EQUAL_ROW_FALLBACK) <= set(found) and len(found) == 17
    for n in EQUAL_ROW_FALLBACK:
        assert decided_inv(np.ones(n, np.float32)) is None
