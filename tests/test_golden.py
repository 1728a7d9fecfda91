"""The committed golden fixtures (tests/golden/moe_config*.json) against a fresh regeneration:
the seeded generator must reproduce the same input bytes and the CPU restatement the same route
and block output, bit for bit. Configs 1-3 here; config 4 (4096 tokens) in the slow group."""
import json
import os

import numpy as np
import pytest

from golden import make_fixtures as mf

HERE = os.path.dirname(os.path.abspath(__file__))


def load(c):
    with open(os.path.join(HERE, "golden", f"moe_config{c}.json")) as f:
        return json.load(f)


@pytest.mark.parametrize("c", [1, 2, 3, pytest.param(4, marks=pytest.mark.slow)])
def test_fixture_regenerates(oracle, c):
    want = load(c)
    got = mf.fixture(oracle, c)
    assert got["inputs_sha256"] == want["inputs_sha256"], "generator output changed"
    assert got["route"] == want["route"]
    assert got["output"] == want["output"]


def test_fixture_shapes():
    for c in (1, 2, 3, 4):
        fx = load(c)
        assert fx["output"]["n"] == fx["tokens"] * fx["shape"]["hidden"]
        assert sum(fx["route"]["counts"]) == fx["tokens"] * fx["shape"]["top_k"]
        assert fx["route"]["offsets"][-1] == sum(fx["route"]["counts"])
        assert fx["route"]["ties"] == 0
