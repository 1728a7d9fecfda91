"""The committed golden fixtures (tests/golden/moe_config*.json) against a fresh regeneration:
the seeded generator must reproduce the same input bytes and the CPU restatement the same route,
selection margins and block output, bit for bit. Configs 1-3 here; config 4 (4096 tokens) and
config 5 (the 24-layer stack, ~4.75 GB of weights) in the slow group."""
import json
import os

import pytest

from golden import make_fixtures as mf

HERE = os.path.dirname(os.path.abspath(__file__))


def load(c):
    with open(os.path.join(HERE, "golden", f"moe_config{c}.json")) as f:
        return json.load(f)


@pytest.mark.parametrize("c", [1, 2, 3, pytest.param(4, marks=pytest.mark.slow), pytest.param(5, marks=pytest.mark.slow)])
def test_fixture_regenerates(oracle, c):
    want = load(c)
    got = json.loads(json.dumps(mf.fixture(oracle, c)))
    assert got["inputs_sha256"] == want["inputs_sha256"], "generator output changed"
    assert got == want


def test_fixture_shapes():
    for c in (1, 2, 3, 4):
        fx = load(c)
        assert fx["output"]["n"] == fx["tokens"] * fx["shape"]["hidden"]
        assert sum(fx["route"]["counts"]) == fx["tokens"] * fx["shape"]["top_k"]
        assert fx["route"]["offsets"][-1] == sum(fx["route"]["counts"])
        assert fx["route"]["ties"] == 0
        assert fx["margin"]["min"] > 0
    fx = load(5)
    assert fx["shape"]["layers"] == 24 and fx["shape"]["dense_layers"] == 2
    assert [L["layer"] for L in fx["layers"]] == list(range(2, 24))
    assert all(len(L["sel"]) == fx["shape"]["top_k"] and L["margin"]["min"] > 0 for L in fx["layers"])
    assert fx["output"]["n"] == fx["shape"]["hidden"]
