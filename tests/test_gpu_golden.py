"""The HIP library against the committed golden fixtures (configs 1-4 at full size): the block
output's SHA-256 and boundary values, and the route (selections, weights, counts, offsets,
permutation), must match what the CPU restatement recorded."""
import json
import os

import numpy as np
import pytest

from bebelm_amd.model import MoeLayer, RouteTrace
from golden import make_fixtures as mf

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.parametrize("c", [1, 2, 3, 4])
def test_gpu_matches_golden(gpu_ctx, c):
    with open(os.path.join(HERE, "golden", f"moe_config{c}.json")) as f:
        want = json.load(f)
    cfg, w, x = mf.inputs(c)
    assert mf.input_hashes(w, x) == want["inputs_sha256"]
    print(f"golden config {c}: T={cfg.tokens}", flush=True)
    layer = MoeLayer(gpu_ctx, w)
    try:
        t = cfg.tokens
        tr = RouteTrace(t, w.n_experts, w.n_used)
        y = layer.forward(np.ascontiguousarray(x.reshape(-1)), t, np.empty(t * w.hidden, np.float32), tr)
        got = mf.summarize(np.asarray(y, np.float32), tr, t)
        assert got["route"] == want["route"]
        assert got["output"] == want["output"]
    finally:
        layer.close()
