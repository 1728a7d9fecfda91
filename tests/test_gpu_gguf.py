"""A decoder loaded from a GGUF file (bb_model_load: Model::load, model.rs:36-50, with every tensor
uploaded from the file's mapping into HBM) against the CPU restatement and against the decoder
built from the same weights in memory. The bar is bit-exactness, as for the decoder itself."""
import os

import numpy as np
import pytest

from bebelm_amd import gguf, synth
from bebelm_amd.model import Model
from oracle import bbo

from test_gpu_model import check, check_caches, small_weights
from test_gpu_parity import log

pytestmark = pytest.mark.gpu


def test_small_model_from_gguf(gpu_ctx, tmp_path):
    mw = small_weights()
    path = tmp_path / "small.gguf"
    synth.model_gguf(mw).save(path)
    gm = Model.load(gpu_ctx, path, 800, validate=False)
    dm = Model(gpu_ctx, mw, 800)
    om = bbo.Model(mw, 800)
    try:
        ids = list(np.random.default_rng(2).integers(0, mw.vocab, 600))
        log("GGUF small model: absorb 600 tokens")
        gm.absorb(ids, max_context=700)
        dm.absorb(ids, max_context=700)
        om.absorb(ids, max_context=700)
        assert gm.pos == om.pos == 600
        check_caches(gm, om, "GGUF model after absorb")
        for step, tok in enumerate((3, 456)):
            log(f"GGUF small model: forward_step {step}")
            want = om.forward_step(tok)
            check(gm.forward_step(tok), want, f"GGUF logits step {step}")
            check(dm.forward_step(tok), want, f"in-memory logits step {step}")
        gm.reset()
        check(gm.run_layers([5, 6]), bbo.Model(mw, 8).run_layers([5, 6]), "GGUF model after reset")
    finally:
        gm.close()
        dm.close()


def test_validate_gates_the_load(gpu_ctx, tmp_path):
    path = tmp_path / "small.gguf"
    synth.model_gguf(small_weights()).save(path)
    with pytest.raises(gguf.BBError, match="lfm2moe.block_count: expected 24, got 6"):
        Model.load(gpu_ctx, path, 16)            # validate=True pins LFM2.5-8B-A1B's constants


def test_full_size_model_from_gguf(gpu_ctx, tmp_path):
    log("full-size GGUF: generating weights")
    mw = synth.model_weights(seed=1)
    path = tmp_path / "full.gguf"
    log("full-size GGUF: writing the file")
    synth.model_gguf(mw).save(path)
    log(f"full-size GGUF: {os.path.getsize(path) / 1e9:.2f} GB; open, validate, load")
    with gguf.GgufFile.open(path) as g:
        g.validate()
        assert g.check_tensors() == 256
        gm = Model.load(gpu_ctx, g, 64)
    os.remove(path)
    om = bbo.Model(mw, 64)
    try:
        ids = [2, 77, 127000, 9]
        log("full-size GGUF: prefill 4 tokens")
        check(gm.run_layers(ids), om.run_layers(ids), "prefill hidden states")
        log("full-size GGUF: forward_step")
        check(gm.forward_step(31), om.forward_step(31), "logits")
        check_caches(gm, om, "full size from GGUF")
    finally:
        gm.close()
