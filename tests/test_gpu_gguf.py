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
    gm = Model.load(gpu_ctx, path, validate=False)
    dm = Model(gpu_ctx, mw)
    gc, dc = gm.new_cache(800), dm.new_cache(800)
    om = bbo.Model(mw, 800)
    try:
        ids = list(np.random.default_rng(2).integers(0, mw.vocab, 600))
        log("GGUF small model: absorb 600 tokens")
        gm.absorb(gc, ids, max_context=700)
        dm.absorb(dc, ids, max_context=700)
        om.absorb(ids, max_context=700)
        assert gc.pos == om.pos == 600
        check_caches(gc, om, "GGUF model after absorb")
        for step, tok in enumerate((3, 456)):
            log(f"GGUF small model: forward_step {step}")
            want = om.forward_step(tok)
            check(gm.forward_step(tok, gc), want, f"GGUF logits step {step}")
            check(dm.forward_step(tok, dc), want, f"in-memory logits step {step}")
        gc.reset()
        check(gm.run_layers([5, 6], gc), bbo.Model(mw, 8).run_layers([5, 6]), "GGUF model after reset")
    finally:
        gc.close()
        dc.close()
        gm.close()
        dm.close()


def test_validate_gates_the_load(gpu_ctx, tmp_path):
    path = tmp_path / "small.gguf"
    synth.model_gguf(small_weights()).save(path)
    with pytest.raises(gguf.BBError, match="lfm2moe.block_count: expected 24, got 6"):
        Model.load(gpu_ctx, path)                # validate=True pins LFM2.5-8B-A1B's constants


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
        gm = Model.load(gpu_ctx, g)
    os.remove(path)
    gc = gm.new_cache(64)
    om = bbo.Model(mw, 64)
    try:
        ids = [2, 77, 127000, 9]
        log("full-size GGUF: prefill 4 tokens")
        check(gm.run_layers(ids, gc), om.run_layers(ids), "prefill hidden states")
        log("full-size GGUF: forward_step")
        check(gm.forward_step(31, gc), om.forward_step(31), "logits")
        check_caches(gc, om, "full size from GGUF")
    finally:
        gc.close()
        gm.close()


def test_load_rejects_bad_files(gpu_ctx):
    # Model::load's failures (model.rs:36-67, :572-584) come back as error codes with the
    # reference's messages, before or during the upload, and leave nothing behind
    from bebelm_amd import _lib

    mw = small_weights()
    w = synth.model_gguf(mw)
    w.tensors = [t for t in w.tensors if t[0] != "blk.4.attn_k.weight"]
    with pytest.raises(gguf.BBError, match="missing tensor blk.4.attn_k.weight") as e:
        Model.load(gpu_ctx, gguf.GgufFile.from_bytes(w.to_bytes()), validate=False)
    assert e.value.code == _lib.BB_ERR_MISSING

    w = synth.model_gguf(mw)
    i = [t[0] for t in w.tensors].index("blk.0.attn_norm.weight")
    name, dims, ty, data = w.tensors[i]
    w.tensors[i] = (name, dims, synth.F16, np.zeros(dims[0], np.float16))
    with pytest.raises(gguf.BBError, match="f32 tensor not precomputed: blk.0.attn_norm.weight") as e:
        Model.load(gpu_ctx, gguf.GgufFile.from_bytes(w.to_bytes()), validate=False)
    assert e.value.code == _lib.BB_ERR_DTYPE

    w = synth.model_gguf(mw)
    i = [t[0] for t in w.tensors].index("blk.5.ffn_up_exps.weight")
    name, dims, ty, data = w.tensors[i]
    w.tensors[i] = (name, [dims[0], dims[1] // 2, dims[2] * 2], ty, data)
    with pytest.raises(gguf.BBError, match=r"tensor blk.5.ffn_up_exps.weight: shape \[512, 256, 16\] != expected"):
        Model.load(gpu_ctx, gguf.GgufFile.from_bytes(w.to_bytes()), validate=False)
    # the context still works
    gm = Model.load(gpu_ctx, gguf.GgufFile.from_bytes(synth.model_gguf(mw).to_bytes()), validate=False)
    gc = gm.new_cache(16)
    try:
        assert gm.run_layers([1, 2], gc).shape == (2 * mw.hidden,)
    finally:
        gc.close()
        gm.close()
