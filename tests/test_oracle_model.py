"""The CPU restatement of the whole decoder (Model, model.rs:99-181, and Agent::absorb,
agent.rs:454-476) against the reference's own invariant (model.rs:668-705,
batched_prefill_matches_per_token): prefilling in one batch, in chunks, or token by token leaves
identical caches and identical next-token logits. Run on a small synthetic model (the GGUF the
reference's test loads is not available offline)."""
import numpy as np

from bebelm_amd import synth
from oracle import bbo


def small_model():
    return synth.model_weights(seed=3, hidden=256, vocab=300, n_layers=4, n_dense=1, attention_layers=(1,),
                               moe_ff=256, dense_ff=512, n_experts=8, n_heads=4, n_kv_heads=2)


def _caches(m):
    out = []
    for i in sorted(m.state):
        c = m.state[i]
        if isinstance(c, bbo.KvCache):
            out += [c.k[:c.n * c.kv_dim].copy(), c.v[:c.n * c.kv_dim].copy()]
        else:
            out.append(c.copy())
    return out


def test_batched_prefill_matches_per_token():
    mw = small_model()
    ids = [5, 17, 250, 3, 99, 42, 7]
    rest, last = ids[:-1], ids[-1]
    a = bbo.Model(mw, 16)
    for t in rest:
        a.run_layers([t])
    la = a.forward_step(last)
    for chunk in (len(rest), 3):
        b = bbo.Model(mw, 16)
        for i in range(0, len(rest), chunk):
            b.run_layers(rest[i:i + chunk])
        lb = b.forward_step(last)
        assert a.pos == b.pos
        for x, y in zip(_caches(a), _caches(b)):
            assert x.view(np.uint32).tolist() == y.view(np.uint32).tolist()
        assert la.view(np.uint32).tolist() == lb.view(np.uint32).tolist()
    assert np.all(np.isfinite(la)) and np.abs(la).max() > 0


def test_absorb_slides_the_window_token_by_token():
    # agent.rs:454-476: a batch that would overflow max_context runs token by token and trims
    mw = small_model()
    m = bbo.Model(mw, 16)
    m.absorb(list(range(10, 22)), max_context=8)
    assert m.pos == 12 and m.kv_len() == 8
    ref = bbo.Model(mw, 16)
    for t in range(10, 22):
        ref.run_layers([t])
        if ref.kv_len() > 8:
            ref.evict_front(ref.kv_len() - 8)
    for x, y in zip(_caches(m), _caches(ref)):
        assert x.view(np.uint32).tolist() == y.view(np.uint32).tolist()
