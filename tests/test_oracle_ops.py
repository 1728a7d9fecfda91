"""Pins the CPU restatement of the decoder layer's operators (conv, softmax, attention, RoPE, the
conv and attention operators) against the reference's own unit tests and known answers:
src/kernels/conv.rs:77-144, softmax.rs:34-108, attention.rs:64-92, rope.rs:37-78, and the
batched-equals-per-token invariant of model.rs:668-705 (run on synthetic weights: the GGUF the
reference's test loads is not available offline).

Where the reference calls libm (f32 exp, sin, cos, powf), the restatement calls the same platform
functions; the RoPE test checks that bit for bit against libm through ctypes.
"""
import ctypes
import ctypes.util

import numpy as np
import pytest

from bebelm_amd import synth
from oracle import bbo


# ---- conv.rs:77-144 --------------------------------------------------------------------------

def test_conv_single_tap_is_pointwise():
    assert bbo.conv_step([], [3.0], [5.0], 1, 1).tolist() == [15.0]


def test_conv_causal_alignment_one_channel():
    # weight [w0 = 1 (oldest), w1 = 10, w2 = 100 (current)], state [2, 3], current 4 -> 432
    assert bbo.conv_step([2.0, 3.0], [4.0], [1.0, 10.0, 100.0], 1, 3).tolist() == [432.0]


def test_conv_zero_state_uses_only_current_tap():
    assert bbo.conv_step([0.0, 0.0], [4.0], [1.0, 10.0, 100.0], 1, 3).tolist() == [400.0]


def test_conv_per_channel_independent_layout():
    assert bbo.conv_step([10.0, 20.0], [1.0, 1.0], [1.0, 2.0, 3.0, 4.0], 2, 2).tolist() == [12.0, 64.0]


def test_conv_prefill_matches_rolling_conv_step():
    # conv.rs:105-131 with its exact data: 3 channels, l_cache 3, 5 positions
    C, L, n = 3, 3, 5
    w = np.array([(i - 4.0) * 0.5 for i in range(C * L)], np.float32)
    bx = np.array([((i % 7) - 3.0) * 0.3 for i in range(C * n)], np.float32)
    init = np.array([(i + 1.0) * 0.1 for i in range(C * (L - 1))], np.float32)
    state = init.copy()
    ref = []
    for t in range(n):
        ref.append(bbo.conv_step(state, bx[t * C:(t + 1) * C], w, C, L))
        state = np.concatenate([state[C:], bx[t * C:(t + 1) * C]])
    out, st = bbo.conv_prefill(init, bx, w, C, L, n)
    assert out.view(np.uint32).tolist() == np.concatenate(ref).view(np.uint32).tolist()
    assert st.view(np.uint32).tolist() == state.view(np.uint32).tolist()


def test_conv_step_is_the_spelled_out_sum():
    # out[c] = w[c, L-1]·bx[c] + w[c, 0]·s[0, c] + w[c, 1]·s[1, c], f32, in that order
    g = np.random.default_rng(3)
    C, L = 64, 3
    w = g.standard_normal(C * L).astype(np.float32)
    st = g.standard_normal(C * (L - 1)).astype(np.float32)
    bx = g.standard_normal(C).astype(np.float32)
    W = w.reshape(C, L)
    want = (W[:, 2] * bx + W[:, 0] * st[:C]) + W[:, 1] * st[C:]
    assert bbo.conv_step(st, bx, w, C, L).view(np.uint32).tolist() == want.astype(np.float32).view(np.uint32).tolist()


# ---- softmax.rs:34-108 -----------------------------------------------------------------------

def test_softmax_uniform_input_uniform_output():
    np.testing.assert_allclose(bbo.softmax([1.0, 1.0, 1.0, 1.0]), [0.25] * 4, atol=1e-7)


def test_softmax_known_distribution_sums_to_one():
    x = bbo.softmax([1.0, 2.0, 3.0])
    np.testing.assert_allclose(x, [0.09003057, 0.24472847, 0.66524096], atol=1e-6)
    assert abs(float(np.sum(x, dtype=np.float32)) - 1.0) < 1e-6


def test_softmax_stable_for_large_inputs():
    np.testing.assert_allclose(bbo.softmax([1000.0, 1000.0]), [0.5, 0.5], atol=1e-7)


def test_softmax_empty_is_noop():
    assert bbo.softmax([]).size == 0


def _peaked_logits(n):
    return np.array([0.0 if i < 16 else -15.0 + (i % 3) * 0.2 for i in range(n)], np.float32)


def test_softmax_sum_uses_wide_accumulator():
    # softmax.rs:77-108: against the f32 exps summed in f64 the error stays below 1e-6, while an
    # f32 accumulator drifts past it (the test is discriminating)
    libm = ctypes.CDLL(ctypes.util.find_library("m"))
    libm.expf.restype = ctypes.c_float
    libm.expf.argtypes = [ctypes.c_float]
    logits = _peaked_logits(4096)
    mx = np.float32(logits.max())
    exps = np.array([libm.expf(float(np.float32(v - mx))) for v in logits], np.float32)
    s64 = float(np.sum(exps.astype(np.float64)))
    ref = (exps.astype(np.float64) / s64).astype(np.float32)
    got = bbo.softmax(logits)
    rel = np.max(np.abs(got - ref) / np.maximum(np.abs(ref), 1e-9))
    assert rel < 1e-6
    s32 = np.float32(0.0)
    for e in exps:
        s32 = np.float32(s32 + e)
    regressed = np.max(np.abs(exps * np.float32(1.0 / s32) - ref) / np.maximum(np.abs(ref), 1e-9))
    assert regressed > 1e-6


def test_softmax_bits_follow_the_stated_order():
    # exps by libm expf, the f64 sum left to right, one f32 reciprocal of the f64 quotient
    libm = ctypes.CDLL(ctypes.util.find_library("m"))
    libm.expf.restype = ctypes.c_float
    libm.expf.argtypes = [ctypes.c_float]
    x = np.random.default_rng(5).standard_normal(300).astype(np.float32) * np.float32(4)
    mx = x.max()
    e = np.array([libm.expf(float(np.float32(v - mx))) for v in x], np.float32)
    s = 0.0
    for v in e:
        s += float(v)
    inv = np.float32(1.0 / s)
    assert bbo.softmax(x).view(np.uint32).tolist() == (e * inv).view(np.uint32).tolist()


# ---- attention.rs:64-92 ----------------------------------------------------------------------

def test_attention_single_context_returns_value():
    assert bbo.attention_decode([1.0, 0.0], [1.0, 0.0], [5.0, 7.0], 1, 1, 1, 2).tolist() == [5.0, 7.0]


def test_attention_averages_equal_scored_context():
    out = bbo.attention_decode([1.0, 0.0], [1.0, 0.0, 1.0, 0.0], [2.0, 0.0, 4.0, 0.0], 2, 1, 1, 2)
    assert abs(out[0] - 3.0) < 1e-6 and out[1] == 0.0


def test_attention_gqa_shares_kv_head():
    out = bbo.attention_decode([1.0, 0.0, 0.0, 1.0], [1.0, 1.0], [5.0, 7.0], 1, 2, 1, 2)
    assert out.tolist() == [5.0, 7.0, 5.0, 7.0]


def test_attention_matches_f64_brute_force():
    g = np.random.default_rng(7)
    n_ctx, nh, nkv, hd = 37, 8, 2, 64
    q = g.standard_normal(nh * hd).astype(np.float32)
    k = g.standard_normal(n_ctx * nkv * hd).astype(np.float32)
    v = g.standard_normal(n_ctx * nkv * hd).astype(np.float32)
    got = bbo.attention_decode(q, k, v, n_ctx, nh, nkv, hd)
    K = k.reshape(n_ctx, nkv, hd).astype(np.float64)
    V = v.reshape(n_ctx, nkv, hd).astype(np.float64)
    want = np.zeros((nh, hd))
    for h in range(nh):
        kv = h // (nh // nkv)
        s = K[:, kv] @ q[h * hd:(h + 1) * hd].astype(np.float64) / np.sqrt(hd)
        p = np.exp(s - s.max())
        want[h] = (p / p.sum()) @ V[:, kv]
    np.testing.assert_allclose(got.reshape(nh, hd), want, rtol=1e-5, atol=1e-5)
    # a wrong kv-head mapping (h % n_kv instead of h / group) would fail this
    wrong = np.zeros((nh, hd))
    for h in range(nh):
        kv = h % nkv
        s = K[:, kv] @ q[h * hd:(h + 1) * hd].astype(np.float64) / np.sqrt(hd)
        p = np.exp(s - s.max())
        wrong[h] = (p / p.sum()) @ V[:, kv]
    assert np.abs(got.reshape(nh, hd) - wrong).max() > 1e-2


# ---- rope.rs:37-78 ---------------------------------------------------------------------------

THETA = 5_000_000.0


def test_rope_position_zero_is_identity():
    orig = np.array([0.3, -1.2, 0.7, 2.5, -0.1, 0.9], np.float32)
    assert bbo.rope_neox(orig, 0, THETA).tolist() == orig.tolist()


def test_rope_rotates_first_pair_by_pos_radians():
    x = bbo.rope_neox([1.0, 0.0], 1, THETA)
    assert abs(x[0] - np.cos(1.0)) < 1e-6 and abs(x[1] - np.sin(1.0)) < 1e-6


def test_rope_pairs_split_half_not_interleaved():
    x = bbo.rope_neox([1.0, 0.0, 0.0, 0.0], 1, THETA)
    assert abs(x[0] - np.cos(1.0)) < 1e-6 and abs(x[2] - np.sin(1.0)) < 1e-6
    assert x[1] == 0.0 and x[3] == 0.0


def test_rope_preserves_vector_norm():
    orig = np.array([0.5, -1.5, 2.0, 0.25, -0.75, 1.1, 0.9, -0.4], np.float32)
    x = bbo.rope_neox(orig, 7, THETA)
    assert abs(float(np.sum(orig * orig)) - float(np.sum(x * x))) < 1e-4


def test_rope_bits_follow_libm():
    # theta_scale = powf(base, -2/d); theta from (float)pos, times theta_scale per pair in f32;
    # libm sinf / cosf; x[i] = a·cos - b·sin, x[i+half] = a·sin + b·cos
    libm = ctypes.CDLL(ctypes.util.find_library("m"))
    for f in ("sinf", "cosf"):
        getattr(libm, f).restype = ctypes.c_float
        getattr(libm, f).argtypes = [ctypes.c_float]
    libm.powf.restype = ctypes.c_float
    libm.powf.argtypes = [ctypes.c_float, ctypes.c_float]
    d = 64
    x = np.random.default_rng(11).standard_normal(d).astype(np.float32)
    for pos in (0, 1, 17, 300, 4095, 70000):
        scale = np.float32(libm.powf(THETA, float(np.float32(-2.0) / np.float32(d))))
        th = np.float32(pos)
        want = x.copy()
        for i in range(d // 2):
            s, c = np.float32(libm.sinf(float(th))), np.float32(libm.cosf(float(th)))
            a, b = x[i], x[i + d // 2]
            want[i] = np.float32(a * c) - np.float32(b * s)
            want[i + d // 2] = np.float32(a * s) + np.float32(b * c)
            th = np.float32(th * scale)
        assert bbo.rope_neox(x, pos, THETA).view(np.uint32).tolist() == want.view(np.uint32).tolist(), pos


def test_norm_rope_heads_is_rmsnorm_then_rope():
    g = np.random.default_rng(13)
    nh, hd = 4, 64
    buf = g.standard_normal(nh * hd).astype(np.float32) * np.float32(3)
    gain = (1 + 0.1 * g.standard_normal(hd)).astype(np.float32)
    got = bbo.norm_rope_heads(buf, nh, hd, gain, 1e-5, 9, THETA)
    want = np.concatenate([bbo.rope_neox(bbo.rmsnorm(buf[h * hd:(h + 1) * hd], gain, 1e-5), 9, THETA)
                           for h in range(nh)])
    assert got.view(np.uint32).tolist() == want.view(np.uint32).tolist()


# ---- operators: batched == token by token (model.rs:668-705) ------------------------------------

def _conv_small():
    return synth.conv_weights(3, hidden=512, in_dtype=synth.Q4_K, out_dtype=synth.Q6_K)


def test_conv_batch_matches_per_token_and_chunks():
    w = _conv_small()
    t = 9
    x = synth.hidden_states(4, t, hidden=512).reshape(-1)
    st0 = np.zeros(512 * 2, np.float32)
    st = st0.copy()
    per = []
    for i in range(t):
        o, st = bbo.conv_forward(w, st, x[i * 512:(i + 1) * 512], 1)
        per.append(o)
    per = np.concatenate(per)
    ob, sb = bbo.conv_forward(w, st0, x, t)
    assert ob.view(np.uint32).tolist() == per.view(np.uint32).tolist()
    assert sb.view(np.uint32).tolist() == st.view(np.uint32).tolist()
    # chunks of 4, 4, 1
    sc = st0.copy()
    parts = []
    for a, b in ((0, 4), (4, 8), (8, 9)):
        o, sc = bbo.conv_forward(w, sc, x[a * 512:b * 512], b - a)
        parts.append(o)
    assert np.concatenate(parts).view(np.uint32).tolist() == per.view(np.uint32).tolist()
    assert np.all(np.isfinite(per)) and np.abs(per).max() > 0


def _attn_small():
    return synth.attn_weights(5, hidden=512, n_heads=8, n_kv_heads=2)


def test_attn_batch_matches_per_token_and_chunks():
    w = _attn_small()
    t = 7
    x = synth.hidden_states(6, t, hidden=512).reshape(-1)
    ca = bbo.KvCache(w.kv_dim, 16)
    per = np.concatenate([bbo.attn_forward(w, ca, i, x[i * 512:(i + 1) * 512], 1) for i in range(t)])
    cb = bbo.KvCache(w.kv_dim, 16)
    ob = bbo.attn_forward(w, cb, 0, x, t)
    assert ob.view(np.uint32).tolist() == per.view(np.uint32).tolist()
    assert cb.n == ca.n == t
    assert cb.k.view(np.uint32).tolist() == ca.k.view(np.uint32).tolist()
    assert cb.v.view(np.uint32).tolist() == ca.v.view(np.uint32).tolist()
    cc = bbo.KvCache(w.kv_dim, 16)
    parts = [bbo.attn_forward(w, cc, a, x[a * 512:b * 512], b - a) for a, b in ((0, 3), (3, 6), (6, 7))]
    assert np.concatenate(parts).view(np.uint32).tolist() == per.view(np.uint32).tolist()
    assert np.all(np.isfinite(per)) and np.abs(per).max() > 0


def test_attn_first_token_attends_to_itself_only():
    # one cached position: the softmax weight is exactly 1, so the attention output is the value
    # row of each head's kv head (before o_proj): checked through the mirror with n_ctx = 1
    w = _attn_small()
    x = synth.hidden_states(8, 1, hidden=512).reshape(-1)
    c = bbo.KvCache(w.kv_dim, 4)
    bbo.attn_forward(w, c, 0, x, 1)
    v = c.v[:w.kv_dim]
    q = np.random.default_rng(1).standard_normal(w.n_heads * w.head_dim).astype(np.float32)
    out = bbo.attention_decode(q, c.k[:w.kv_dim], v, 1, w.n_heads, w.n_kv_heads, w.head_dim)
    group = w.n_heads // w.n_kv_heads
    want = np.concatenate([v[(h // group) * w.head_dim:(h // group + 1) * w.head_dim] for h in range(w.n_heads)])
    assert out.tolist() == want.tolist()
