"""GPU parity of the decoder layer's operators (the full decode layer and the batched prefill
operators around the MoE block): the kernel mirrors conv_step / conv_prefill, softmax,
attention_decode and rope_neox, and the gated short-conv and GQA attention operators, against
the CPU restatement on the same inputs. The bar is bit-exactness (every value is computed with
the reference's operations in its order; see bb_ops.hip).

Reference: kernels/conv.rs:18-68, softmax.rs:9-22, attention.rs:17-55, rope.rs:17-30,
model.rs:399-427 / :190-216 (conv), :430-456 / :222-259 (attention), :692-701 (q/k norm + RoPE),
cache.rs:40-50 (eviction).
"""
import numpy as np
import pytest

from bebelm_amd import kernels as K
from bebelm_amd import synth
from bebelm_amd.model import AttnOp, ConvOp

from test_gpu_parity import log

pytestmark = pytest.mark.gpu


def bits(a):
    return np.asarray(a, np.float32).reshape(-1).view(np.uint32)


def same(got, want, what):
    got, want = bits(got), bits(want)
    assert got.size == want.size, what
    diff = np.count_nonzero(got != want)
    assert diff == 0, f"{what}: {diff}/{got.size} values differ in bits"


# ---- kernel mirrors ------------------------------------------------------------------------------

def test_conv_step_known_answers(gpu_ctx):
    out = np.zeros(1, np.float32)
    K.conv_step(gpu_ctx, np.array([2.0, 3.0], np.float32), np.array([4.0], np.float32),
                np.array([1.0, 10.0, 100.0], np.float32), 1, 3, out)
    assert out.tolist() == [432.0]
    out2 = np.zeros(2, np.float32)
    K.conv_step(gpu_ctx, np.array([10.0, 20.0], np.float32), np.ones(2, np.float32),
                np.array([1.0, 2.0, 3.0, 4.0], np.float32), 2, 2, out2)
    assert out2.tolist() == [12.0, 64.0]
    out3 = np.zeros(1, np.float32)
    K.conv_step(gpu_ctx, np.zeros(0, np.float32), np.array([3.0], np.float32), np.array([5.0], np.float32), 1, 1, out3)
    assert out3.tolist() == [15.0]


@pytest.mark.parametrize("C,L,n", [(2048, 3, 1), (2048, 3, 7), (512, 2, 5), (300, 4, 2), (64, 3, 33)])
def test_conv_prefill_matches_oracle(gpu_ctx, oracle, C, L, n):
    g = np.random.default_rng(C + 7 * L + n)
    w = g.standard_normal(C * L).astype(np.float32)
    st = g.standard_normal(C * (L - 1)).astype(np.float32)
    bx = g.standard_normal(n * C).astype(np.float32)
    out = np.zeros(n * C, np.float32)
    s_gpu = st.copy()
    K.conv_prefill(gpu_ctx, s_gpu, bx, w, C, L, n, out)
    want, s_want = oracle.conv_prefill(st, bx, w, C, L, n)
    same(out, want, f"conv_prefill C={C} L={L} n={n}")
    same(s_gpu, s_want, f"conv state C={C} L={L} n={n}")
    one = np.zeros(C, np.float32)
    K.conv_step(gpu_ctx, st, bx[:C], w, C, L, one)
    same(one, oracle.conv_step(st, bx[:C], w, C, L), "conv_step")


@pytest.mark.parametrize("n", [1, 3, 64, 65, 1000, 4096, 20000, 40000, 41000])
def test_softmax_matches_oracle(gpu_ctx, oracle, n):
    g = np.random.default_rng(n)
    rows = 3
    x = (g.standard_normal(rows * n) * 5).astype(np.float32)
    if n == 4096:
        x[:n] = np.array([0.0 if i < 16 else -15.0 + (i % 3) * 0.2 for i in range(n)], np.float32)  # softmax.rs:69
    got = x.copy()
    K.softmax(gpu_ctx, got, rows)
    want = np.concatenate([oracle.softmax(x[r * n:(r + 1) * n]) for r in range(rows)])
    same(got, want, f"softmax n={n}")


@pytest.mark.parametrize("n", [21324, 33825, 40880, 20000])
def test_softmax_of_equal_scores(gpu_ctx, oracle, n):
    # every exp is 1.0, so the sum is exactly n: at 21,324, 33,825 and 40,880 positions the
    # interval test cannot settle (float)(1 / sum) and the kernel runs the reference's chain of
    # adds (in LDS, and past the 40,000 positions LDS takes, in global memory); at 20,000 the
    # interval settles it (tests/test_softmax_interval.py)
    x = np.full(2 * n, 0.75, np.float32)
    x[n:] = -3.5
    got = x.copy()
    K.softmax(gpu_ctx, got, 2)
    want = np.concatenate([oracle.softmax(x[:n]), oracle.softmax(x[n:])])
    same(got, want, f"softmax of equal scores n={n}")
    assert np.all(got.view(np.uint32) == np.float32(1.0 / n).view(np.uint32))


@pytest.mark.parametrize("n_ctx,G", [(21324, 4), (33825, 1), (40880, 2)])
def test_attention_decode_equal_scores(gpu_ctx, oracle, n_ctx, G):
    # identical key rows give every head a row of equal scores (the chain-of-adds case above),
    # through the softmax and k_attn_pv_long
    g = np.random.default_rng(n_ctx)
    nkv, hd = 2, 64
    nh = nkv * G
    q = g.standard_normal(nh * hd).astype(np.float32)
    k = np.tile(g.standard_normal(nkv * hd).astype(np.float32), n_ctx)
    v = g.standard_normal(n_ctx * nkv * hd).astype(np.float32)
    out = np.zeros(nh * hd, np.float32)
    K.attention_decode(gpu_ctx, q, k, v, n_ctx, nh, nkv, hd, out)
    same(out, oracle.attention_decode(q, k, v, n_ctx, nh, nkv, hd), f"attention of equal scores n_ctx={n_ctx}")


@pytest.mark.parametrize("n_ctx,nh,nkv,hd", [(1, 1, 1, 2), (2, 1, 1, 2), (1, 2, 1, 2), (37, 8, 2, 64),
                                             (300, 32, 8, 64), (129, 4, 4, 40), (1000, 32, 8, 64), (16000, 8, 2, 64),
                                             (32769, 8, 2, 64), (41000, 4, 1, 64), (500, 4, 4, 64),
                                             (700, 4, 2, 64), (900, 16, 2, 64), (333, 16, 1, 64), (65, 2, 2, 64)])
def test_attention_decode_matches_oracle(gpu_ctx, oracle, n_ctx, nh, nkv, hd):
    g = np.random.default_rng(n_ctx * 131 + nh)
    q = g.standard_normal(nh * hd).astype(np.float32)
    k = g.standard_normal(n_ctx * nkv * hd).astype(np.float32)
    v = g.standard_normal(n_ctx * nkv * hd).astype(np.float32)
    out = np.zeros(nh * hd, np.float32)
    K.attention_decode(gpu_ctx, q, k, v, n_ctx, nh, nkv, hd, out)
    same(out, oracle.attention_decode(q, k, v, n_ctx, nh, nkv, hd), f"attention n_ctx={n_ctx} {nh}/{nkv}x{hd}")


def test_attention_known_answers(gpu_ctx):
    out = np.zeros(4, np.float32)
    K.attention_decode(gpu_ctx, np.array([1.0, 0.0, 0.0, 1.0], np.float32), np.array([1.0, 1.0], np.float32),
                       np.array([5.0, 7.0], np.float32), 1, 2, 1, 2, out)
    assert out.tolist() == [5.0, 7.0, 5.0, 7.0]


@pytest.mark.parametrize("pos", [0, 1, 7, 300, 4095, 70000])
def test_rope_matches_oracle(gpu_ctx, oracle, pos):
    g = np.random.default_rng(pos + 1)
    hd, nv = 64, 40
    x = g.standard_normal(nv * hd).astype(np.float32)
    got = x.copy()
    K.rope_neox(gpu_ctx, got, hd, pos, synth.ROPE_THETA)
    want = np.concatenate([oracle.rope_neox(x[i * hd:(i + 1) * hd], pos, synth.ROPE_THETA) for i in range(nv)])
    same(got, want, f"rope pos={pos}")


# ---- operators --------------------------------------------------------------------------------------

@pytest.mark.parametrize("hidden,dtypes,steps", [(512, (synth.Q4_K, synth.Q6_K), (1, 1, 5, 1, 9)),
                                                 (2048, (synth.Q4_K, synth.Q4_K), (1, 1, 3, 1)),
                                                 (2048, (synth.Q6_K, synth.Q4_K), (12, 1)),
                                                 # batches of 32+ tokens: projections on the grouped GEMM
                                                 (2048, (synth.Q4_K, synth.Q6_K), (32, 1, 300)),
                                                 (512, (synth.Q6_K, synth.Q6_K), (200, 2, 33))])
def test_conv_op_matches_oracle(gpu_ctx, oracle, hidden, dtypes, steps):
    w = synth.conv_weights(21, hidden=hidden, in_dtype=dtypes[0], out_dtype=dtypes[1])
    op = ConvOp(gpu_ctx, w)
    try:
        st_gpu = op.new_state()
        st_cpu = st_gpu.copy()
        for i, t in enumerate(steps):
            log(f"conv op hidden={hidden} dtypes={dtypes} call {i}: T={t}")
            x = synth.hidden_states(30 + i, t, hidden=hidden).reshape(-1)
            got = op.forward(st_gpu, x, t, np.empty(t * hidden, np.float32))
            want, st_cpu = oracle.conv_forward(w, st_cpu, x, t)
            same(got, want, f"conv op call {i} T={t}")
            same(st_gpu, st_cpu, f"conv state after call {i}")
    finally:
        op.close()


@pytest.mark.parametrize("hidden,nh,nkv,steps", [(512, 8, 2, (7, 1, 1, 3, 1)),
                                                 (2048, 32, 8, (1, 1, 1, 1)),
                                                 (2048, 32, 8, (40, 1, 2)),
                                                 (2048, 32, 8, (300, 1, 64)),
                                                 (512, 8, 2, (33, 100))])
def test_attn_op_matches_oracle(gpu_ctx, oracle, hidden, nh, nkv, steps):
    w = synth.attn_weights(23, hidden=hidden, n_heads=nh, n_kv_heads=nkv)
    op = AttnOp(gpu_ctx, w)
    cap = sum(steps) + 4
    cache = op.new_cache(cap)
    ref = oracle.KvCache(w.kv_dim, cap)
    try:
        pos = 0
        for i, t in enumerate(steps):
            log(f"attn op hidden={hidden} heads={nh}/{nkv} call {i}: T={t} pos0={pos}")
            x = synth.hidden_states(40 + i, t, hidden=hidden).reshape(-1)
            got = op.forward(cache, pos, x, t, np.empty(t * hidden, np.float32))
            want = oracle.attn_forward(w, ref, pos, x, t)
            same(got, want, f"attn op call {i} T={t}")
            pos += t
        k, v = cache.read()
        assert len(cache) == ref.n == pos
        same(k, ref.k[:pos * w.kv_dim], "k cache")
        same(v, ref.v[:pos * w.kv_dim], "v cache")
    finally:
        cache.close()
        op.close()


def test_attn_op_after_eviction(gpu_ctx, oracle):
    # cache.rs:40-50: dropping the oldest positions keeps the remaining keys' rotations; the
    # next token attends over the window that is left
    w = synth.attn_weights(25, hidden=512, n_heads=8, n_kv_heads=2)
    op = AttnOp(gpu_ctx, w)
    cache = op.new_cache(16)
    ref = oracle.KvCache(w.kv_dim, 16)
    try:
        x = synth.hidden_states(50, 6, hidden=512).reshape(-1)
        op.forward(cache, 0, x, 6, np.empty(6 * 512, np.float32))
        oracle.attn_forward(w, ref, 0, x, 6)
        cache.evict_front(4)
        keep = (ref.n - 4) * w.kv_dim
        ref.k[:keep] = ref.k[4 * w.kv_dim:ref.n * w.kv_dim].copy()
        ref.v[:keep] = ref.v[4 * w.kv_dim:ref.n * w.kv_dim].copy()
        ref.n -= 4
        x1 = synth.hidden_states(51, 1, hidden=512).reshape(-1)
        got = op.forward(cache, 6, x1, 1, np.empty(512, np.float32))
        want = oracle.attn_forward(w, ref, 6, x1, 1)
        same(got, want, "attention after eviction")
        assert len(cache) == 3
    finally:
        cache.close()
        op.close()
