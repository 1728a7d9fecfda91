"""Pins of the CPU restatement beyond the reference's own tests.

Each check is an independent computation chosen so a plausible restatement mistake (a swapped
nibble half, a scale paired with the wrong sub-block, a dropped min term, a wrong rounding mode,
a reordered combine) fails it: exhaustive f16, closed-form Q8 quantisation, integer dots
recomputed from a separately written numpy unpack, and the real-number identity
Σ_i w_i·x_i = d·sd − dmin·sm against the textbook dequantisation.
"""
import numpy as np
import pytest

from bebelm_amd import synth

Q4_K, Q6_K = 12, 14


def test_f16_exhaustive(oracle):
    h = np.arange(65536, dtype=np.uint32)
    # through the F16 dequantiser (dequant.rs:158-162), which writes the f32 bits to memory
    got = oracle.dequantize(1, h.astype(np.uint16).view(np.uint8), 65536)
    want = h.astype(np.uint16).view(np.float16).astype(np.float32)
    finite = ~np.isnan(want)
    assert np.array_equal(got[finite].view(np.uint32), want[finite].view(np.uint32))
    # NaN: sign | exponent all ones | mantissa << 13, quiet bit not forced (dequant.rs:45-47)
    nan_bits = ((h & 0x8000) << 16) | 0x7F800000 | ((h & 0x3FF) << 13)
    assert np.array_equal(got[~finite].view(np.uint32), nan_bits[~finite].astype(np.uint32))


def np_unpack_q4k(block):
    """Independent numpy unpack of one Q4_K block: (d, dmin, sc[8], m[8], nib[256])."""
    b = block.astype(np.int64)
    d = np.frombuffer(block[0:2].tobytes(), np.float16)[0].astype(np.float64)
    dmin = np.frombuffer(block[2:4].tobytes(), np.float16)[0].astype(np.float64)
    s = b[4:16]
    sc = np.empty(8, np.int64)
    m = np.empty(8, np.int64)
    sc[:4] = s[0:4] & 63
    m[:4] = s[4:8] & 63
    sc[4:] = (s[8:12] & 0xF) | ((s[0:4] >> 6) << 4)
    m[4:] = (s[8:12] >> 4) | ((s[4:8] >> 6) << 4)
    qs = b[16:144].reshape(4, 32)
    nib = np.stack([qs & 0xF, qs >> 4], axis=1).reshape(256)  # chunk c: low nibbles then high
    return d, dmin, sc, m, nib


def np_unpack_q6k(block):
    b = block.astype(np.int64)
    d = np.frombuffer(block[208:210].tobytes(), np.float16)[0].astype(np.float64)
    sc = block[192:208].view(np.int8).astype(np.int64)
    q = np.empty(256, np.int64)
    for n in range(2):
        ql = b[64 * n:64 * n + 64]
        qh = b[128 + 32 * n:128 + 32 * n + 32]
        base = 128 * n
        q[base:base + 32] = (ql[:32] & 0xF) | ((qh & 3) << 4)
        q[base + 32:base + 64] = (ql[32:] & 0xF) | (((qh >> 2) & 3) << 4)
        q[base + 64:base + 96] = (ql[:32] >> 4) | (((qh >> 4) & 3) << 4)
        q[base + 96:base + 128] = (ql[32:] >> 4) | (((qh >> 6) & 3) << 4)
    return d, sc, q - 32


@pytest.mark.parametrize("seed", range(6))
def test_q4k_integer_dot_brute_force(oracle, seed):
    g = np.random.default_rng(seed)
    blocks = synth.q4k_blocks(synth.rng(seed, 1), 16).reshape(16, 144)
    for blk in blocks:
        x = g.standard_normal(256).astype(np.float32) * np.float32(g.uniform(0.1, 5))
        a = oracle.quantize_q8(x)
        d, dmin, sc, m, nib = np_unpack_q4k(blk)
        qx = a.q.astype(np.int64)
        sd = int(np.sum(np.repeat(sc, 32) * nib * qx))
        sm = int(np.sum(m * a.sums.astype(np.int64)))
        assert oracle.q4k_block_sd(blk, a.q) == sd
        want = np.float32(a.scales[0]) * (np.float32(d) * np.float32(sd) - np.float32(dmin) * np.float32(sm))
        got = np.float32(oracle.dot_q4k_block_q8(blk, a.q, a.scales[0], a.sums))
        assert got.view(np.uint32) == np.float32(want).view(np.uint32)
        # textbook dequantisation (dequant.rs:75-106) against the factored integer form
        w = oracle.dequantize(Q4_K, blk, 256).astype(np.float64)
        real = float(np.sum(w * qx))
        assert abs(real - (d * sd - dmin * sm)) <= 1e-5 * max(abs(real), 1e-3) + 1e-6 * np.sum(np.abs(w * qx))


@pytest.mark.parametrize("fill", [0xFF, 0x00, 0xF0, 0x0F])
@pytest.mark.parametrize("xv", [127, -127])
def test_integer_dots_at_extremes(oracle, fill, xv):
    # every quant and scale at its largest (or smallest) value against activations all +-127
    # (and alternating): the vector forms of the block dots must not saturate or wrap
    for alt in (False, True):
        qx = np.full(256, xv, np.int8)
        if alt:
            qx[1::2] = -xv
        blk4 = np.full(144, fill, np.uint8)
        _, _, sc, _, nib = np_unpack_q4k(blk4)
        assert oracle.q4k_block_sd(blk4, qx) == int(np.sum(np.repeat(sc, 32) * nib * qx.astype(np.int64)))
        for scale_byte in (0x7F, 0x80):
            blk6 = np.full(210, fill, np.uint8)
            blk6[192:208] = scale_byte
            _, sc6, q6 = np_unpack_q6k(blk6)
            want = int(np.sum(np.repeat(sc6, 16) * q6 * qx.astype(np.int64)))
            assert oracle.q6k_block_idot(blk6, qx) == want
            assert oracle.q6k_block_idot(blk6, qx, buffered=True) == want


@pytest.mark.parametrize("seed", range(6))
def test_q6k_integer_dot_brute_force(oracle, seed):
    g = np.random.default_rng(100 + seed)
    blocks = synth.q6k_blocks(synth.rng(seed, 2), 16).reshape(16, 210)
    for blk in blocks:
        x = g.standard_normal(256).astype(np.float32)
        a = oracle.quantize_q8(x)
        d, sc, q = np_unpack_q6k(blk)
        s = int(np.sum(np.repeat(sc, 16) * q * a.q.astype(np.int64)))
        assert oracle.q6k_block_idot(blk, a.q) == s
        assert oracle.q6k_block_idot(blk, a.q, buffered=True) == s
        want = np.float32(a.scales[0]) * (np.float32(d) * np.float32(s))
        got = np.float32(oracle.dot_q6k_block_q8(blk, a.q, a.scales[0]))
        assert got.view(np.uint32) == np.float32(want).view(np.uint32)
        w = oracle.dequantize(Q6_K, blk, 256).astype(np.float64)
        assert abs(float(np.sum(w * a.q)) - d * s) <= 1e-9 * max(1.0, abs(d * s))


def test_quantize_q8_closed_form(oracle):
    g = np.random.default_rng(7)
    for trial in range(20):
        x = (g.standard_normal(1024) * g.uniform(1e-3, 1e3)).astype(np.float32)
        if trial == 0:
            x[:256] = 0.0  # amax = 0 -> all zero, scale 0
        if trial == 1:
            x[256:512] = np.float32(2.5) * np.sign(g.standard_normal(256)).astype(np.float32)  # ±amax -> ±127
        if trial == 2:
            x[512:768] = (np.arange(256, dtype=np.float32) - 128) * np.float32(0.5)  # exact .5 ties
        a = oracle.quantize_q8(x)
        for b in range(4):
            xb = x[b * 256:(b + 1) * 256]
            amax = np.float32(np.max(np.abs(xb)))
            assert a.scales[b].view(np.uint32) == np.float32(amax / np.float32(127)).view(np.uint32)
            inv = np.float32(127) / amax if amax > 0 else np.float32(0)
            y = (xb * inv).astype(np.float32)
            r = np.sign(y) * np.floor(np.abs(y) + np.float32(0.5))  # half away from zero
            want = np.clip(r, -127, 127).astype(np.int8)
            assert np.array_equal(a.q[b * 256:(b + 1) * 256], want)
            assert np.array_equal(a.sums[b * 8:(b + 1) * 8], want.astype(np.int32).reshape(8, 32).sum(1))
        if trial == 0:
            assert np.all(a.q[:256] == 0) and a.scales[0] == 0
        if trial == 1:
            assert np.all(np.abs(a.q[256:512]) == 127)


def test_router_dot_close_to_exact(oracle):
    # The f32 dot's last bits depend on the `wide` crate's reduce order (parity unpinned);
    # its value is pinned to the exact sum within f32 accumulation error.
    g = np.random.default_rng(3)
    for n in (256, 2048, 2049, 2056):
        a = g.standard_normal(n).astype(np.float32)
        b = g.standard_normal(n).astype(np.float32)
        exact = float(np.dot(a.astype(np.float64), b.astype(np.float64)))
        got = oracle.dot(a, b)
        assert abs(got - exact) <= 1e-5 * float(np.sum(np.abs(a.astype(np.float64) * b)))


def test_router_dot_reduce_order_is_the_avx_tree(oracle):
    # The restatement assumes the `wide` AVX reduce ((v0+v4)+(v2+v6))+((v1+v5)+(v3+v7)) of the
    # eight lane values (parity unpinned: the crate is not vendored). These lane values make each
    # candidate order give a different f32 result, worked out by hand from the rounding of
    # 2^24 + 1 (a tie, which rounds to the even 2^24):
    #   AVX tree:        ((2^24 + 1) + (1 + 0)) + ((-2^24 + 0) + (1 + 0)) = 2^24 - (2^24 - 1) = 1
    #   pairwise fold:   f = (2^24 + 1, -2^24 + 0, 1 + 0, 1 + 0) = (2^24, -2^24, 1, 1) -> 0 + 2 = 2
    #   left to right:   2^24 - 2^24 + 1 + 1 + 1 = 3 (also the exact sum)
    # One product per chain (chains 0..7 only, b = 1), so lane l's value is a[l] exactly.
    n = 32
    a = np.zeros(n, np.float32)
    a[:8] = [2.0 ** 24, -2.0 ** 24, 1.0, 1.0, 1.0, 0.0, 0.0, 0.0]
    b = np.ones(n, np.float32)
    assert np.float32(oracle.dot(a, b)) == np.float32(1.0)
    assert np.float32(oracle.dot_variant(a, b, 0)) == np.float32(1.0)
    assert np.float32(oracle.dot_variant(a, b, 1)) == np.float32(1.0)  # no FMA, same tree
    assert np.float32(oracle.dot_variant(a, b, 2)) == np.float32(2.0)
    assert np.float32(oracle.dot_variant(a, b, 6)) == np.float32(2.0)
    assert np.float32(oracle.dot_variant(a, b, 3)) == np.float32(3.0)
    assert np.float32(oracle.dot_variant(a, b, 5)) == np.float32(3.0)
    # the lane combine (acc0 + acc1) + (acc2 + acc3) of one lane: chains l, 8+l, 16+l, 24+l
    c = np.zeros(n, np.float32)
    c[[0, 8, 16, 24]] = [2.0 ** 24, 1.0, 1.0, -2.0 ** 24]
    # (2^24 + 1) + (1 - 2^24) = 2^24 - (2^24 - 1) = 1; the scalar left-to-right sum instead gives
    # ((2^24 + 1) + 1) - 2^24 = (2^24 + 1) - 2^24 = 2^24 - 2^24 = 0
    assert np.float32(oracle.dot(c, b)) == np.float32(1.0)
    assert np.float32(oracle.dot_variant(c, b, 4)) == np.float32(0.0)


def test_pack_q4k_scales_inverts_get_scale_min_k4(oracle):
    g = np.random.default_rng(11)
    for _ in range(50):
        sc = g.integers(0, 64, 8)
        m = g.integers(0, 64, 8)
        packed = synth.pack_q4k_scales(sc[None], m[None])[0]
        for j in range(8):
            assert oracle.get_scale_min_k4(j, packed) == (sc[j], m[j])


def test_moe_batch_equals_per_token(oracle):
    # model.rs:280-285: moe_ffn_batch is bit-identical to moe_ffn per token.
    w = synth.moe_weights(5, hidden=512, moe_ff=512, n_experts=8, down_dtype=Q6_K)
    x = synth.hidden_states(5, 6, hidden=512)
    batch = oracle.moe_ffn_batch(w, x, 6)
    per = np.concatenate([oracle.moe_ffn(w, x[i]) for i in range(6)])
    assert np.array_equal(batch.view(np.uint32), per.view(np.uint32))


def test_moe_decode_matches_composed_kernels(oracle):
    # moe_ffn = router matvec -> sigmoid/top-k/renorm -> fused gate/up -> swiglu -> down -> combine,
    # recomposed here from the oracle's kernel-level functions and numpy glue.
    w = synth.moe_weights(9, hidden=512, moe_ff=256, n_experts=8)
    x = synth.hidden_states(9, 1, hidden=512)[0]
    out, tr = oracle.moe_ffn(w, x, trace=True)
    H, F, E, K = 512, 256, 8, 4
    logits = oracle.matvec(0, w.router.view(np.uint8), H, E, x)
    assert np.array_equal(logits.view(np.uint32), tr.logits.view(np.uint32))
    s = np.array([oracle.sigmoid(v) for v in logits], np.float32)
    key = (s + w.exp_probs_b).astype(np.float32)
    order = sorted(range(E), key=lambda e: (-key[e], e))
    sel = order[:K]
    assert list(tr.sel) == sel
    denom = np.float32(-0.0)
    for e in sel:
        denom = np.float32(denom + s[e])
    denom = np.float32(denom + np.float32(1e-6))
    assert np.array_equal(tr.w, (s[sel] / denom).astype(np.float32))
    q8 = oracle.quantize_q8(x)
    gs = synth.byte_size(Q4_K, H * F)
    ds = synth.byte_size(Q4_K, F * H)
    res = np.zeros(H, np.float32)
    for k, e in enumerate(sel):
        g = oracle.matvec_fused_batch([(Q4_K, w.gate_exps[e * gs:(e + 1) * gs], H, F, x, q8)])
        u = oracle.matvec_fused_batch([(Q4_K, w.up_exps[e * gs:(e + 1) * gs], H, F, x, q8)])
        act = oracle.swiglu(g, u)
        dn = oracle.matvec_fused_batch([(Q4_K, w.down_exps[e * ds:(e + 1) * ds], F, H, act, oracle.quantize_q8(act))])
        res = oracle.add_scaled(res, dn, tr.w[k])
    assert np.array_equal(res.view(np.uint32), out.view(np.uint32))
