"""GPU parity: libbebelm_moe.so (through its C ABI) against the CPU restatement.

The bar is bit-exactness: integer sub-dots are exact and every f32 epilogue follows the
reference's operation order, so each value must equal the oracle's bit for bit (routing indices,
weights, permutation, gate/up/down rows, combined outputs). Sizes are the real model's where the
oracle finishes in seconds (one full MoE layer, 1 and 16 tokens) and reduced elsewhere.
"""
import numpy as np
import pytest

from bebelm_amd import synth
from bebelm_amd import kernels as K
from bebelm_amd.model import DenseLayer, FfnStack, MoeLayer, RouteTrace, Tensor

pytestmark = pytest.mark.gpu

F32, F16, Q4_K, Q6_K = 0, 1, 12, 14


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def assert_bits(got, want, what=""):
    got, want = np.asarray(got, np.float32).reshape(-1), np.asarray(want, np.float32).reshape(-1)
    if not np.array_equal(bits(got), bits(want)):
        bad = np.nonzero(bits(got) != bits(want))[0]
        i = bad[0]
        raise AssertionError(f"{what}: {bad.size}/{got.size} differ; first at {i}: {got[i]!r} vs {want[i]!r}")


def log(msg):
    print(msg, flush=True)


# ---- kernel-level mirrors ---------------------------------------------------------------------

def test_quantize_q8(gpu_ctx, oracle):
    g = np.random.default_rng(1)
    x = (g.standard_normal(4096) * 3).astype(np.float32)
    x[:256] = 0.0
    x[256:512] = (np.arange(256, dtype=np.float32) - 128) * np.float32(0.5)
    got = K.quantize_q8(gpu_ctx, x)
    want = oracle.quantize_q8(x)
    assert np.array_equal(got.q, want.q)
    assert_bits(got.scales, want.scales, "scales")
    assert np.array_equal(got.sums, want.sums)


@pytest.mark.parametrize("dtype", [Q4_K, Q6_K])
@pytest.mark.parametrize("n_in,n_out", [(256, 7), (2048, 1792), (1792, 2048), (7168, 64)])
def test_matvec_quantized(gpu_ctx, oracle, dtype, n_in, n_out):
    log(f"matvec dtype={dtype} {n_in}x{n_out}")
    w = synth.quant_tensor(synth.rng(3, dtype, n_in), dtype, n_in, n_out)
    x = synth.hidden_states(4, 1, hidden=n_in)[0]
    t = Tensor(gpu_ctx, dtype, w, (n_in, n_out))
    y = np.empty(n_out, np.float32)
    K.matvec(gpu_ctx, dtype, t, n_in, n_out, x, y)
    assert_bits(y, oracle.matvec(dtype, w, n_in, n_out, x), "matvec")


@pytest.mark.parametrize("dtype", [Q4_K, Q6_K])
@pytest.mark.parametrize("n_in,nt", [(3072, 1), (12288, 1), (12288, 3), (16640, 2)])
def test_rows_long(gpu_ctx, oracle, dtype, n_in, nt):
    # rows of 12, 48 and 65 super-blocks: two blocks per lane group, two passes of loads per
    # row (weights reloaded per token past 32 blocks), and past 64 blocks the 8-lane kernel
    n_out = 40
    w = synth.quant_tensor(synth.rng(7, dtype, n_in), dtype, n_in, n_out)
    x = synth.hidden_states(8, nt, hidden=n_in).reshape(-1)
    t = Tensor(gpu_ctx, dtype, w, (n_in, n_out))
    y = np.empty(nt * n_out, np.float32)
    if nt == 1:
        K.matvec(gpu_ctx, dtype, t, n_in, n_out, x, y)
        want = oracle.matvec(dtype, w, n_in, n_out, x)
    else:
        K.matmul(gpu_ctx, dtype, t, n_in, n_out, x, nt, y)
        want = oracle.matmul(dtype, w, n_in, n_out, x, nt)
    assert_bits(y, want, f"rows n_in={n_in} nt={nt}")


@pytest.mark.parametrize("dtype", [Q4_K, Q6_K])
@pytest.mark.parametrize("n_in,n_out,nt", [(2048, 16384, 1), (512, 16390, 1), (2048, 16391, 3)])
def test_rows_many(gpu_ctx, oracle, dtype, n_in, n_out, nt):
    # matrices of 16384 rows and more take several rows per wave; 16390 and 16391 rows leave a
    # last wave with rows past the matrix
    w = synth.quant_tensor(synth.rng(9, dtype, n_out), dtype, n_in, n_out)
    x = synth.hidden_states(10, nt, hidden=n_in).reshape(-1)
    t = Tensor(gpu_ctx, dtype, w, (n_in, n_out))
    y = np.empty(nt * n_out, np.float32)
    if nt == 1:
        K.matvec(gpu_ctx, dtype, t, n_in, n_out, x, y)
        want = oracle.matvec(dtype, w, n_in, n_out, x)
    else:
        K.matmul(gpu_ctx, dtype, t, n_in, n_out, x, nt, y)
        want = oracle.matmul(dtype, w, n_in, n_out, x, nt)
    assert_bits(y, want, f"rows n_in={n_in} n_out={n_out} nt={nt}")


def test_logits_head_shape(gpu_ctx, oracle):
    # logits_from_hidden's matvec (model.rs:380-388): Q6_K 2048 -> 128000, 215 MB of rows
    n_in, n_out = 2048, 128000
    w = synth.quant_tensor(synth.rng(11, Q6_K), Q6_K, n_in, n_out)
    x = synth.hidden_states(12, 1, hidden=n_in).reshape(-1)
    t = Tensor(gpu_ctx, Q6_K, w, (n_in, n_out))
    y = np.empty(n_out, np.float32)
    K.matvec(gpu_ctx, Q6_K, t, n_in, n_out, x, y)
    assert_bits(y, oracle.matvec(Q6_K, w, n_in, n_out, x), "logits head")


@pytest.mark.parametrize("dtype,vocab,on_device", [(Q6_K, 32771, False), (Q6_K, 32771, True), (Q4_K, 5000, False)])
def test_logits_from_hidden(gpu_ctx, oracle, dtype, vocab, on_device):
    import torch
    n_in = 2048
    w = synth.quant_tensor(synth.rng(13, dtype, vocab), dtype, n_in, vocab)
    h = synth.hidden_states(14, 1, hidden=n_in).reshape(-1) * 3.0
    gain = synth.rng(15).uniform(0.5, 1.5, n_in).astype(np.float32)
    t = Tensor(gpu_ctx, dtype, w, (n_in, vocab))
    want = oracle.matvec(dtype, w, n_in, vocab, oracle.rmsnorm(h, gain, 1e-5))
    if on_device:
        hd, gd = torch.from_numpy(h).cuda(), torch.from_numpy(gain).cuda()
        yd = torch.empty(vocab, dtype=torch.float32, device="cuda")
        K.logits_from_hidden(gpu_ctx, t, gd, 1e-5, hd, yd)
        gpu_ctx.synchronize()
        y = yd.cpu().numpy()
    else:
        y = np.empty(vocab, np.float32)
        K.logits_from_hidden(gpu_ctx, t, gain, 1e-5, h, y)
    assert_bits(y, want, f"logits_from_hidden vocab={vocab}")


@pytest.mark.parametrize("dtype", [Q4_K, Q6_K])
def test_matmul_quantized_and_expert_slice(gpu_ctx, oracle, dtype):
    n_in, n_out, n_exp, nt = 512, 96, 3, 5
    w = synth.quant_tensor(synth.rng(5, dtype), dtype, n_in, n_out, n_exp)
    x = synth.hidden_states(6, nt, hidden=n_in).reshape(-1)
    t = Tensor(gpu_ctx, dtype, w, (n_in, n_out, n_exp))
    stride = synth.byte_size(dtype, n_in * n_out)
    for e in range(n_exp):
        y = np.empty(nt * n_out, np.float32)
        K.matmul(gpu_ctx, dtype, t, n_in, n_out, x, nt, y, byte_off=e * stride)
        assert_bits(y, oracle.matmul(dtype, w[e * stride:(e + 1) * stride], n_in, n_out, x, nt), f"expert {e}")


@pytest.mark.parametrize("dtype", [F32, F16])
@pytest.mark.parametrize("n_in,n_out,nt", [(2, 3, 1), (40, 128, 1), (2048, 32, 1), (2048, 32, 5), (35, 9, 3)])
def test_matvec_float(gpu_ctx, oracle, dtype, n_in, n_out, nt):
    g = np.random.default_rng(n_in * 7 + n_out)
    w = g.standard_normal(n_in * n_out).astype(np.float32 if dtype == F32 else np.float16)
    x = g.standard_normal(n_in * nt).astype(np.float32)
    t = Tensor(gpu_ctx, dtype, w, (n_in, n_out))
    y = np.empty(n_out * nt, np.float32)
    K.matmul(gpu_ctx, dtype, t, n_in, n_out, x, nt, y)
    assert_bits(y, oracle.matmul(dtype, w.view(np.uint8), n_in, n_out, x, nt), "float matmul")


def test_reference_small_matrices(gpu_ctx, oracle):
    # matmul.rs:1088-1105, :1191-1216 on the GPU
    w = np.array([1, 2, 3, 4, 5, 6], np.float32)
    t = Tensor(gpu_ctx, F32, w, (2, 3))
    y = np.empty(3, np.float32)
    assert K.matvec(gpu_ctx, F32, t, 2, 3, np.array([1, 1], np.float32), y).tolist() == [3.0, 7.0, 11.0]
    assert K.matvec(gpu_ctx, F32, t, 2, 3, np.array([0, 1], np.float32), y).tolist() == [2.0, 4.0, 6.0]
    block = np.zeros(144, np.uint8)
    block[0:2] = [0x00, 0x3C]
    block[4] = 1
    block[16] = 0x07
    x = np.zeros(256, np.float32)
    x[0] = 1.0
    tq = Tensor(gpu_ctx, Q4_K, block, (256, 1))
    y1 = np.empty(1, np.float32)
    assert K.matvec(gpu_ctx, Q4_K, tq, 256, 1, x, y1)[0] == 7.0


def test_fused_batch(gpu_ctx, oracle):
    H, F = 2048, 1792
    wg = synth.quant_tensor(synth.rng(8, 1), Q4_K, H, F, 2)
    wd = synth.quant_tensor(synth.rng(8, 2), Q6_K, F, H, 2)
    tg = Tensor(gpu_ctx, Q4_K, wg, (H, F, 2))
    td = Tensor(gpu_ctx, Q6_K, wd, (F, H, 2))
    x = synth.hidden_states(8, 1)[0]
    a = synth.hidden_states(9, 1, hidden=F)[0]
    qx, qa = K.quantize_q8(gpu_ctx, x), K.quantize_q8(gpu_ctx, a)
    gs, ds = synth.byte_size(Q4_K, H * F), synth.byte_size(Q6_K, F * H)
    jobs = [K.FusedJob(Q4_K, tg, H, F, qx, byte_off=gs), K.FusedJob(Q6_K, td, F, H, qa, byte_off=ds),
            K.FusedJob(Q4_K, tg, H, F, qx, byte_off=0)]
    out = np.empty(F + H + F, np.float32)
    K.matvec_fused_batch(gpu_ctx, jobs, out)
    oq, oa = oracle.quantize_q8(x), oracle.quantize_q8(a)
    want = oracle.matvec_fused_batch([(Q4_K, wg[gs:], H, F, x, oq), (Q6_K, wd[ds:], F, H, a, oa),
                                      (Q4_K, wg[:gs], H, F, x, oq)])
    assert_bits(out, want, "fused batch")


def test_fused_batch_f32_arm(gpu_ctx, oracle):
    # FusedJob with qx: None takes fused_row_dot (matmul.rs:777-785, :1045): jobs of both dtypes
    # without qx, mixed with a pre-quantised one, as one call (matmul.rs:1519-1528 checks the
    # Q4_K f32 fallback against standalone fused_row_dot rows)
    H, F = 2048, 1792
    wg = synth.quant_tensor(synth.rng(9, 1), Q4_K, H, F, 2)
    wd = synth.quant_tensor(synth.rng(9, 2), Q6_K, F, H, 1)
    tg = Tensor(gpu_ctx, Q4_K, wg, (H, F, 2))
    td = Tensor(gpu_ctx, Q6_K, wd, (F, H, 1))
    x = (synth.hidden_states(10, 1)[0] * 3).astype(np.float32)
    a = synth.hidden_states(11, 1, hidden=F)[0]
    qx = K.quantize_q8(gpu_ctx, x)
    gs = synth.byte_size(Q4_K, H * F)
    jobs = [K.FusedJob(Q4_K, tg, H, F, x=x, byte_off=gs), K.FusedJob(Q6_K, td, F, H, x=a),
            K.FusedJob(Q4_K, tg, H, F, qx, byte_off=0)]
    out = np.empty(F + H + F, np.float32)
    K.matvec_fused_batch(gpu_ctx, jobs, out)
    want = oracle.matvec_fused_batch([(Q4_K, wg[gs:], H, F, x, None), (Q6_K, wd, F, H, a, None),
                                      (Q4_K, wg[:gs], H, F, x, oracle.quantize_q8(x))])
    assert_bits(out, want, "fused batch, f32 arm")
    rows = [oracle.fused_row_dot(Q4_K, wg[gs + o * 8 * 144:gs + (o + 1) * 8 * 144], x) for o in range(0, F, 97)]
    assert_bits(out[0:F:97], np.array(rows, np.float32), "f32 arm == fused_row_dot")


def test_elementwise_and_rmsnorm(gpu_ctx, oracle):
    g = np.random.default_rng(2)
    a = (g.standard_normal(5000) * 8).astype(np.float32)
    b = g.standard_normal(5000).astype(np.float32)
    out = np.empty_like(a)
    assert_bits(K.swiglu(gpu_ctx, a, b, out), oracle.swiglu(a, b), "swiglu")
    s = a.copy()
    K.sigmoid_slice(gpu_ctx, s)
    assert_bits(s, np.array([oracle.sigmoid(v) for v in a], np.float32), "sigmoid")
    o = b.copy()
    assert_bits(K.add_scaled(gpu_ctx, o, a, 0.37), oracle.add_scaled(b, a, 0.37), "add_scaled")
    o = b.copy()
    assert_bits(K.add_assign(gpu_ctx, o, a), oracle.add_assign(b, a), "add_assign")
    x = synth.hidden_states(3, 4).reshape(-1)
    gain = (1 + g.standard_normal(2048) * 0.1).astype(np.float32)
    out = np.empty_like(x)
    K.rmsnorm(gpu_ctx, x, gain, 1e-5, out, n_vec=4)
    want = np.concatenate([oracle.rmsnorm(x[i * 2048:(i + 1) * 2048], gain, 1e-5) for i in range(4)])
    assert_bits(out, want, "rmsnorm")


def test_silu_sigmoid_extremes(gpu_ctx, oracle):
    x = np.array([0.0, -0.0, 1.0, -1.0, 20.0, -20.0, 88.0, 89.0, -88.0, -104.0, -110.0, 1e-30, 32.5641136,
                  -63.0994, np.inf, -np.inf], np.float32)
    s = x.copy()
    K.sigmoid_slice(gpu_ctx, s)
    assert_bits(s, np.array([oracle.sigmoid(v) for v in x], np.float32), "sigmoid extremes")
    out = np.empty_like(x)
    K.swiglu(gpu_ctx, x[np.isfinite(x)], np.ones(np.isfinite(x).sum(), np.float32), out[: np.isfinite(x).sum()])
    assert_bits(out[: np.isfinite(x).sum()], oracle.swiglu(x[np.isfinite(x)], np.ones(np.isfinite(x).sum())), "silu")


# ---- the MoE block ----------------------------------------------------------------------------

def check_moe(gpu_ctx, oracle, w, x, t, tag):
    log(f"moe {tag}: T={t} H={w.hidden} F={w.moe_ff} E={w.n_experts} down={w.down_dtype}")
    layer = MoeLayer(gpu_ctx, w)
    try:
        tr = RouteTrace(t, w.n_experts, w.n_used)
        got = layer.forward(np.ascontiguousarray(x.reshape(-1)), t, np.empty(t * w.hidden, np.float32), tr)
        if t == 1:
            want, otr = oracle.moe_ffn(w, x.reshape(-1), trace=True)
        else:
            want, otr = oracle.moe_ffn_batch(w, x.reshape(-1), t, trace=True)
        assert np.array_equal(tr.sel, otr.sel), f"{tag}: selected experts differ"
        assert np.array_equal(tr.counts, otr.counts) and np.array_equal(tr.offsets, otr.offsets), f"{tag}: counts"
        assert np.array_equal(tr.perm, otr.perm), f"{tag}: dispatch permutation differs"
        assert_bits(tr.logits, otr.logits, f"{tag}: router logits")
        assert_bits(tr.w, otr.w, f"{tag}: gate weights")
        assert tr.ties[0] == otr.ties[0]
        assert_bits(got, want, f"{tag}: block output")
        return got, tr
    finally:
        layer.close()


@pytest.fixture(scope="module")
def full_layer():
    return synth.config_layer(1, seed=0)


def test_moe_config1_decode_full_size(gpu_ctx, oracle, full_layer):
    x = synth.hidden_states(0, 1)
    _, tr = check_moe(gpu_ctx, oracle, full_layer, x, 1, "config1")
    assert tr.ties[0] == 0


def test_moe_config2_decode16_full_size(gpu_ctx, oracle, full_layer):
    x = synth.hidden_states(0, 16)
    _, tr = check_moe(gpu_ctx, oracle, full_layer, x, 16, "config2")
    assert tr.ties[0] == 0
    assert tr.counts.sum() == 64


@pytest.mark.parametrize("t", [1, 2, 3, 7, 33, 64])
@pytest.mark.parametrize("down", [Q4_K, Q6_K])
def test_moe_small_dims(gpu_ctx, oracle, t, down):
    w = synth.moe_weights(11, hidden=512, moe_ff=512, n_experts=8, down_dtype=down)
    x = synth.hidden_states(12, t, hidden=512)
    check_moe(gpu_ctx, oracle, w, x, t, f"small t={t}")


def test_moe_all_tokens_one_expert_group(gpu_ctx, oracle):
    # A dominant selection bias sends every token to the same 4 experts (one big group each).
    bias = np.zeros(32, np.float32)
    bias[[3, 9, 17, 30]] = [4.0, 3.0, 2.0, 1.0]
    w = synth.moe_weights(13, hidden=512, moe_ff=256, n_experts=32, bias=bias)
    x = synth.hidden_states(13, 40, hidden=512)
    _, tr = check_moe(gpu_ctx, oracle, w, x, 40, "one group")
    assert sorted(np.nonzero(tr.counts)[0].tolist()) == [3, 9, 17, 30]


def test_moe_zero_and_scaled_inputs(gpu_ctx, oracle):
    w = synth.moe_weights(14, hidden=512, moe_ff=256, n_experts=8)
    x = synth.hidden_states(14, 3, hidden=512)
    x[0] = 0.0                      # amax = 0 blocks: scale 0, q = 0
    x[1, :256] = 0.0                # one zero block
    x[2] *= np.float32(1e3)
    check_moe(gpu_ctx, oracle, w, x, 3, "zero/scaled")


def test_moe_batch_equals_per_token_on_gpu(gpu_ctx, full_layer):
    layer = MoeLayer(gpu_ctx, full_layer)
    try:
        x = synth.hidden_states(21, 5)
        batch = layer.moe_ffn_batch(x, 5)
        per = np.concatenate([layer.moe_ffn(x[i]) for i in range(5)])
        assert_bits(batch, per, "batch vs per-token")
        again = layer.moe_ffn_batch(x, 5)
        assert_bits(again, batch, "repeatability")
    finally:
        layer.close()


def test_moe_device_pointers(gpu_ctx, oracle, full_layer):
    import torch

    layer = MoeLayer(gpu_ctx, full_layer)
    try:
        x = synth.hidden_states(22, 16)
        xd = torch.from_numpy(x).cuda()
        od = torch.empty_like(xd)
        layer.forward(xd, 16, od)
        gpu_ctx.synchronize()
        assert_bits(od.cpu().numpy(), oracle.moe_ffn_batch(full_layer, x, 16), "device pointers")
    finally:
        layer.close()


def test_moe_rejects_bad_shapes(gpu_ctx):
    from bebelm_amd import BBError

    w = synth.moe_weights(1, hidden=512, moe_ff=256, n_experts=8)
    bad = Tensor(gpu_ctx, Q4_K, w.gate_exps, (512, 256, 8))
    router = Tensor(gpu_ctx, F32, w.router, (512, 8))
    import ctypes

    from bebelm_amd import _lib

    h = ctypes.c_void_p()
    rc = _lib.lib().bb_moe_create(gpu_ctx.handle, router.handle, w.exp_probs_b.ctypes.data, bad.handle, bad.handle,
                                  bad.handle, 4, ctypes.byref(h))
    assert rc == _lib.BB_ERR_SHAPE
    with pytest.raises(BBError):
        Tensor(gpu_ctx, Q4_K, w.gate_exps[:-1], (512, 256, 8))


# ---- dense FFN and the layer stack -------------------------------------------------------------

def test_dense_ffn(gpu_ctx, oracle):
    d = synth.dense_weights(2, hidden=2048, ff=7168)
    layer = DenseLayer(gpu_ctx, d)
    try:
        x = synth.hidden_states(2, 3)
        for t in (1, 3):
            got = layer.forward(np.ascontiguousarray(x[:t].reshape(-1)), t, np.empty(t * 2048, np.float32))
            assert_bits(got, oracle.dense_ffn(d, x[:t].reshape(-1), t), f"dense t={t}")
    finally:
        layer.close()


@pytest.mark.parametrize("hidden,ff,dts,ts", [(2048, 7168, (Q4_K, Q4_K, Q4_K), (32, 77, 512)),
                                               (512, 1024, (Q6_K, Q6_K, Q6_K), (40, 130, 200)),
                                               (512, 1024, (Q4_K, Q6_K, Q6_K), (64,))])
def test_dense_ffn_batches(gpu_ctx, oracle, hidden, ff, dts, ts):
    # batches of 32 tokens and more: gate/up + swiglu and down on the grouped GEMM with every token
    # in one group (Q6_K down of 128+ tokens: member tiles of 128; 192+: k_gemm_wide); gate and up
    # of two dtypes stay on the row kernels
    g = synth.rng(7, hidden)
    d = synth.DenseWeights(hidden, ff, dts[0], dts[1], dts[2], synth.quant_tensor(g, dts[0], hidden, ff),
                           synth.quant_tensor(g, dts[1], hidden, ff), synth.quant_tensor(g, dts[2], ff, hidden))
    layer = DenseLayer(gpu_ctx, d)
    try:
        for t in ts:
            log(f"dense batch hidden={hidden} ff={ff} dtypes={dts} t={t}")
            x = synth.hidden_states(8 + t, t, hidden=hidden).reshape(-1)
            got = layer.forward(np.ascontiguousarray(x), t, np.empty(t * hidden, np.float32))
            assert_bits(got, oracle.dense_ffn(d, x, t), f"dense batch {dts} t={t}")
    finally:
        layer.close()


@pytest.mark.parametrize("dts", [(Q6_K, Q6_K, Q6_K), (Q4_K, Q6_K, Q4_K)])
def test_dense_ffn_other_dtypes(gpu_ctx, oracle, dts):
    # gate and up of one dtype take the fused gate/up/swiglu pass; of two dtypes, separate passes
    g = synth.rng(5, 0)
    gate = synth.quant_tensor(g, dts[0], 512, 1024)
    up = synth.quant_tensor(g, dts[1], 512, 1024)
    down = synth.quant_tensor(g, dts[2], 1024, 512)
    d = synth.DenseWeights(512, 1024, dts[0], dts[1], dts[2], gate, up, down)
    layer = DenseLayer(gpu_ctx, d)
    try:
        x = synth.hidden_states(6, 2, hidden=512)
        for t in (1, 2):
            got = layer.forward(np.ascontiguousarray(x[:t].reshape(-1)), t, np.empty(t * 512, np.float32))
            assert_bits(got, oracle.dense_ffn(d, x[:t].reshape(-1), t), f"dense {dts} t={t}")
    finally:
        layer.close()


def test_ffn_stack_reduced(gpu_ctx, oracle):
    layers = synth.stack_layers(seed=4, hidden=512, moe_ff=256, dense_ff=1024, n_experts=8, n_layers=6, n_dense=2)
    objs = []
    try:
        for gain, w in layers:
            objs.append((gain, MoeLayer(gpu_ctx, w) if hasattr(w, "router") else DenseLayer(gpu_ctx, w)))
        stack = FfnStack(gpu_ctx, objs)
        for t in (1, 4):
            x = synth.hidden_states(4, t, hidden=512).reshape(-1)
            got = stack.forward(x, t, np.empty_like(x))
            assert_bits(got, oracle.ffn_stack(layers, x, t), f"stack t={t}")
        stack.close()
    finally:
        for _, o in objs:
            o.close()
