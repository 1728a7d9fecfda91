"""The reference's own unit tests for the hot path, re-created against the CPU restatement.

Each test names the Rust test it re-creates (file:line under the reference's src/). Byte
patterns, inputs and asserted values are the reference's; where the reference prints a measured
value (the two LCG precision tests) the restatement must reproduce it to the printed digits.
"""
import numpy as np
import pytest

F32, F16, Q4_K, Q6_K = 0, 1, 12, 14


def f32b(vals):
    return np.asarray(vals, np.float32).view(np.uint8)


def f32_seq_sum(vals):
    """Rust `Iterator::sum::<f32>()` (sequential, starts at -0.0)."""
    acc = np.float32(-0.0)
    for v in np.asarray(vals, np.float32):
        acc = np.float32(acc + v)
    return acc


# ---- dequant.rs:188-276 ----

def test_f16_known_values(oracle):  # dequant.rs:189-202
    f = oracle.f16_to_f32
    assert f(0x0000) == 0.0 and np.signbit(np.float32(f(0x0000))) == False  # noqa: E712
    assert f(0x8000) == 0.0 and np.signbit(np.float32(f(0x8000)))
    assert f(0x3C00) == 1.0
    assert f(0x4000) == 2.0
    assert f(0xC000) == -2.0
    assert f(0x7C00) == np.inf
    assert f(0xFC00) == -np.inf
    assert np.isnan(f(0x7E00))
    assert f(0x0001) == 2.0 ** -24
    assert abs(f(0x3555) - 0.33325195) < 1e-6


def test_q4_k_block_known(oracle):  # dequant.rs:205-225
    block = np.zeros(144, np.uint8)
    block[0:2] = [0x00, 0x3C]
    block[4], block[5], block[8], block[9] = 3, 5, 0, 0
    block[16] = 0x21
    out = oracle.dequantize(Q4_K, block, 256)
    assert out[0] == 3.0 and out[32] == 10.0 and out[1] == 0.0


def test_q6_k_block_known(oracle):  # dequant.rs:228-242
    block = np.zeros(210, np.uint8)
    block[208:210] = [0x00, 0x3C]
    block[192] = 2
    block[0] = 0x05
    block[128] = 0x01
    out = oracle.dequantize(Q6_K, block, 256)
    assert out[0] == -22.0 and out[1] == -64.0


def test_dispatch_f32_passthrough(oracle):  # dequant.rs:245-252
    out = oracle.dequantize(F32, f32b([1.0, -2.5, 3.25]), 3)
    assert out.tolist() == [1.0, -2.5, 3.25]


def test_dispatch_f16_tensor(oracle):  # dequant.rs:255-261
    data = np.array([0x3C00, 0x4000, 0xC000, 0x3800], np.uint16).view(np.uint8)
    assert oracle.dequantize(F16, data, 4).tolist() == [1.0, 2.0, -2.0, 0.5]


def test_dispatch_two_q4k_blocks(oracle):  # dequant.rs:264-276
    block = np.zeros(144, np.uint8)
    block[0:2] = [0x00, 0x3C]
    block[4] = 1
    block[16] = 0x07
    out = oracle.dequantize(Q4_K, np.concatenate([block, block]), 512)
    assert out[0] == 7.0 and out[256] == 7.0


# ---- matmul.rs:1063-1548 ----

def test_dot_basic(oracle):  # matmul.rs:1064-1067
    assert oracle.dot([1.0, 2.0, 3.0], [4.0, 5.0, 6.0]) == 32.0
    assert oracle.dot(np.zeros(0, np.float32), np.zeros(0, np.float32)) == 0.0


def test_dot_covers_simd_and_tail_lengths(oracle):  # matmul.rs:1070-1085
    for n in [8, 11, 16, 19, 32, 35, 40, 64, 100]:
        a = (np.arange(n, dtype=np.float32) * np.float32(0.1) - np.float32(1.0)).astype(np.float32)
        b = ((np.arange(n) % 5).astype(np.float32) - np.float32(2.0)) * np.float32(0.3)
        got = oracle.dot(a, b)
        want = f32_seq_sum(a * b)
        assert abs(got - want) <= 1e-4 * max(abs(want), 1.0), n


def test_matvec_f32_small(oracle):  # matmul.rs:1088-1095
    y = oracle.matvec(F32, f32b([1, 2, 3, 4, 5, 6]), 2, 3, np.array([1, 1], np.float32))
    assert y.tolist() == [3.0, 7.0, 11.0]


def test_matvec_f32_selects_with_basis_vector(oracle):  # matmul.rs:1098-1105
    y = oracle.matvec(F32, f32b([1, 2, 3, 4, 5, 6]), 2, 3, np.array([0, 1], np.float32))
    assert y.tolist() == [2.0, 4.0, 6.0]


def q4k_test_block():  # matmul.rs:1108-1120
    block = np.zeros(144, np.uint8)
    block[0:2] = [0x00, 0x3C]
    block[2:4] = [0x00, 0x34]
    block[4:16] = [(j * 17 + 5) & 0xFF for j in range(12)]
    block[16:144] = [(i * 37 + 11) & 0xFF for i in range(128)]
    x = (((np.arange(256) % 7).astype(np.float32) - np.float32(3.0)) * np.float32(0.1)).astype(np.float32)
    return block, x


def q6k_test_block():  # matmul.rs:1149-1163
    block = np.zeros(210, np.uint8)
    block[208:210] = [0x00, 0x3C]
    block[0:128] = [(i * 53 + 17) & 0xFF for i in range(128)]
    block[128:192] = [(i * 97 + 5) & 0xFF for i in range(64)]
    block[192:208] = [(j * 29 + 3) & 0xFF for j in range(16)]
    x = (((np.arange(256) % 5).astype(np.float32) - np.float32(2.0)) * np.float32(0.1)).astype(np.float32)
    return block, x


@pytest.mark.parametrize("dtype,maker", [(Q4_K, q4k_test_block), (Q6_K, q6k_test_block)])
def test_fused_row_dot_matches_dequant(oracle, dtype, maker):  # matmul.rs:1122-1130, :1165-1174
    block, x = maker()
    w = oracle.dequantize(dtype, block, 256)
    ref = f32_seq_sum(w * x)
    got = oracle.fused_row_dot(dtype, block, x)
    assert abs(got - ref) <= 1e-3 * max(abs(ref), 1.0)


@pytest.mark.parametrize("dtype,maker", [(Q4_K, q4k_test_block), (Q6_K, q6k_test_block)])
def test_matvec_q8_matches_quantized_reference(oracle, dtype, maker):  # matmul.rs:1132-1145, :1176-1189
    block, x = maker()
    w = oracle.dequantize(dtype, block, 256)
    a = oracle.quantize_q8(x)
    ref = f32_seq_sum(w * (a.scales[0] * a.q.astype(np.float32)))
    y = oracle.matvec(dtype, block, 256, 1, x)
    assert abs(y[0] - ref) <= 1e-3 * max(abs(ref), 1.0)


def test_matvec_q4k_single_row(oracle):  # matmul.rs:1191-1204
    block = np.zeros(144, np.uint8)
    block[0:2] = [0x00, 0x3C]
    block[4] = 1
    block[16] = 0x07
    x = np.zeros(256, np.float32)
    x[0] = 1.0
    assert oracle.matvec(Q4_K, block, 256, 1, x)[0] == 7.0


def test_matvec_f16_small(oracle):  # matmul.rs:1206-1216
    w = np.array([0x3C00, 0x4000, 0x4200, 0x4400, 0x4500, 0x4600], np.uint16).view(np.uint8)
    assert oracle.matvec(F16, w, 2, 3, np.array([1, 1], np.float32)).tolist() == [3.0, 7.0, 11.0]


def test_matvec_parallel_path_matches_per_row_dot(oracle):  # matmul.rs:1218-1232
    n_in, n_out = 40, 128
    w = (((np.arange(n_in * n_out) % 13).astype(np.float32) - 6) * np.float32(0.05)).astype(np.float32)
    x = (((np.arange(n_in) % 7).astype(np.float32) - 3) * np.float32(0.1)).astype(np.float32)
    y = oracle.matvec(F32, w.view(np.uint8), n_in, n_out, x)
    for o in range(n_out):
        assert y[o] == oracle.dot(w[o * n_in:(o + 1) * n_in], x), o


def q4k_matrix(n_out, seed):  # matmul.rs:1235-1250
    out = []
    for r in range(n_out):
        b = np.zeros(144, np.uint8)
        b[0:2] = [0x00, 0x3C]
        b[2:4] = [0x00, 0x34]
        b[4:16] = [((r + seed) * 7 + j * 17 + 5) & 0xFF for j in range(12)]
        b[16:144] = [((r + seed) * 3 + i * 37 + 11) & 0xFF for i in range(128)]
        out.append(b)
    return np.concatenate(out)


def q6k_matrix(n_out, seed):  # matmul.rs:1253-1270
    out = []
    for r in range(n_out):
        b = np.zeros(210, np.uint8)
        b[208:210] = [0x00, 0x3C]
        b[0:128] = [((r + seed) * 5 + i * 53 + 17) & 0xFF for i in range(128)]
        b[128:192] = [((r + seed) * 11 + i * 97 + 5) & 0xFF for i in range(64)]
        b[192:208] = [((r + seed) * 29 + j * 13 + 3) & 0xFF for j in range(16)]
        out.append(b)
    return np.concatenate(out)


def test_matvec_fused_batch_matches_separate_jobs(oracle):  # matmul.rs:1272-1303
    x1 = (((np.arange(256) % 7).astype(np.float32) - 3) * np.float32(0.1)).astype(np.float32)
    x2 = (((np.arange(256) % 5).astype(np.float32) - 2) * np.float32(0.07)).astype(np.float32)
    q8 = oracle.quantize_q8(x1)
    for n_a, n_b in [(3, 5), (40, 50)]:
        wa, wb = q4k_matrix(n_a, 1), q6k_matrix(n_b, 99)
        out = oracle.matvec_fused_batch([(Q4_K, wa, 256, n_a, x1, q8), (Q6_K, wb, 256, n_b, x2, None)])
        for o in range(n_a):
            want = oracle.matvec_fused_batch([(Q4_K, wa[o * 144:(o + 1) * 144], 256, 1, x1, q8)])[0]
            assert out[o] == want
        for o in range(n_b):
            assert out[n_a + o] == oracle.fused_row_dot(Q6_K, wb[o * 210:(o + 1) * 210], x2)


def lcg(seed):
    state = seed
    M = (1 << 64) - 1
    while True:
        state = (state * 6364136223846793005 + 1442695040888963407) & M
        yield state >> 33


def realistic_q4k_block():  # matmul.rs:1318-1340
    nx = lcg(0x2545F4914F6CDD1D)
    block = np.zeros(144, np.uint8)
    block[0:2] = [0x00, 0x10]
    block[2:4] = [0x00, 0x1C]
    for i in range(4, 16):
        block[i] = 16 + next(nx) % 32
    for i in range(16, 144):
        block[i] = next(nx) & 0xFF
    x = np.array([np.float32(next(nx) % 2000) / np.float32(1000.0) - np.float32(1.0) for _ in range(256)], np.float32)
    return block, x


def realistic_q6k_block():  # matmul.rs:1376-1398
    nx = lcg(0x9E3779B97F4A7C15)
    block = np.zeros(210, np.uint8)
    block[208:210] = [0x00, 0x1C]
    for i in range(0, 128):
        block[i] = next(nx) & 0xFF
    for i in range(128, 192):
        block[i] = next(nx) & 0xFF
    for i in range(192, 208):
        block[i] = 8 + next(nx) % 32
    x = np.array([np.float32(next(nx) % 2000) / np.float32(1000.0) - np.float32(1.0) for _ in range(256)], np.float32)
    return block, x


def test_dot_q4k_block_q8_precision_vs_fp32(oracle):  # matmul.rs:1342-1363
    block, x = realistic_q4k_block()
    ref = f32_seq_sum(oracle.dequantize(Q4_K, block, 256) * x)
    a = oracle.quantize_q8(x)
    got = np.float32(oracle.dot_q4k_block_q8(block, a.q, a.scales[0], a.sums[:8]))
    rel = np.float32(abs(np.float32(got - ref)) / abs(ref))
    assert rel < 0.0045
    assert f"{rel:.7f}" == "0.0041545"  # the value the reference's comment reports


def test_dot_q6k_block_q8_precision_vs_fp32(oracle):  # matmul.rs:1400-1421
    block, x = realistic_q6k_block()
    ref = f32_seq_sum(oracle.dequantize(Q6_K, block, 256) * x)
    a = oracle.quantize_q8(x)
    got = np.float32(oracle.dot_q6k_block_q8(block, a.q, a.scales[0]))
    rel = np.float32(abs(np.float32(got - ref)) / abs(ref))
    assert rel < 0.0062
    assert f"{rel:.7f}" == "0.0057328"


def test_q6k_block_idot_portable_matches_buffered(oracle):  # matmul.rs:1423-1436
    for seed in range(4):
        block = q6k_matrix(1, seed * 7)
        x = (((np.arange(256) * 13 + seed) % 17).astype(np.float32) * np.float32(0.05) - np.float32(0.4)).astype(np.float32)
        q8 = oracle.quantize_q8(x)
        assert oracle.q6k_block_idot(block, q8.q) == oracle.q6k_block_idot(block, q8.q, buffered=True)


def assert_matmul_eq_per_token(oracle, dtype, w, n_in, n_out, n_tokens):  # matmul.rs:1490-1499
    x = (((np.arange(n_in * n_tokens) % 11).astype(np.float32) - 5) * np.float32(0.05)).astype(np.float32)
    batched = oracle.matmul(dtype, w, n_in, n_out, x, n_tokens)
    for t in range(n_tokens):
        single = oracle.matvec(dtype, w, n_in, n_out, x[t * n_in:(t + 1) * n_in])
        assert np.array_equal(batched[t * n_out:(t + 1) * n_out].view(np.uint32), single.view(np.uint32)), (dtype, t)


def test_matmul_matches_per_token_matvec(oracle):  # matmul.rs:1501-1510
    for n_out in [50, 100]:
        assert_matmul_eq_per_token(oracle, Q4_K, q4k_matrix(n_out, 3), 256, n_out, 4)
        assert_matmul_eq_per_token(oracle, Q6_K, q6k_matrix(n_out, 7), 256, n_out, 4)
        f32w = ((np.arange(2 * n_out, dtype=np.float32) - np.float32(3.0)) * np.float32(0.1)).astype(np.float32)
        assert_matmul_eq_per_token(oracle, F32, f32w.view(np.uint8), 2, n_out, 4)


def test_matmul_single_token_matches_matvec(oracle):  # matmul.rs:1512-1516
    assert_matmul_eq_per_token(oracle, Q4_K, q4k_matrix(80, 1), 256, 80, 1)


def test_matvec_fused_batch_q4k_without_qx_falls_back_to_f32(oracle):  # matmul.rs:1518-1530
    x = (((np.arange(256) % 7).astype(np.float32) - 3) * np.float32(0.1)).astype(np.float32)
    w = q4k_matrix(4, 7)
    out = oracle.matvec_fused_batch([(Q4_K, w, 256, 4, x, None)])
    for o in range(4):
        assert out[o] == oracle.fused_row_dot(Q4_K, w[o * 144:(o + 1) * 144], x)


def test_matvec_fused_batch_q6k_with_qx_uses_int_dot(oracle):  # matmul.rs:1532-1548
    x = (((np.arange(256) % 5).astype(np.float32) - 2) * np.float32(0.07)).astype(np.float32)
    q8 = oracle.quantize_q8(x)
    for n_out in [4, 80]:
        w = q6k_matrix(n_out, 99)
        out = oracle.matvec_fused_batch([(Q6_K, w, 256, n_out, x, q8)])
        for o in range(n_out):
            row = w[o * 210:(o + 1) * 210]
            assert out[o] == np.float32(oracle.dot_q6k_block_q8(row, q8.q, q8.scales[0])) + np.float32(-0.0)


# ---- activation.rs:31-63, elementwise.rs:23-35, rmsnorm.rs:123-217 ----

def test_sigmoid_silu_values(oracle):  # activation.rs:35-46
    assert abs(oracle.sigmoid(0.0) - 0.5) < 1e-7
    assert oracle.sigmoid(-100.0) < 1e-6
    assert oracle.sigmoid(100.0) > 1.0 - 1e-6
    assert oracle.silu(0.0) == 0.0
    assert abs(oracle.silu(1.0) - 0.7310586) < 1e-6
    assert abs(oracle.silu(20.0) - 20.0) < 1e-3


def test_swiglu_glue(oracle):  # activation.rs:48-56
    out = oracle.swiglu([0.0, 1.0], [5.0, 2.0])
    assert out[0] == 0.0
    assert abs(out[1] - 0.7310586 * 2.0) < 1e-6


def test_add_and_scaled_accumulate(oracle):  # elementwise.rs:24-35
    assert oracle.add_assign([1, 2, 3], [10, 20, 30]).tolist() == [11, 22, 33]
    assert oracle.add_scaled([1, 1, 1], [2, 4, 6], 0.5).tolist() == [2, 3, 4]


def test_rmsnorm_normalizes_to_unit_rms(oracle):  # rmsnorm.rs:127-142
    out = oracle.rmsnorm(np.array([1, 2, 3, 4], np.float32), np.ones(4, np.float32), 0.0)
    ms = f32_seq_sum(out * out) / np.float32(4.0)
    assert abs(ms - 1.0) < 1e-5
    s = np.float32(1.0) / np.sqrt(np.float32(7.5))
    assert abs(out[0] - s) < 1e-6 and abs(out[3] - 4 * s) < 1e-6


def test_rmsnorm_applies_gain(oracle):  # rmsnorm.rs:144-152
    out = oracle.rmsnorm(np.ones(4, np.float32), np.array([2.0, 0.5, 1.0, 3.0], np.float32), 0.0)
    assert out.tolist() == [2.0, 0.5, 1.0, 3.0]


def test_rmsnorm_sum_of_squares_uses_wide_accumulator(oracle):  # rmsnorm.rs:164-208
    n = 4096
    i = np.arange(n)
    x = np.where(i < 8, np.float32(50.0), np.float32(0.05) * ((i % 7).astype(np.float32) - np.float32(3.0))).astype(np.float32)
    eps = 1e-5
    ss64 = np.sum(x.astype(np.float64) ** 2)
    scale64 = 1.0 / np.sqrt(ss64 / n + eps)
    ref = (x.astype(np.float64) * scale64).astype(np.float32)
    out = oracle.rmsnorm(x, np.ones(n, np.float32), eps)
    got = np.max(np.abs(out - ref) / np.maximum(np.abs(ref), 1e-6))
    assert got < 3e-7


def test_rmsnorm_eps_guards_zero_input(oracle):  # rmsnorm.rs:210-217
    assert oracle.rmsnorm(np.zeros(4, np.float32), np.ones(4, np.float32), 1e-5).tolist() == [0, 0, 0, 0]
