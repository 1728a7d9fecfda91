"""GPU parity of the Q4_K GEMMs of decode batches (at most 16 tokens, T*k <= 64) on the grouped
path: the gate/up kernel k_gateup16 (hidden 512 or 2048, member tiles of every token of the batch,
weight rows streamed into registers, 16-wave blocks over 256 outputs of one expert that also write
the act rows' Q8) and, where the down experts are Q4_K, the down kernel k_down16 (the expert's at
most 16 members, act Q8 rows at 16e + m, 16-wave blocks over 256 rows), against the CPU
restatement of Model::moe_ffn_batch (model.rs:286-371): routing, weights and block outputs
bit-identical. The cases reach their edges: a single expert, experts nobody chose (their blocks
leave early), one-member experts (sums started at -0.0), k = 8 with 8 tokens (64 entries), k = E,
moe_ff of 1, 3, 4, 5, 7 and 8 act super-blocks, zero and scaled input rows (a zero act block
quantises to scale 0).
"""
import numpy as np
import pytest

from bebelm_amd import synth

from test_gpu_parity import Q4_K, Q6_K, check_moe

pytestmark = pytest.mark.gpu

DEFAULT_MIN_ENTRIES = 64


@pytest.fixture
def batched(gpu_ctx):
    gpu_ctx.set_batched_min_entries(1)
    yield gpu_ctx
    gpu_ctx.set_batched_min_entries(DEFAULT_MIN_ENTRIES)


# (seed, hidden, moe_ff, experts, k, tokens, down)
CASES = [
    (1, 512, 512, 1, 1, 3, Q4_K),      # one expert: every token its member
    (2, 512, 256, 32, 4, 1, Q4_K),     # 4 one-member experts, 28 nobody chose; one block each
    (3, 512, 1792, 32, 4, 16, Q6_K),   # the decode-batch shape at hidden 512
    (4, 2048, 1792, 32, 8, 8, Q4_K),   # 64 entries, k = 8
    (5, 2048, 1024, 13, 3, 11, Q4_K),   # 13 experts x 4 blocks
    (6, 2048, 256, 5, 5, 12, Q6_K),    # k = E: every token chooses every expert
    (7, 512, 1280, 7, 2, 16, Q4_K),    # moe_ff 1280: 5 blocks per expert, 40 packed tiles
    (8, 2048, 1792, 32, 4, 2, Q6_K),
    (9, 512, 2048, 16, 2, 16, Q4_K),   # moe_ff 2048: k_down16 over 8 act super-blocks, 2 blocks per expert
    (10, 2048, 768, 32, 4, 16, Q4_K),  # moe_ff 768: k_down16 over 3, the padded act rows of 32 experts
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"s{c[0]}-H{c[1]}-F{c[2]}-E{c[3]}-k{c[4]}-T{c[5]}")
def test_decode_batch_gate_up(batched, oracle, case):
    seed, hidden, ff, E, K, T, down = case
    w = synth.moe_weights(600 + seed, hidden=hidden, moe_ff=ff, n_experts=E, n_used=K, gate_dtype=Q4_K,
                          down_dtype=down)
    x = synth.hidden_states(700 + seed, T, hidden=hidden)
    check_moe(batched, oracle, w, x, T, f"gateup16 case {seed}")


def test_decode_batch_gate_up_zero_and_scaled_rows(batched, oracle):
    w = synth.moe_weights(620, hidden=512, moe_ff=512, n_experts=8, n_used=2)
    x = synth.hidden_states(720, 9, hidden=512)
    x[0] = 0.0
    x[3, :256] = 0.0
    x[6] *= np.float32(1e3)
    check_moe(batched, oracle, w, x, 9, "gateup16 zero/scaled rows")


def test_decode_batch_at_default_threshold(gpu_ctx, oracle):
    # 16 tokens x k = 4 = 64 entries: the default batched threshold, the config-2 path
    w = synth.moe_weights(630, hidden=2048, moe_ff=1792, n_experts=32, n_used=4)
    x = synth.hidden_states(730, 16, hidden=2048)
    check_moe(gpu_ctx, oracle, w, x, 16, "gateup16 at the default threshold")
