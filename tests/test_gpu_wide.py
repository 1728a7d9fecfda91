"""GPU parity of the batched path at group sizes that take the grouped GEMM for large groups
(k_gemm_wide: blocks of up to 256 members x 128 rows), which Q6_K down GEMMs whose experts
average at least 192 members run (config 4 at full size does); the other GEMMs of these calls
run k_gemm with tiles of 64 members.

Bit-exact against the CPU restatement of Model::moe_ffn_batch (model.rs:286-371): the shapes
cover groups that end mid-tile and mid-chunk, groups of exactly one and several 256-member
chunks, 1, 2, 3 and 7 super-blocks per row (odd counts end the kernel's two-stage loop early),
and Q4_K / Q6_K in both GEMMs.
"""
import numpy as np
import pytest

from bebelm_amd import synth

from test_gpu_parity import Q4_K, Q6_K, check_moe, log

pytestmark = pytest.mark.gpu

WIDE_MIN_AVG = 192  # members per expert on average from which Q6_K down GEMMs take the wide kernel


def wide(t, k, e):
    return t * k >= WIDE_MIN_AVG * e


@pytest.mark.parametrize("hidden,ff,down", [(512, 512, Q6_K), (768, 256, Q4_K), (256, 768, Q6_K),
                                            (1792, 512, Q4_K)])
def test_wide_shapes(gpu_ctx, oracle, hidden, ff, down):
    t, k, e = 400, 2, 4
    assert wide(t, k, e)
    w = synth.moe_weights(61, hidden=hidden, moe_ff=ff, n_experts=e, n_used=k, down_dtype=down)
    x = synth.hidden_states(62, t, hidden=hidden)
    log(f"wide hidden={hidden} ff={ff} down={down}")
    _, tr = check_moe(gpu_ctx, oracle, w, x, t, f"wide {hidden}x{ff}")
    assert tr.counts.sum() == t * k


def test_wide_q6k_gate_up(gpu_ctx, oracle):
    t, k, e = 640, 4, 8
    assert wide(t, k, e)
    w = synth.moe_weights(63, hidden=512, moe_ff=512, n_experts=e, n_used=k, down_dtype=Q6_K, gate_dtype=Q6_K)
    x = synth.hidden_states(64, t, hidden=512)
    check_moe(gpu_ctx, oracle, w, x, t, "wide q6k gate/up")


@pytest.mark.parametrize("t", [256, 300, 513])
def test_wide_every_token_same_experts(gpu_ctx, oracle, t):
    # all four experts take every token: groups of exactly 1, 2 and 3 tiles (the last partial)
    bias = np.array([4.0, 3.0, 2.0, 1.0], np.float32)
    w = synth.moe_weights(65, hidden=512, moe_ff=256, n_experts=4, n_used=4, bias=bias)
    x = synth.hidden_states(66, t, hidden=512)
    _, tr = check_moe(gpu_ctx, oracle, w, x, t, f"wide all-same t={t}")
    assert tr.counts.tolist() == [t] * 4


def test_wide_skewed_groups(gpu_ctx, oracle):
    # a Zipf selection bias over 8 experts: groups from a few dozen to over a thousand members
    bias = synth.zipf_bias(7, n_experts=8, kappa=1.5)
    t, k, e = 1024, 2, 8
    assert wide(t, k, e)
    w = synth.moe_weights(67, hidden=512, moe_ff=512, n_experts=e, n_used=k, down_dtype=Q6_K, bias=bias)
    x = synth.hidden_states(68, t, hidden=512)
    _, tr = check_moe(gpu_ctx, oracle, w, x, t, "wide skewed")
    log(f"wide skewed counts {tr.counts.tolist()}")
