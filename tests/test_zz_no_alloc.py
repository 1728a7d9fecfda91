"""bb_moe_forward_noalloc (the allocation-free MoE entry point) against bb_moe_forward.

The allocation-free entry point runs the same kernels with its workspace in the library's
static per-GPU scratch area. Its outputs must equal bb_moe_forward's bit for bit, on two calls
in a row (the second with fewer tokens, so it runs on the scratch area the first one left
behind, and on the other kernel path), and a call too large for the area must fail on the host
with BB_ERR_RANGE before any kernel runs.
"""
import numpy as np
import pytest

from bebelm_amd import _lib, synth
from bebelm_amd.model import MoeLayer

pytestmark = pytest.mark.gpu


def noalloc(ctx, layer, x, t, out):
    return _lib.lib().bb_moe_forward_noalloc(ctx.handle, layer.handle, x.data_ptr(), t, out.data_ptr())


def test_noalloc_matches_forward(gpu_ctx, oracle):
    import torch

    w = synth.config_layer(4, seed=11, layer=0)  # Q4_K gate/up, Q6_K down, Zipf selection bias
    layer = MoeLayer(gpu_ctx, w)
    try:
        for t in (16, 3):  # batched grouped-GEMM path, then the GEMV path with the route inside
            print(f"noalloc: T={t}", flush=True)
            xh = synth.hidden_states(23, t)
            x = torch.from_numpy(xh).cuda()
            want = torch.empty_like(x)
            got = torch.full_like(x, float("nan"))
            torch.cuda.synchronize()
            layer.forward(x, t, want)
            gpu_ctx.synchronize()
            _lib.check(noalloc(gpu_ctx, layer, x, t, got))
            gpu_ctx.synchronize()
            g, wv = got.cpu().numpy(), want.cpu().numpy()
            assert np.array_equal(g.view(np.uint32), wv.view(np.uint32)), f"T={t}: noalloc differs from bb_moe_forward"
            if t == 3:
                ref = oracle.moe_ffn_batch(w, xh, t)
                assert np.array_equal(g.reshape(-1).view(np.uint32), ref.reshape(-1).view(np.uint32)), \
                    "T=3: noalloc differs from the CPU restatement"
        # 4096 tokens need about 300 MB of workspace: refused on the host, nothing launched
        big = torch.zeros((4096, w.hidden), dtype=torch.float32, device="cuda")
        out = torch.empty_like(big)
        torch.cuda.synchronize()
        rc = noalloc(gpu_ctx, layer, big, 4096, out)
        assert rc == _lib.BB_ERR_RANGE, rc
        assert b"scratch" in _lib.lib().bb_last_error()
    finally:
        layer.close()


def test_noalloc_at_the_scratch_limit(gpu_ctx):
    # hidden = ff = 2048, 32 experts, k = 4: 440 tokens fill the scratch area up to its tail
    # slack (the padding every allocated workspace has); 441 tokens are refused.
    import torch

    w = synth.moe_weights(5, hidden=2048, moe_ff=2048)
    layer = MoeLayer(gpu_ctx, w)
    try:
        for t in (440, 17):
            print(f"noalloc: T={t} (hidden = ff = 2048)", flush=True)
            x = torch.from_numpy(synth.hidden_states(29, t)).cuda()
            want = torch.empty_like(x)
            got = torch.full_like(x, float("nan"))
            torch.cuda.synchronize()
            layer.forward(x, t, want)
            gpu_ctx.synchronize()
            _lib.check(noalloc(gpu_ctx, layer, x, t, got))
            gpu_ctx.synchronize()
            assert np.array_equal(got.cpu().numpy().view(np.uint32), want.cpu().numpy().view(np.uint32)), \
                f"T={t}: noalloc differs from bb_moe_forward"
        x = torch.zeros((441, 2048), dtype=torch.float32, device="cuda")
        out = torch.empty_like(x)
        torch.cuda.synchronize()
        assert noalloc(gpu_ctx, layer, x, 441, out) == _lib.BB_ERR_RANGE
        assert b"scratch" in _lib.lib().bb_last_error()
    finally:
        layer.close()
