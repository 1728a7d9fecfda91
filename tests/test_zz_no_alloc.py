"""bb_moe_forward_noalloc (the allocation-free MoE entry point) against bb_moe_forward.

The allocation-free entry point runs the same kernels with its workspace in the library's
static per-GPU scratch area. Its outputs must equal bb_moe_forward's bit for bit, on two calls
in a row (the second with fewer tokens, so it runs on the scratch area the first one left
behind, and on the other kernel path), and a call too large for the area must fail on the host
with BB_ERR_RANGE before any kernel runs. Captured into a HIP graph (the callers it is for), its
replays must equal bb_moe_forward too, with eager work between them.
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


def test_noalloc_replayed_from_a_hip_graph(gpu_ctx):
    # the caller the entry point is for: a HIP graph captured around it (on a torch side stream),
    # replayed several times with eager library and torch work in between; every replay must
    # equal the eager bb_moe_forward of the same input bit for bit
    import torch

    w = synth.config_layer(2, seed=13)  # 16 tokens: the grouped-GEMM path of config 2
    layer = MoeLayer(gpu_ctx, w)
    s = torch.cuda.Stream()
    try:
        xs = [torch.from_numpy(synth.hidden_states(40 + i, 16)).cuda() for i in range(2)]
        wants = [torch.empty_like(x) for x in xs]
        torch.cuda.synchronize()
        for x, want in zip(xs, wants):
            layer.forward(x, 16, want)
        gpu_ctx.synchronize()
        x_in = xs[0].clone()
        out = torch.full_like(x_in, float("nan"))
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        print("noalloc: capturing a graph of one call (T=16)", flush=True)
        with torch.cuda.graph(g, stream=s):
            gpu_ctx.set_stream(s.cuda_stream)
            _lib.check(noalloc(gpu_ctx, layer, x_in, 16, out))
        gpu_ctx.set_stream(None)
        torch.cuda.synchronize()
        for r in range(4):
            i = r % 2
            print(f"noalloc: graph replay {r} (input {i})", flush=True)
            x_in.copy_(xs[i])
            out.fill_(float("nan"))
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert np.array_equal(out.cpu().numpy().view(np.uint32), wants[i].cpu().numpy().view(np.uint32)), \
                f"replay {r}: the graph's output differs from bb_moe_forward"
            # eager work between replays, on the context's own stream and on torch's
            tmp = torch.empty_like(x_in)
            layer.forward(xs[1 - i], 16, tmp)
            gpu_ctx.synchronize()
            assert torch.equal(tmp, wants[1 - i])
    finally:
        gpu_ctx.set_stream(None)
        torch.cuda.synchronize()
        layer.close()
