"""Kernel-level mirror of the reference's src/kernels API over the C ABI.

  quantize_q8(x) -> Q8Vec                  kernels/matmul.rs:141
  matvec(dtype, w, n_in, n_out, x, y)      kernels/matmul.rs:850
  matmul(dtype, w, n_in, n_out, x, t, y)   kernels/matmul.rs:908
  FusedJob / matvec_fused_batch            kernels/matmul.rs:995-1053
  swiglu / sigmoid_slice                   kernels/activation.rs:16, :25
  add_scaled / add_assign                  kernels/elementwise.rs:12, :4
  rmsnorm                                  kernels/rmsnorm.rs:10
  logits_from_hidden                       model.rs:380-388
  conv_step / conv_prefill                 kernels/conv.rs:18, :48
  softmax                                  kernels/softmax.rs:9
  attention_decode                         kernels/attention.rs:17
  rope_neox                                kernels/rope.rs:17
Each function takes the Context first; `w` is an uploaded Tensor (plus a byte offset where the
reference passes a sub-slice of the weight bytes).
"""
import ctypes
from dataclasses import dataclass

import numpy as np

from . import _lib
from ._lib import check, lib
from .model import _ptr, _same_loc


@dataclass
class Q8Vec:
    q: object       # int8 [n]
    scales: object  # f32 [n/256]
    sums: object    # i32 [n/32]


def quantize_q8(ctx, x, out=None):
    n = x.shape[-1] if hasattr(x, "shape") else len(x)
    if out is None:
        out = Q8Vec(np.empty(n, np.int8), np.empty(n // 256, np.float32), np.empty(n // 32, np.int32))
    loc = _same_loc(x, out.q, out.scales, out.sums)
    check(lib().bb_quantize_q8(ctx.handle, _ptr(x)[0], n, _ptr(out.q)[0], _ptr(out.scales)[0], _ptr(out.sums)[0], loc))
    return out


def matvec(ctx, dtype, w, n_in, n_out, x, y, byte_off=0):
    loc = _same_loc(x, y)
    check(lib().bb_matvec(ctx.handle, dtype, w.handle, byte_off, n_in, n_out, _ptr(x)[0], _ptr(y)[0], loc))
    return y


def matmul(ctx, dtype, w, n_in, n_out, x, n_tokens, y, byte_off=0):
    loc = _same_loc(x, y)
    check(lib().bb_matmul(ctx.handle, dtype, w.handle, byte_off, n_in, n_out, _ptr(x)[0], n_tokens, _ptr(y)[0], loc))
    return y


@dataclass
class FusedJob:
    """FusedJob (matmul.rs:995-1005): qx (Q8Vec) for the integer dot, or qx None and x (f32) for
    the f32 fused dot."""
    dtype: int
    w: object
    n_in: int
    n_out: int
    qx: object = None
    byte_off: int = 0
    x: object = None


def matvec_fused_batch(ctx, jobs, out):
    arr = (_lib.FusedJob * len(jobs))()
    arrays = [out]
    for i, j in enumerate(jobs):
        if j.qx is not None:
            arr[i] = _lib.FusedJob(j.dtype, j.w.handle, j.byte_off, j.n_in, j.n_out, _ptr(j.qx.q)[0],
                                   _ptr(j.qx.scales)[0], _ptr(j.qx.sums)[0], None)
            arrays += [j.qx.q, j.qx.scales, j.qx.sums]
        else:
            arr[i] = _lib.FusedJob(j.dtype, j.w.handle, j.byte_off, j.n_in, j.n_out, None, None, None, _ptr(j.x)[0])
            arrays += [j.x]
    loc = _same_loc(*arrays)
    check(lib().bb_matvec_fused_batch(ctx.handle, arr, len(jobs), _ptr(out)[0], loc))
    return out


def swiglu(ctx, gate, up, out):
    check(lib().bb_swiglu(ctx.handle, _ptr(gate)[0], _ptr(up)[0], _ptr(out)[0], _n(out), _same_loc(gate, up, out)))
    return out


def sigmoid_slice(ctx, x):
    check(lib().bb_sigmoid_slice(ctx.handle, _ptr(x)[0], _n(x), _same_loc(x)))
    return x


def add_scaled(ctx, out, b, s):
    check(lib().bb_add_scaled(ctx.handle, _ptr(out)[0], _ptr(b)[0], ctypes.c_float(s), _n(out), _same_loc(out, b)))
    return out


def add_assign(ctx, a, b):
    check(lib().bb_add_assign(ctx.handle, _ptr(a)[0], _ptr(b)[0], _n(a), _same_loc(a, b)))
    return a


def rmsnorm(ctx, x, gain, eps, out, n_vec=1):
    n = _n(gain)
    check(lib().bb_rmsnorm(ctx.handle, _ptr(x)[0], _ptr(gain)[0], ctypes.c_float(eps), n, n_vec, _ptr(out)[0],
                           _same_loc(x, gain, out)))
    return out


def logits_from_hidden(ctx, tok_embd, gain, eps, h, logits):
    """Model::logits_from_hidden (model.rs:380-388): rmsnorm, then the token_embd matvec."""
    loc = _same_loc(h, gain, logits)
    check(lib().bb_logits_from_hidden(ctx.handle, tok_embd.handle, _ptr(gain)[0], eps, _ptr(h)[0], _ptr(logits)[0], loc))
    return logits


def conv_step(ctx, state, bx, weight, channels, l_cache, out):
    """conv.rs:18-39: out[c] = w[c, L-1]·bx[c] + Σ_k w[c, k]·state[k, c]."""
    loc = _same_loc(state, bx, weight, out)
    check(lib().bb_conv_step(ctx.handle, _ptr(state)[0], _ptr(bx)[0], _ptr(weight)[0], channels, l_cache, _ptr(out)[0],
                             loc))
    return out


def conv_prefill(ctx, state, bx, weight, channels, l_cache, n_tokens, out):
    """conv.rs:48-68 over n_tokens positions; state is updated in place."""
    loc = _same_loc(state, bx, weight, out)
    check(lib().bb_conv_prefill(ctx.handle, _ptr(state)[0], _ptr(bx)[0], _ptr(weight)[0], channels, l_cache, n_tokens,
                                _ptr(out)[0], loc))
    return out


def softmax(ctx, x, n_vec=1):
    """softmax.rs:9-22 on each of n_vec rows, in place."""
    n = _n(x) // n_vec
    check(lib().bb_softmax(ctx.handle, _ptr(x)[0], n, n_vec, _same_loc(x)))
    return x


def attention_decode(ctx, q, k, v, n_ctx, n_heads, n_kv_heads, head_dim, out):
    """attention.rs:17-55."""
    loc = _same_loc(q, k, v, out)
    check(lib().bb_attention_decode(ctx.handle, _ptr(q)[0], _ptr(k)[0], _ptr(v)[0], n_ctx, n_heads, n_kv_heads,
                                    head_dim, _ptr(out)[0], loc))
    return out


def rope_neox(ctx, x, head_dim, pos, freq_base):
    """rope.rs:17-30 on each head vector of x, in place."""
    check(lib().bb_rope_neox(ctx.handle, _ptr(x)[0], head_dim, _n(x) // head_dim, pos, ctypes.c_float(freq_base),
                             _same_loc(x)))
    return x


def _n(a):
    return a.numel() if hasattr(a, "numel") else a.size
