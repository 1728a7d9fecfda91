"""Host-side mirror of the reference's MoE FFN interface over the C ABI.

Names follow the reference so call sites read alike:
  Model::moe_ffn / moe_ffn_batch (model.rs:473, :286)  -> MoeLayer.moe_ffn / moe_ffn_batch
  Model::dense_ffn (model.rs:459)                       -> DenseLayer.dense_ffn
  run_layers' FFN path (model.rs:105-130)               -> FfnStack.run_layers
  Model::conv_step_op / conv_batch (model.rs:399, :190) -> ConvOp.forward
  Model::attn_step / attn_batch (model.rs:430, :222)    -> AttnOp.forward (KvCache: cache.rs)
  Model::run_layers(_batch) / forward_step, Agent::absorb -> Model (model.rs:97-181, agent.rs:454)
  Cache (cache.rs:10-49), Cache: Clone                  -> Cache (Model.new_cache, Cache.clone)
Arrays are numpy (host memory, BB_LOC_HOST) or torch CUDA tensors (device memory,
BB_LOC_DEVICE). Everything runs on the GPU through libbebelm_moe.so; there is no other path.
"""
import ctypes

import numpy as np

from . import _lib
from ._lib import LOC_DEVICE, LOC_HOST, check, lib


def _ptr(a):
    """(pointer, loc) for a numpy array or a torch tensor."""
    if a is None:
        return None, LOC_HOST
    if isinstance(a, np.ndarray):
        if not a.flags["C_CONTIGUOUS"]:
            raise ValueError("arrays must be C-contiguous")
        return a.ctypes.data, LOC_HOST
    if hasattr(a, "data_ptr"):
        if not a.is_contiguous():
            raise ValueError("tensors must be contiguous")
        return a.data_ptr(), (LOC_DEVICE if a.is_cuda else LOC_HOST)
    raise TypeError(f"unsupported array type {type(a)}")


def _same_loc(*arrays):
    locs = {_ptr(a)[1] for a in arrays if a is not None}
    if len(locs) != 1:
        raise ValueError("all arrays of one call must be host or all device")
    return locs.pop()


class Context:
    def __init__(self, device=0):
        h = ctypes.c_void_p()
        check(lib().bb_ctx_create(device, ctypes.byref(h)))
        self.handle = h
        self.device = device

    def close(self):
        if self.handle:
            check(lib().bb_ctx_destroy(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def synchronize(self):
        check(lib().bb_ctx_synchronize(self.handle))

    def set_stream(self, stream_ptr):
        check(lib().bb_ctx_set_stream(self.handle, stream_ptr))

    def stream(self):
        s = ctypes.c_void_p()
        check(lib().bb_ctx_get_stream(self.handle, ctypes.byref(s)))
        return s.value

    def profile(self, enable=True):
        check(lib().bb_ctx_profile(self.handle, 1 if enable else 0))

    def reset_stats(self):
        check(lib().bb_ctx_reset_stats(self.handle))

    def set_batched_min_entries(self, n):
        """MoE calls with T*k >= n take the grouped-GEMM (batched) kernels."""
        check(lib().bb_ctx_set_batched_min_entries(self.handle, int(n)))

    def kernel_stats(self):
        """{kernel name: (total ms, launches)} for kernels launched while profiling."""
        out = {}
        for i in range(lib().bb_kernel_count()):
            name = ctypes.c_char_p()
            ms = ctypes.c_double()
            n = ctypes.c_int64()
            check(lib().bb_ctx_kernel_stats(self.handle, i, ctypes.byref(name), ctypes.byref(ms), ctypes.byref(n)))
            if n.value:
                out[name.value.decode()] = (ms.value, n.value)
        return out


class Tensor:
    """A weight tensor uploaded once to HBM in its native GGUF block layout."""

    def __init__(self, ctx, dtype, data, dims):
        data = np.ascontiguousarray(data)
        raw = data.view(np.uint8).reshape(-1)
        d = (ctypes.c_uint64 * len(dims))(*dims)
        h = ctypes.c_void_p()
        check(lib().bb_tensor_upload(ctx.handle, dtype, raw.ctypes.data, raw.nbytes, d, len(dims), ctypes.byref(h)))
        self.handle = h
        self.ctx = ctx
        self.dtype = dtype
        self.dims = tuple(dims)
        self.nbytes = raw.nbytes

    def close(self):
        if self.handle:
            check(lib().bb_tensor_free(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class RouteTrace:
    """Host copies of one call's routing state (bb_route_trace)."""

    def __init__(self, t, n_experts, k):
        self.logits = np.zeros(t * n_experts, np.float32)
        self.sel = np.zeros(t * k, np.int32)
        self.w = np.zeros(t * k, np.float32)
        self.counts = np.zeros(n_experts, np.int32)
        self.offsets = np.zeros(n_experts + 1, np.int32)
        self.perm = np.zeros(t * k, np.int32)
        self.ties = np.zeros(1, np.int32)
        self.margin = np.zeros(t, np.float32)

    def as_struct(self):
        return _lib.RouteTrace(*(a.ctypes.data for a in (self.logits, self.sel, self.w, self.counts, self.offsets,
                                                         self.perm, self.ties, self.margin)))


class MoeLayer:
    """One sparse-MoE FFN layer (router, exp_probs_b, stacked gate/up/down experts)."""

    def __init__(self, ctx, weights, n_used=None):
        w = weights
        self.ctx = ctx
        self.hidden, self.moe_ff, self.n_experts = w.hidden, w.moe_ff, w.n_experts
        self.n_used = n_used or w.n_used
        E, H, F = w.n_experts, w.hidden, w.moe_ff
        self.router = Tensor(ctx, 0, w.router, (H, E))
        self.gate = Tensor(ctx, w.gate_dtype, w.gate_exps, (H, F, E))
        self.up = Tensor(ctx, w.up_dtype, w.up_exps, (H, F, E))
        self.down = Tensor(ctx, w.down_dtype, w.down_exps, (F, H, E))
        bias = np.ascontiguousarray(w.exp_probs_b, np.float32)
        h = ctypes.c_void_p()
        try:
            check(lib().bb_moe_create(ctx.handle, self.router.handle, bias.ctypes.data, self.gate.handle,
                                      self.up.handle, self.down.handle, self.n_used, ctypes.byref(h)))
        finally:
            # the layer keeps its own regrouped copies: the uploads are freed at once, so each
            # layer occupies its packed bytes in HBM only
            for t in (self.router, self.gate, self.up, self.down):
                t.close()
        self.handle = h

    def close(self):
        if self.handle:
            check(lib().bb_moe_destroy(self.handle))
            self.handle = None

    def forward(self, x, t, out, trace=None):
        """x, out: token-major [t, hidden]; numpy (host) or torch CUDA (device, async)."""
        loc = _same_loc(x, out)
        tr = trace.as_struct() if trace is not None else None
        check(lib().bb_moe_forward(self.ctx.handle, self.handle, _ptr(x)[0], t, _ptr(out)[0], loc,
                                   ctypes.byref(tr) if tr is not None else None))
        return out

    def moe_ffn(self, x, trace=None):
        """Model::moe_ffn (model.rs:473-555): one token, host arrays."""
        x = np.ascontiguousarray(x, np.float32).reshape(self.hidden)
        out = np.empty(self.hidden, np.float32)
        return self.forward(x, 1, out, trace)

    def moe_ffn_batch(self, x, t, trace=None):
        """Model::moe_ffn_batch (model.rs:286-371): t tokens, token-major host arrays."""
        x = np.ascontiguousarray(x, np.float32).reshape(t * self.hidden)
        out = np.empty(t * self.hidden, np.float32)
        return self.forward(x, t, out, trace)


class DenseLayer:
    def __init__(self, ctx, weights):
        w = weights
        self.ctx = ctx
        self.hidden, self.ff = w.hidden, w.ff
        self.gate = Tensor(ctx, w.gate_dtype, w.gate, (w.hidden, w.ff))
        self.up = Tensor(ctx, w.up_dtype, w.up, (w.hidden, w.ff))
        self.down = Tensor(ctx, w.down_dtype, w.down, (w.ff, w.hidden))
        h = ctypes.c_void_p()
        check(lib().bb_dense_create(ctx.handle, self.gate.handle, self.up.handle, self.down.handle, ctypes.byref(h)))
        self.handle = h

    def close(self):
        if self.handle:
            check(lib().bb_dense_destroy(self.handle))
            self.handle = None
        for t in (self.gate, self.up, self.down):
            t.close()

    def forward(self, x, t, out):
        loc = _same_loc(x, out)
        check(lib().bb_dense_forward(self.ctx.handle, self.handle, _ptr(x)[0], t, _ptr(out)[0], loc))
        return out

    def dense_ffn(self, x):
        """Model::dense_ffn (model.rs:459-469)."""
        x = np.ascontiguousarray(x, np.float32).reshape(self.hidden)
        out = np.empty(self.hidden, np.float32)
        return self.forward(x, 1, out)


class FfnStack:
    """run_layers' FFN path with the operator sub-layer contributing nothing (model.rs:105-130)."""

    def __init__(self, ctx, layers, eps=1e-5):
        """layers: list of (ffn_norm gain f32[hidden], MoeLayer | DenseLayer)."""
        self.ctx = ctx
        self.layers = layers
        self.hidden = layers[0][1].hidden
        self._gains = [np.ascontiguousarray(g, np.float32) for g, _ in layers]
        descs = (_lib.LayerDesc * len(layers))()
        for i, ((_, layer), g) in enumerate(zip(layers, self._gains)):
            descs[i].ffn_norm = g.ctypes.data
            descs[i].moe = layer.handle if isinstance(layer, MoeLayer) else None
            descs[i].dense = layer.handle if isinstance(layer, DenseLayer) else None
        h = ctypes.c_void_p()
        check(lib().bb_stack_create(ctx.handle, descs, len(layers), eps, ctypes.byref(h)))
        self.handle = h

    def close(self):
        if self.handle:
            check(lib().bb_stack_destroy(self.handle))
            self.handle = None

    def forward(self, x, t, out):
        loc = _same_loc(x, out)
        check(lib().bb_stack_forward(self.ctx.handle, self.handle, _ptr(x)[0], t, _ptr(out)[0], loc))
        return out

    def run_layers(self, x):
        x = np.ascontiguousarray(x, np.float32).reshape(-1)
        out = np.empty_like(x)
        return self.forward(x, x.size // self.hidden, out)


class ConvOp:
    """The gated short-conv operator of one layer (model.rs:399-427 / :190-216)."""

    def __init__(self, ctx, weights):
        w = weights
        self.ctx = ctx
        self.hidden, self.l_cache = w.hidden, w.l_cache
        self.in_proj = Tensor(ctx, w.in_dtype, w.in_proj, (w.hidden, 3 * w.hidden))
        self.out_proj = Tensor(ctx, w.out_dtype, w.out_proj, (w.hidden, w.hidden))
        conv_w = np.ascontiguousarray(w.conv_w, np.float32)
        h = ctypes.c_void_p()
        check(lib().bb_conv_op_create(ctx.handle, self.in_proj.handle, conv_w.ctypes.data, w.l_cache,
                                      self.out_proj.handle, ctypes.byref(h)))
        self.handle = h

    def new_state(self):
        """A fresh conv cache: l_cache - 1 zero columns (cache.rs:29)."""
        return np.zeros((self.l_cache - 1) * self.hidden, np.float32)

    def close(self):
        if self.handle:
            check(lib().bb_conv_op_destroy(self.handle))
            self.handle = None
        for t in (self.in_proj, self.out_proj):
            t.close()

    def forward(self, state, x, t, out):
        loc = _same_loc(state, x, out)
        check(lib().bb_conv_op_forward(self.ctx.handle, self.handle, _ptr(state)[0], _ptr(x)[0], t, _ptr(out)[0], loc))
        return out


class KvCache:
    """One attention layer's key/value history in device memory (cache.rs:10-17)."""

    def __init__(self, ctx, kv_dim, capacity):
        self.ctx, self.kv_dim, self.capacity = ctx, kv_dim, capacity
        h = ctypes.c_void_p()
        check(lib().bb_kv_cache_create(ctx.handle, kv_dim, capacity, ctypes.byref(h)))
        self.handle = h

    def __len__(self):
        n = ctypes.c_size_t()
        check(lib().bb_kv_cache_length(self.handle, ctypes.byref(n)))
        return n.value

    def read(self):
        n = len(self)
        k = np.empty(n * self.kv_dim, np.float32)
        v = np.empty(n * self.kv_dim, np.float32)
        check(lib().bb_kv_cache_read(self.ctx.handle, self.handle, k.ctypes.data, v.ctypes.data, LOC_HOST))
        return k, v

    def evict_front(self, n):
        check(lib().bb_kv_cache_evict_front(self.ctx.handle, self.handle, n))

    def close(self):
        if self.handle:
            check(lib().bb_kv_cache_destroy(self.handle))
            self.handle = None


class AttnOp:
    """The GQA attention operator of one layer (model.rs:430-456 / :222-259)."""

    def __init__(self, ctx, weights):
        w = weights
        self.ctx = ctx
        self.hidden, self.n_heads, self.n_kv_heads, self.head_dim = w.hidden, w.n_heads, w.n_kv_heads, w.head_dim
        qd, kvd = w.n_heads * w.head_dim, w.n_kv_heads * w.head_dim
        self.kv_dim = kvd
        self.q = Tensor(ctx, w.q_dtype, w.q, (w.hidden, qd))
        self.k = Tensor(ctx, w.k_dtype, w.k, (w.hidden, kvd))
        self.v = Tensor(ctx, w.v_dtype, w.v, (w.hidden, kvd))
        self.o = Tensor(ctx, w.o_dtype, w.o, (qd, w.hidden))
        qn = np.ascontiguousarray(w.q_norm, np.float32)
        kn = np.ascontiguousarray(w.k_norm, np.float32)
        h = ctypes.c_void_p()
        check(lib().bb_attn_op_create(ctx.handle, self.q.handle, self.k.handle, self.v.handle, self.o.handle,
                                      qn.ctypes.data, kn.ctypes.data, w.n_heads, w.n_kv_heads, w.eps, w.freq_base,
                                      ctypes.byref(h)))
        self.handle = h

    def new_cache(self, capacity):
        return KvCache(self.ctx, self.kv_dim, capacity)

    def close(self):
        if self.handle:
            check(lib().bb_attn_op_destroy(self.handle))
            self.handle = None
        for t in (self.q, self.k, self.v, self.o):
            t.close()

    def forward(self, cache, pos0, x, t, out):
        loc = _same_loc(x, out)
        check(lib().bb_attn_op_forward(self.ctx.handle, self.handle, cache.handle, pos0, _ptr(x)[0], t, _ptr(out)[0],
                                       loc))
        return out


class Model:
    """The decoder's weights (Model, model.rs:25-31) built from a bebelm_amd.synth.ModelWeights:
    every operator, FFN and the logits head run on the GPU. The decode-time state is a Cache
    (cache.rs:10-19); one model serves any number of caches (agent.rs:85-86)."""

    def __init__(self, ctx, weights):
        mw = weights
        self.ctx, self.hidden, self.vocab = ctx, mw.hidden, mw.vocab
        self.token_embd = Tensor(ctx, mw.embd_dtype, mw.token_embd, (mw.hidden, mw.vocab))
        self.ops, self.ffns, self._keep = [], [], []
        # per layer: ("conv", conv state floats) or ("attn", kv_dim)
        self.layer_kinds = [("conv", (L.op.l_cache - 1) * mw.hidden) if hasattr(L.op, "conv_w")
                            else ("attn", L.op.n_kv_heads * L.op.head_dim) for L in mw.layers]
        descs = (_lib.DecoderLayer * len(mw.layers))()
        try:
            for i, L in enumerate(mw.layers):
                op = ConvOp(ctx, L.op) if hasattr(L.op, "conv_w") else AttnOp(ctx, L.op)
                self.ops.append(op)
                ffn = MoeLayer(ctx, L.ffn) if hasattr(L.ffn, "router") else DenseLayer(ctx, L.ffn)
                self.ffns.append(ffn)
                an = np.ascontiguousarray(L.attn_norm, np.float32)
                fn = np.ascontiguousarray(L.ffn_norm, np.float32)
                self._keep += [an, fn]
                descs[i].attn_norm, descs[i].ffn_norm = an.ctypes.data, fn.ctypes.data
                descs[i].conv = op.handle if isinstance(op, ConvOp) else None
                descs[i].attn = op.handle if isinstance(op, AttnOp) else None
                descs[i].moe = ffn.handle if isinstance(ffn, MoeLayer) else None
                descs[i].dense = ffn.handle if isinstance(ffn, DenseLayer) else None
            fin = np.ascontiguousarray(mw.final_norm, np.float32)
            h = ctypes.c_void_p()
            check(lib().bb_model_create(ctx.handle, self.token_embd.handle, fin.ctypes.data, descs, len(mw.layers),
                                        mw.eps, ctypes.byref(h)))
            self.handle = h
        except Exception:
            self.handle = None
            self.close()
            raise

    @classmethod
    def load(cls, ctx, gguf, validate=True):
        """Model::load (model.rs:36-50) from a GGUF (a path or an open gguf.GgufFile): with
        `validate`, config::validate first (the LFM2.5-8B-A1B constants); then the tensor-table
        check and the upload of every tensor into HBM (bb_model_load). The model owns its weights."""
        from .gguf import GgufFile
        own = not isinstance(gguf, GgufFile)
        g = GgufFile.open(gguf) if own else gguf
        try:
            if validate:
                g.validate()
            g.check_tensors()
            h = ctypes.c_void_p()
            check(lib().bb_model_load(ctx.handle, g.handle, ctypes.byref(h)))
            self = cls.__new__(cls)
            self.ctx, self.handle = ctx, h
            arch = g.architecture() + "."
            self.hidden, self.vocab = g.get_u32(arch + "embedding_length"), g.get_u32(arch + "vocab_size")
            head_dim = self.hidden // g.get_u32(arch + "attention.head_count")
            l_cache = g.get_u32(arch + "shortconv.l_cache")
            self.layer_kinds = [("attn", kv * head_dim) if kv else ("conv", (l_cache - 1) * self.hidden)
                                for kv in g.get_u32_array(arch + "attention.head_count_kv")]
            self.ops, self.ffns, self._keep, self.token_embd = [], [], [], None
            return self
        finally:
            if own:
                g.close()

    def close(self):
        if getattr(self, "handle", None):
            check(lib().bb_model_destroy(self.handle))
            self.handle = None
        for o in self.ops + self.ffns:
            o.close()
        self.ops, self.ffns = [], []
        if self.token_embd is not None:
            self.token_embd.close()

    def new_cache(self, kv_capacity=4096):
        """Cache::new for this model (kv_capacity: the initial room of each KV history)."""
        return Cache(self, kv_capacity)

    def run_layers(self, tokens, cache):
        """run_layers(token, &mut Cache) / run_layers_batch(tokens, &mut Cache): the final hidden
        states f32[T*hidden]."""
        tok = np.ascontiguousarray(tokens, np.uint32)
        out = np.empty(tok.size * self.hidden, np.float32)
        check(lib().bb_model_run_layers(self.ctx.handle, self.handle, tok.ctypes.data, tok.size, cache.handle,
                                        out.ctypes.data, LOC_HOST))
        return out

    def forward_step(self, token, cache):
        """Model::forward_step(&self, token, &mut Cache) (model.rs:97-103): next-token logits."""
        logits = np.empty(self.vocab, np.float32)
        check(lib().bb_model_forward_step(self.ctx.handle, self.handle, int(token), cache.handle, logits.ctypes.data,
                                          LOC_HOST))
        return logits

    def absorb(self, cache, tokens, max_context):
        """Agent::absorb(model, cache, tokens, max_context) (agent.rs:454-476)."""
        tok = np.ascontiguousarray(tokens, np.uint32)
        check(lib().bb_model_absorb(self.ctx.handle, self.handle, cache.handle, tok.ctypes.data, tok.size,
                                    max_context))


class Cache:
    """Cache (cache.rs:10-19) of one conversation on a Model: conv states, device KV histories and
    the next position. Cache::new (cache.rs:21-28) when created; clone() is Cache: Clone
    (Agent: Clone forks a prefilled prompt, agent.rs:87-91). Close it before its model."""

    def __init__(self, model, kv_capacity=4096, _handle=None):
        self.model, self.ctx = model, model.ctx
        if _handle is not None:
            self.handle = _handle
            return
        h = ctypes.c_void_p()
        check(lib().bb_cache_create(self.ctx.handle, model.handle, kv_capacity, ctypes.byref(h)))
        self.handle = h

    def clone(self):
        h = ctypes.c_void_p()
        check(lib().bb_cache_clone(self.ctx.handle, self.handle, ctypes.byref(h)))
        return Cache(self.model, _handle=h)

    def close(self):
        if getattr(self, "handle", None):
            check(lib().bb_cache_destroy(self.handle))
            self.handle = None

    @property
    def pos(self):
        n = ctypes.c_size_t()
        check(lib().bb_cache_position(self.handle, ctypes.byref(n)))
        return n.value

    def kv_len(self):
        n = ctypes.c_size_t()
        check(lib().bb_cache_kv_length(self.handle, ctypes.byref(n)))
        return n.value

    def reset(self):
        check(lib().bb_cache_reset(self.ctx.handle, self.handle))

    def evict_front(self, n):
        check(lib().bb_cache_evict_front(self.ctx.handle, self.handle, n))

    def layer_state(self, layer):
        """(conv state, k, v) of one layer; the absent ones are None."""
        kind, size = self.model.layer_kinds[layer]
        if kind == "conv":
            st = np.empty(size, np.float32)
            check(lib().bb_cache_layer_state(self.ctx.handle, self.handle, layer, st.ctypes.data, None, None,
                                             LOC_HOST))
            return st, None, None
        n = self.kv_len()
        k = np.empty(n * size, np.float32)
        v = np.empty(n * size, np.float32)
        check(lib().bb_cache_layer_state(self.ctx.handle, self.handle, layer, None, k.ctypes.data, v.ctypes.data,
                                         LOC_HOST))
        return None, k, v
