"""ctypes wrapper of the CPU restatement (liboracle.so) — TEST INFRASTRUCTURE ONLY.

Imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, never by the
product package. See bb_oracle.h for what each function restates and how it is pinned.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")  # x86-64-v3 (AVX2 + FMA): runs on any host here
# The same source built for AVX-512 with VNNI (the reference's x86 build is target-cpu=native,
# .cargo/config.toml, whose int8 dots take VNNI where the CPU has it). Loaded when the host has
# those features; both give the same bits (no FP contraction or reassociation in either).
LIB_AVX512_PATH = os.path.join(HERE, "liboracle_avx512.so")
AVX512_FLAGS = ("avx512f", "avx512bw", "avx512vl", "avx512dq", "avx512cd", "avx512_vnni")

F32, F16, Q4_K, Q6_K = 0, 1, 12, 14
c_void_p, c_size_t, c_int, c_float = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_float


class Q8(ctypes.Structure):
    _fields_ = [("q", c_void_p), ("scales", c_void_p), ("sums", c_void_p)]


class Job(ctypes.Structure):
    _fields_ = [("dtype", ctypes.c_uint32), ("w", c_void_p), ("n_in", c_size_t), ("n_out", c_size_t),
                ("x", c_void_p), ("has_qx", c_int), ("qx", Q8)]


class Moe(ctypes.Structure):
    _fields_ = [("router_dtype", ctypes.c_uint32), ("router", c_void_p), ("exp_probs_b", c_void_p),
                ("gate_dtype", ctypes.c_uint32), ("up_dtype", ctypes.c_uint32), ("down_dtype", ctypes.c_uint32),
                ("gate_exps", c_void_p), ("up_exps", c_void_p), ("down_exps", c_void_p),
                ("hidden", c_int), ("moe_ff", c_int), ("n_experts", c_int), ("n_used", c_int)]


class Trace(ctypes.Structure):
    _fields_ = [(n, c_void_p) for n in ("logits", "sel", "w", "counts", "offsets", "perm", "ties", "margin")]


class Dense(ctypes.Structure):
    _fields_ = [("gate_dtype", ctypes.c_uint32), ("up_dtype", ctypes.c_uint32), ("down_dtype", ctypes.c_uint32),
                ("gate", c_void_p), ("up", c_void_p), ("down", c_void_p), ("hidden", c_int), ("ff", c_int)]


class Layer(ctypes.Structure):
    _fields_ = [("ffn_norm", c_void_p), ("is_moe", c_int), ("dense", Dense), ("moe", Moe)]


_lib = None


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def host_has_avx512_vnni():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("flags"):
                    flags = set(line.split(":", 1)[1].split())
                    return all(x in flags for x in AVX512_FLAGS)
    except OSError:
        pass
    return False


def lib_path():
    """The build this host runs: BBO_ISA=v3 or avx512 forces one, else the widest it supports."""
    isa = os.environ.get("BBO_ISA", "")
    if isa == "v3":
        return LIB_PATH
    if isa == "avx512" or (isa == "" and host_has_avx512_vnni() and os.path.exists(LIB_AVX512_PATH)):
        return LIB_AVX512_PATH
    return LIB_PATH


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(lib_path())
        L.bbo_f16_to_f32.restype = c_float
        L.bbo_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.bbo_dot.restype = c_float
        L.bbo_dot.argtypes = [c_void_p, c_void_p, c_size_t]
        L.bbo_dot_q4k_block_q8.restype = c_float
        L.bbo_dot_q4k_block_q8.argtypes = [c_void_p, c_void_p, c_float, c_void_p]
        L.bbo_dot_q6k_block_q8.restype = c_float
        L.bbo_dot_q6k_block_q8.argtypes = [c_void_p, c_void_p, c_float]
        for n in ("bbo_q4k_block_sd", "bbo_q6k_block_idot", "bbo_q6k_block_idot_buffered"):
            getattr(L, n).restype = ctypes.c_int32
            getattr(L, n).argtypes = [c_void_p, c_void_p]
        L.bbo_fused_row_dot.restype = c_float
        L.bbo_fused_row_dot.argtypes = [ctypes.c_uint32, c_void_p, c_void_p, c_size_t]
        L.bbo_sigmoid.restype = c_float
        L.bbo_sigmoid.argtypes = [c_float]
        L.bbo_silu.restype = c_float
        L.bbo_silu.argtypes = [c_float]
        L.bbo_get_scale_min_k4.argtypes = [c_int, c_void_p, c_void_p, c_void_p]
        L.bbo_dequantize.argtypes = [ctypes.c_uint32, c_void_p, c_size_t, c_void_p]
        L.bbo_quantize_q8.argtypes = [c_void_p, c_size_t, Q8]
        L.bbo_matvec.argtypes = [ctypes.c_uint32, c_void_p, c_size_t, c_size_t, c_void_p, c_void_p]
        L.bbo_matmul.argtypes = [ctypes.c_uint32, c_void_p, c_size_t, c_size_t, c_void_p, c_size_t, c_void_p]
        L.bbo_matvec_fused_batch.argtypes = [ctypes.POINTER(Job), c_size_t, c_void_p]
        L.bbo_swiglu.argtypes = [c_void_p, c_void_p, c_void_p, c_size_t]
        L.bbo_add_scaled.argtypes = [c_void_p, c_void_p, c_float, c_size_t]
        L.bbo_add_assign.argtypes = [c_void_p, c_void_p, c_size_t]
        L.bbo_rmsnorm.argtypes = [c_void_p, c_void_p, c_float, c_size_t, c_void_p]
        L.bbo_moe_ffn.argtypes = [ctypes.POINTER(Moe), c_void_p, c_void_p, ctypes.POINTER(Trace)]
        L.bbo_moe_ffn_batch.argtypes = [ctypes.POINTER(Moe), c_void_p, c_size_t, c_void_p, ctypes.POINTER(Trace)]
        L.bbo_dense_ffn.argtypes = [ctypes.POINTER(Dense), c_void_p, c_size_t, c_void_p]
        L.bbo_ffn_stack.argtypes = [ctypes.POINTER(Layer), c_size_t, c_void_p, c_size_t, c_float, c_void_p]
        L.bbo_dot_variant.restype = c_float
        L.bbo_dot_variant.argtypes = [c_void_p, c_void_p, c_size_t, c_int]
        L.bbo_router_logits_variant.argtypes = [c_void_p, c_void_p, c_size_t, c_int, c_int, c_int, c_void_p]
        L.bbo_gate.argtypes = [c_void_p, c_void_p, c_size_t, c_int, c_int, c_void_p, c_void_p, c_void_p, c_void_p]
        L.bbo_conv_step.argtypes = [c_void_p, c_void_p, c_void_p, c_size_t, c_size_t, c_void_p]
        L.bbo_conv_prefill.argtypes = [c_void_p, c_void_p, c_void_p, c_size_t, c_size_t, c_size_t, c_void_p]
        L.bbo_softmax.argtypes = [c_void_p, c_size_t]
        L.bbo_attention_decode.argtypes = [c_void_p, c_void_p, c_void_p, c_size_t, c_size_t, c_size_t, c_size_t,
                                           c_void_p]
        L.bbo_rope_neox.argtypes = [c_void_p, c_size_t, c_size_t, c_float]
        L.bbo_norm_rope_heads.argtypes = [c_void_p, c_size_t, c_size_t, c_void_p, c_float, c_size_t, c_float]
        L.bbo_conv_forward.argtypes = [ctypes.POINTER(ConvOp), c_void_p, c_void_p, c_size_t, c_void_p]
        L.bbo_attn_forward.argtypes = [ctypes.POINTER(AttnOp), c_void_p, c_void_p, c_size_t,
                                       ctypes.POINTER(c_size_t), c_size_t, c_void_p, c_size_t, c_void_p]
        L.bbo_set_threads.argtypes = [c_int]
        L.bbo_get_threads.restype = c_int
        _lib = L
    return _lib


def _p(a):
    return a.ctypes.data if a is not None else None


def _chk(rc):
    if rc != 0:
        raise ValueError(f"oracle call failed ({rc})")


def set_threads(n):
    lib().bbo_set_threads(int(n))


def get_threads():
    return lib().bbo_get_threads()


def f16_to_f32(h):
    return lib().bbo_f16_to_f32(int(h))


def get_scale_min_k4(j, scales):
    s = np.ascontiguousarray(scales, np.uint8)
    sc, m = np.zeros(1, np.uint8), np.zeros(1, np.uint8)
    lib().bbo_get_scale_min_k4(j, _p(s), _p(sc), _p(m))
    return int(sc[0]), int(m[0])


def dequantize(dtype, data, n):
    data = np.ascontiguousarray(data, np.uint8)
    out = np.zeros(n, np.float32)
    _chk(lib().bbo_dequantize(dtype, _p(data), n, _p(out)))
    return out


class Q8Vec:
    def __init__(self, n):
        self.q = np.zeros(n, np.int8)
        self.scales = np.zeros(n // 256, np.float32)
        self.sums = np.zeros(n // 32, np.int32)

    def struct(self):
        return Q8(_p(self.q), _p(self.scales), _p(self.sums))


def quantize_q8(x):
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    v = Q8Vec(x.size)
    lib().bbo_quantize_q8(_p(x), x.size, v.struct())
    return v


def dot(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return lib().bbo_dot(_p(a), _p(b), a.size)


# Router dot evaluation orders (bb_oracle.cpp dot_variant): 0 is the order the restatement
# assumes for the reference; 1-5 are the other plausible ones.
DOT_VARIANTS = {0: "FMA chains, AVX reduce tree", 1: "mul+add chains, AVX reduce tree",
                2: "FMA chains, pairwise lane fold", 3: "mul+add chains, lanes left to right",
                4: "scalar left-to-right f32", 5: "f64 exact products, one rounding",
                6: "mul+add chains, pairwise lane fold"}


def dot_variant(a, b, variant):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return lib().bbo_dot_variant(_p(a), _p(b), a.size, int(variant))


def router_logits_variant(w, x, t, variant):
    """[t, E] router logits of token-major x under dot variant `variant`."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    router = np.ascontiguousarray(w.router, np.float32)
    out = np.zeros(t * w.n_experts, np.float32)
    lib().bbo_router_logits_variant(_p(router), _p(x), t, w.hidden, w.n_experts, int(variant), _p(out))
    return out.reshape(t, w.n_experts)


def gate(logits, bias, k):
    """model.rs:485-495 for each row of logits [t, E]: (sel [t,k], w [t,k], ties, margin [t])."""
    logits = np.ascontiguousarray(logits, np.float32)
    t, E = logits.shape
    bias = np.ascontiguousarray(bias, np.float32)
    sel = np.zeros((t, k), np.int32)
    w = np.zeros((t, k), np.float32)
    ties = np.zeros(1, np.int32)
    margin = np.zeros(t, np.float32)
    lib().bbo_gate(_p(logits), _p(bias), t, E, k, _p(sel), _p(w), _p(ties), _p(margin))
    return sel, w, int(ties[0]), margin


def dot_q4k_block_q8(block, qx, sx, sums):
    block, qx, sums = (np.ascontiguousarray(block, np.uint8), np.ascontiguousarray(qx, np.int8),
                       np.ascontiguousarray(sums, np.int32))
    return lib().bbo_dot_q4k_block_q8(_p(block), _p(qx), sx, _p(sums))


def dot_q6k_block_q8(block, qx, sx):
    block, qx = np.ascontiguousarray(block, np.uint8), np.ascontiguousarray(qx, np.int8)
    return lib().bbo_dot_q6k_block_q8(_p(block), _p(qx), sx)


def q4k_block_sd(block, qx):
    block, qx = np.ascontiguousarray(block, np.uint8), np.ascontiguousarray(qx, np.int8)
    return lib().bbo_q4k_block_sd(_p(block), _p(qx))


def q6k_block_idot(block, qx, buffered=False):
    block, qx = np.ascontiguousarray(block, np.uint8), np.ascontiguousarray(qx, np.int8)
    f = lib().bbo_q6k_block_idot_buffered if buffered else lib().bbo_q6k_block_idot
    return f(_p(block), _p(qx))


def fused_row_dot(dtype, row, x):
    row, x = np.ascontiguousarray(row, np.uint8), np.ascontiguousarray(x, np.float32)
    return lib().bbo_fused_row_dot(dtype, _p(row), _p(x), x.size)


def matvec(dtype, w, n_in, n_out, x):
    w, x = np.ascontiguousarray(w).view(np.uint8).reshape(-1), np.ascontiguousarray(x, np.float32)
    y = np.zeros(n_out, np.float32)
    _chk(lib().bbo_matvec(dtype, _p(w), n_in, n_out, _p(x), _p(y)))
    return y


def matmul(dtype, w, n_in, n_out, x, n_tokens):
    w, x = np.ascontiguousarray(w).view(np.uint8).reshape(-1), np.ascontiguousarray(x, np.float32)
    y = np.zeros(n_out * n_tokens, np.float32)
    _chk(lib().bbo_matmul(dtype, _p(w), n_in, n_out, _p(x), n_tokens, _p(y)))
    return y


def matvec_fused_batch(jobs):
    """jobs: list of (dtype, w bytes, n_in, n_out, x f32, qx Q8Vec | None)."""
    arr = (Job * len(jobs))()
    keep = []
    total = 0
    for i, (dt, w, n_in, n_out, x, qx) in enumerate(jobs):
        w = np.ascontiguousarray(w, np.uint8)
        x = np.ascontiguousarray(x, np.float32)
        keep += [w, x]
        arr[i] = Job(dt, _p(w), n_in, n_out, _p(x), 1 if qx is not None else 0,
                     qx.struct() if qx is not None else Q8(None, None, None))
        total += n_out
    out = np.zeros(total, np.float32)
    _chk(lib().bbo_matvec_fused_batch(arr, len(jobs), _p(out)))
    return out


def sigmoid(x):
    return lib().bbo_sigmoid(float(x))


def silu(x):
    return lib().bbo_silu(float(x))


def swiglu(gate, up):
    gate, up = np.ascontiguousarray(gate, np.float32), np.ascontiguousarray(up, np.float32)
    out = np.zeros_like(gate)
    lib().bbo_swiglu(_p(gate), _p(up), _p(out), gate.size)
    return out


def add_scaled(out, b, s):
    out = np.array(out, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    lib().bbo_add_scaled(_p(out), _p(b), s, out.size)
    return out


def add_assign(a, b):
    a = np.array(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    lib().bbo_add_assign(_p(a), _p(b), a.size)
    return a


def rmsnorm(x, gain, eps):
    x, gain = np.ascontiguousarray(x, np.float32), np.ascontiguousarray(gain, np.float32)
    out = np.zeros_like(x)
    lib().bbo_rmsnorm(_p(x), _p(gain), eps, x.size, _p(out))
    return out


def _moe_struct(w):
    return Moe(0, _p(w.router), _p(w.exp_probs_b), w.gate_dtype, w.up_dtype, w.down_dtype, _p(w.gate_exps),
               _p(w.up_exps), _p(w.down_exps), w.hidden, w.moe_ff, w.n_experts, w.n_used)


class TraceArrays:
    def __init__(self, t, E, k):
        self.logits = np.zeros(t * E, np.float32)
        self.sel = np.zeros(t * k, np.int32)
        self.w = np.zeros(t * k, np.float32)
        self.counts = np.zeros(E, np.int32)
        self.offsets = np.zeros(E + 1, np.int32)
        self.perm = np.zeros(t * k, np.int32)
        self.ties = np.zeros(1, np.int32)
        self.margin = np.zeros(t, np.float32)

    def struct(self):
        return Trace(*(_p(a) for a in (self.logits, self.sel, self.w, self.counts, self.offsets, self.perm,
                                       self.ties, self.margin)))


def moe_ffn(w, x, trace=False):
    """Model::moe_ffn (one token). Returns out or (out, TraceArrays)."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    out = np.zeros(w.hidden, np.float32)
    m = _moe_struct(w)
    tr = TraceArrays(1, w.n_experts, w.n_used) if trace else None
    ts = tr.struct() if tr else None
    _chk(lib().bbo_moe_ffn(ctypes.byref(m), _p(x), _p(out), ctypes.byref(ts) if ts else None))
    return (out, tr) if trace else out


def moe_ffn_batch(w, x, t, trace=False):
    """Model::moe_ffn_batch (t tokens, token-major)."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    out = np.zeros(t * w.hidden, np.float32)
    m = _moe_struct(w)
    tr = TraceArrays(t, w.n_experts, w.n_used) if trace else None
    ts = tr.struct() if tr else None
    _chk(lib().bbo_moe_ffn_batch(ctypes.byref(m), _p(x), t, _p(out), ctypes.byref(ts) if ts else None))
    return (out, tr) if trace else out


def _dense_struct(d):
    return Dense(d.gate_dtype, d.up_dtype, d.down_dtype, _p(d.gate), _p(d.up), _p(d.down), d.hidden, d.ff)


def dense_ffn(d, x, t=1):
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    out = np.zeros(t * d.hidden, np.float32)
    s = _dense_struct(d)
    _chk(lib().bbo_dense_ffn(ctypes.byref(s), _p(x), t, _p(out)))
    return out


def ffn_stack(layers, x, t=1, eps=1e-5):
    """layers: list of (gain, MoeWeights | DenseWeights) as bebelm_amd.synth.stack_layers makes."""
    arr = (Layer * len(layers))()
    keep = []
    for i, (gain, w) in enumerate(layers):
        gain = np.ascontiguousarray(gain, np.float32)
        keep.append(gain)
        if hasattr(w, "router"):
            arr[i] = Layer(_p(gain), 1, Dense(), _moe_struct(w))
        else:
            arr[i] = Layer(_p(gain), 0, _dense_struct(w), Moe())
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    h = np.zeros_like(x)
    _chk(lib().bbo_ffn_stack(arr, len(layers), _p(x), t, eps, _p(h)))
    return h


# ---- operators of the decoder layer ------------------------------------------------------------

class ConvOp(ctypes.Structure):
    _fields_ = [("hidden", c_int), ("l_cache", c_int), ("in_dtype", ctypes.c_uint32), ("out_dtype", ctypes.c_uint32),
                ("in_proj", c_void_p), ("out_proj", c_void_p), ("conv_w", c_void_p)]


class AttnOp(ctypes.Structure):
    _fields_ = [("hidden", c_int), ("n_heads", c_int), ("n_kv_heads", c_int), ("head_dim", c_int),
                ("q_dtype", ctypes.c_uint32), ("k_dtype", ctypes.c_uint32), ("v_dtype", ctypes.c_uint32),
                ("o_dtype", ctypes.c_uint32), ("q", c_void_p), ("k", c_void_p), ("v", c_void_p), ("o", c_void_p),
                ("q_norm", c_void_p), ("k_norm", c_void_p), ("eps", c_float), ("freq_base", c_float)]


def _f32(a):
    return np.ascontiguousarray(a, np.float32).reshape(-1)


def conv_step(state, bx, weight, channels, l_cache):
    """conv.rs:18-39: out f32[channels]."""
    state, bx, weight = _f32(state), _f32(bx), _f32(weight)
    out = np.zeros(channels, np.float32)
    lib().bbo_conv_step(_p(state), _p(bx), _p(weight), channels, l_cache, _p(out))
    return out


def conv_prefill(state, bx, weight, channels, l_cache, n_tokens):
    """conv.rs:48-68: (out f32[n_tokens·channels], the updated state)."""
    state, bx, weight = _f32(state).copy(), _f32(bx), _f32(weight)
    out = np.zeros(n_tokens * channels, np.float32)
    lib().bbo_conv_prefill(_p(state), _p(bx), _p(weight), channels, l_cache, n_tokens, _p(out))
    return out, state


def softmax(x):
    """softmax.rs:9-22 over one row."""
    x = _f32(x).copy()
    lib().bbo_softmax(_p(x), x.size)
    return x


def attention_decode(q, k, v, n_ctx, n_heads, n_kv_heads, head_dim):
    """attention.rs:17-55: out f32[n_heads·head_dim]."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    out = np.zeros(n_heads * head_dim, np.float32)
    lib().bbo_attention_decode(_p(q), _p(k), _p(v), n_ctx, n_heads, n_kv_heads, head_dim, _p(out))
    return out


def rope_neox(x, pos, freq_base):
    """rope.rs:17-30 on one head vector."""
    x = _f32(x).copy()
    lib().bbo_rope_neox(_p(x), x.size, pos, freq_base)
    return x


def norm_rope_heads(buf, n_heads, head_dim, gain, eps, pos, freq_base):
    """model.rs:692-701."""
    buf, gain = _f32(buf).copy(), _f32(gain)
    lib().bbo_norm_rope_heads(_p(buf), n_heads, head_dim, _p(gain), eps, pos, freq_base)
    return buf


def _conv_struct(w):
    return ConvOp(w.hidden, w.l_cache, w.in_dtype, w.out_dtype, _p(w.in_proj), _p(w.out_proj), _p(w.conv_w))


def conv_forward(w, state, x, t):
    """Model::conv_step_op (t == 1, model.rs:399-427) or conv_batch (model.rs:190-216):
    (out f32[t·hidden], the updated state)."""
    state, x = _f32(state).copy(), _f32(x)
    out = np.zeros(t * w.hidden, np.float32)
    s = _conv_struct(w)
    _chk(lib().bbo_conv_forward(ctypes.byref(s), _p(state), _p(x), t, _p(out)))
    return out, state


class KvCache:
    """One attention layer's key/value history (model.rs:447-448): cap positions of kv_dim floats."""

    def __init__(self, kv_dim, cap):
        self.kv_dim, self.cap = kv_dim, cap
        self.k = np.zeros(cap * kv_dim, np.float32)
        self.v = np.zeros(cap * kv_dim, np.float32)
        self.n = 0

    def copy(self):
        c = KvCache(self.kv_dim, self.cap)
        c.k[:], c.v[:], c.n = self.k, self.v, self.n
        return c


def _attn_struct(w):
    return AttnOp(w.hidden, w.n_heads, w.n_kv_heads, w.head_dim, w.q_dtype, w.k_dtype, w.v_dtype, w.o_dtype,
                  _p(w.q), _p(w.k), _p(w.v), _p(w.o), _p(w.q_norm), _p(w.k_norm), w.eps, w.freq_base)


def attn_forward(w, cache, pos0, x, t):
    """Model::attn_step (t == 1, model.rs:430-456) or attn_batch (model.rs:222-259); appends t
    positions to `cache` and returns out f32[t·hidden]."""
    x = _f32(x)
    out = np.zeros(t * w.hidden, np.float32)
    s = _attn_struct(w)
    n = c_size_t(cache.n)
    rc = lib().bbo_attn_forward(ctypes.byref(s), _p(cache.k), _p(cache.v), cache.cap, ctypes.byref(n), pos0, _p(x),
                                t, _p(out))
    _chk(rc)
    cache.n = n.value
    return out


# ---- the decoder (model.rs:99-181, agent.rs:454-476), composed from the restated pieces ----------

class Model:
    """Model + Cache over a bebelm_amd.synth.ModelWeights: the reference's forward pass with its
    caches, each piece a call of the C restatement above (the loop order of model.rs:105-181)."""

    def __init__(self, mw, kv_capacity):
        self.mw, self.cap = mw, kv_capacity
        self.reset()

    def reset(self):
        self.pos = 0
        self.state = {}
        for i, L in enumerate(self.mw.layers):
            if hasattr(L.op, "conv_w"):
                self.state[i] = np.zeros((L.op.l_cache - 1) * self.mw.hidden, np.float32)
            else:
                self.state[i] = KvCache(L.op.kv_dim, self.cap)

    def kv_len(self):
        return max([c.n for c in self.state.values() if isinstance(c, KvCache)] or [0])

    def fork(self):
        """Cache: Clone (cache.rs:9): a model over the same weights with a copy of this one's
        caches and position, which then evolve independently."""
        other = Model.__new__(Model)
        other.mw, other.cap, other.pos = self.mw, self.cap, self.pos
        other.state = {i: (c.copy() if isinstance(c, KvCache) else c.copy()) for i, c in self.state.items()}
        return other

    def embed(self, tokens):
        H = self.mw.hidden
        be, bb = {12: (256, 144), 14: (256, 210), 0: (1, 4)}[self.mw.embd_dtype]
        rb = H // be * bb
        return np.concatenate([dequantize(self.mw.embd_dtype, self.mw.token_embd[t * rb:(t + 1) * rb], H)
                               for t in tokens]).astype(np.float32)

    def run_layers(self, tokens):
        """run_layers (one token, model.rs:105-130) or run_layers_batch (model.rs:146-181)."""
        t, H = len(tokens), self.mw.hidden
        h = self.embed(tokens)
        for i, L in enumerate(self.mw.layers):
            normed = np.concatenate([rmsnorm(h[r * H:(r + 1) * H], L.attn_norm, self.mw.eps) for r in range(t)])
            if hasattr(L.op, "conv_w"):
                op, self.state[i] = conv_forward(L.op, self.state[i], normed, t)
            else:
                op = attn_forward(L.op, self.state[i], self.pos, normed, t)
            h = (h + op).astype(np.float32)
            normed = np.concatenate([rmsnorm(h[r * H:(r + 1) * H], L.ffn_norm, self.mw.eps) for r in range(t)])
            if hasattr(L.ffn, "router"):
                ffn = moe_ffn(L.ffn, normed) if t == 1 else moe_ffn_batch(L.ffn, normed, t)
            else:
                ffn = dense_ffn(L.ffn, normed, t)
            h = (h + ffn).astype(np.float32)
        self.pos += t
        return h

    def forward_step(self, token):
        """model.rs:99-103: run_layers, then logits_from_hidden (model.rs:380-388)."""
        h = self.run_layers([token])
        normed = rmsnorm(h, self.mw.final_norm, self.mw.eps)
        return matvec(self.mw.embd_dtype, self.mw.token_embd, self.mw.hidden, self.mw.vocab, normed)

    def evict_front(self, n):
        for c in self.state.values():
            if isinstance(c, KvCache) and c.n >= n:
                keep = (c.n - n) * c.kv_dim
                c.k[:keep] = c.k[n * c.kv_dim:c.n * c.kv_dim].copy()
                c.v[:keep] = c.v[n * c.kv_dim:c.n * c.kv_dim].copy()
                c.n -= n

    def absorb(self, tokens, max_context, chunk=512):
        """agent.rs:454-476."""
        if self.kv_len() + len(tokens) <= max_context:
            for a in range(0, len(tokens), chunk):
                self.run_layers(tokens[a:a + chunk])
        else:
            for tok in tokens:
                self.run_layers([tok])
                n = self.kv_len()
                if n > max_context:
                    self.evict_front(n - max_context)
