"""Deterministic synthetic inputs for the MoE FFN benchmark configurations.

Shapes follow the reference's hard-coded LFM2.5-8B-A1B architecture (src/config.rs:14-32):
hidden 2048, expert FFN 1792, 32 experts, top-4, dense FFN 7168 (layers 0-1). There is no GGUF
offline, so weights are random blocks in the native GGUF byte layouts:

  Q4_K (144 B): d, dmin = f16(|N(0, 2e-3)|); 6-bit scales and mins ~ U{0..63} packed as
                get_scale_min_k4 (dequant.rs:64-72) unpacks them; qs bytes ~ U{0..255}.
  Q6_K (210 B): ql, qh bytes ~ U{0..255}; i8 scales ~ U{-64..63}; d = f16(|N(0, 2e-3)|).
  Router (ffn_gate_inp): f32 ~ N(0, 0.02). Hidden states: f32 ~ N(0, 1).

Every tensor draws from its own PCG64 stream keyed by (config seed, tensor id), so any tensor
can be regenerated alone. Gating follows the reference (sigmoid + selection-only bias,
model.rs:485-495); the skewed config puts a Zipf(1.2) ranking into that bias (exp_probs_b).
"""
import os
from concurrent.futures import ThreadPoolExecutor
from dataclasses import dataclass, field

import numpy as np

F32, F16, Q4_K, Q6_K = 0, 1, 12, 14
BLOCK = {F32: (1, 4), F16: (1, 2), Q4_K: (256, 144), Q6_K: (256, 210)}

HIDDEN = 2048
MOE_FF = 1792
DENSE_FF = 7168
N_EXPERTS = 32
N_USED = 4
N_LAYERS = 24
N_DENSE = 2
RMS_EPS = 1e-5


def rng(seed, *stream):
    return np.random.Generator(np.random.PCG64([int(seed), *[int(s) for s in stream]]))


def byte_size(dtype, n_elements):
    be, bb = BLOCK[dtype]
    assert n_elements % be == 0
    return n_elements // be * bb


def _f16_abs_normal(g, n, sigma):
    return np.abs(g.standard_normal(n) * sigma).astype(np.float16).view(np.uint16)


def pack_q4k_scales(sc, m):
    """Inverse of get_scale_min_k4 (dequant.rs:64-72): (..., 8) 6-bit values -> (..., 12) bytes."""
    sc = sc.astype(np.uint8)
    m = m.astype(np.uint8)
    s = np.zeros(sc.shape[:-1] + (12,), np.uint8)
    for j in range(4):
        s[..., j] = sc[..., j] | ((sc[..., j + 4] >> 4) << 6)
        s[..., j + 4] = m[..., j] | ((m[..., j + 4] >> 4) << 6)
        s[..., j + 8] = (sc[..., j + 4] & 0xF) | ((m[..., j + 4] & 0xF) << 4)
    return s


def q4k_blocks(g, n_blocks):
    out = np.empty((n_blocks, 144), np.uint8)
    d = _f16_abs_normal(g, n_blocks, 2e-3)
    dmin = _f16_abs_normal(g, n_blocks, 2e-3)
    out[:, 0:2] = d.view(np.uint8).reshape(n_blocks, 2)
    out[:, 2:4] = dmin.view(np.uint8).reshape(n_blocks, 2)
    sc = g.integers(0, 64, (n_blocks, 8), dtype=np.uint8)
    m = g.integers(0, 64, (n_blocks, 8), dtype=np.uint8)
    out[:, 4:16] = pack_q4k_scales(sc, m)
    out[:, 16:144] = g.integers(0, 256, (n_blocks, 128), dtype=np.uint8)
    return out.reshape(-1)


def q6k_blocks(g, n_blocks):
    out = np.empty((n_blocks, 210), np.uint8)
    out[:, 0:192] = g.integers(0, 256, (n_blocks, 192), dtype=np.uint8)
    out[:, 192:208] = g.integers(-64, 64, (n_blocks, 16), dtype=np.int8).view(np.uint8)
    d = _f16_abs_normal(g, n_blocks, 2e-3)
    out[:, 208:210] = d.view(np.uint8).reshape(n_blocks, 2)
    return out.reshape(-1)


def quant_tensor(g, dtype, n_in, n_out, n_mat=1):
    n_blocks = n_mat * n_out * n_in // 256
    if dtype == Q4_K:
        return q4k_blocks(g, n_blocks)
    if dtype == Q6_K:
        return q6k_blocks(g, n_blocks)
    raise ValueError(f"dtype {dtype}")


def zipf_bias(seed, n_experts=N_EXPERTS, s=1.2, kappa=1.5):
    """exp_probs_b[e] = kappa * p_rank(e), p_r ∝ r^-s over a seeded rank permutation.

    kappa = 1.5 gives config 4 (4096 tokens, seed 0) a top-3 expert share of 35.4% of the
    assignments (0.5: 17.5%, 1.0: 26.6%); the share is checked by the GPU test of config 4."""
    r = np.arange(1, n_experts + 1, dtype=np.float64)
    p = r ** -s
    p /= p.sum()
    perm = rng(seed, 9001).permutation(n_experts)
    bias = np.zeros(n_experts, np.float32)
    bias[perm] = (kappa * p).astype(np.float32)
    return bias


@dataclass
class MoeWeights:
    hidden: int
    moe_ff: int
    n_experts: int
    n_used: int
    router: np.ndarray          # f32 [E, hidden] row-major (GGUF dims [hidden, E])
    exp_probs_b: np.ndarray     # f32 [E]
    gate_dtype: int
    up_dtype: int
    down_dtype: int
    gate_exps: np.ndarray       # u8, E experts x ff rows of hidden
    up_exps: np.ndarray
    down_exps: np.ndarray       # u8, E experts x hidden rows of ff

    def expert_bytes(self, dtype, n_in, n_out):
        return byte_size(dtype, n_in * n_out)

    @property
    def nbytes(self):
        return self.router.nbytes + self.gate_exps.nbytes + self.up_exps.nbytes + self.down_exps.nbytes


@dataclass
class DenseWeights:
    hidden: int
    ff: int
    gate_dtype: int
    up_dtype: int
    down_dtype: int
    gate: np.ndarray
    up: np.ndarray
    down: np.ndarray

    @property
    def nbytes(self):
        return self.gate.nbytes + self.up.nbytes + self.down.nbytes


def moe_weights(seed, layer=0, hidden=HIDDEN, moe_ff=MOE_FF, n_experts=N_EXPERTS, n_used=N_USED,
                down_dtype=Q4_K, gate_dtype=Q4_K, bias=None):
    base = 100 * layer
    router = (rng(seed, base + 1).standard_normal((n_experts, hidden), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    gate = quant_tensor(rng(seed, base + 2), gate_dtype, hidden, moe_ff, n_experts)
    up = quant_tensor(rng(seed, base + 3), gate_dtype, hidden, moe_ff, n_experts)
    down = quant_tensor(rng(seed, base + 4), down_dtype, moe_ff, hidden, n_experts)
    b = np.zeros(n_experts, np.float32) if bias is None else np.asarray(bias, np.float32)
    return MoeWeights(hidden, moe_ff, n_experts, n_used, router, b, gate_dtype, gate_dtype, down_dtype, gate, up, down)


def dense_weights(seed, layer=0, hidden=HIDDEN, ff=DENSE_FF, dtype=Q4_K):
    base = 100 * layer
    gate = quant_tensor(rng(seed, base + 5), dtype, hidden, ff)
    up = quant_tensor(rng(seed, base + 6), dtype, hidden, ff)
    down = quant_tensor(rng(seed, base + 7), dtype, ff, hidden)
    return DenseWeights(hidden, ff, dtype, dtype, dtype, gate, up, down)


# The decoder layer's operators (src/config.rs:20-31): GQA attention with 32 query heads, 8 kv
# heads of 64 dims, NEOX RoPE base 5e6; the gated short conv with a 3-tap filter.
N_HEADS = 32
N_KV_HEADS = 8
HEAD_DIM = HIDDEN // N_HEADS
CONV_L_CACHE = 3
ROPE_THETA = 5_000_000.0


@dataclass
class ConvWeights:
    hidden: int
    l_cache: int
    in_dtype: int
    out_dtype: int
    in_proj: np.ndarray         # u8, [hidden, 3·hidden]: 3·hidden rows of hidden
    out_proj: np.ndarray        # u8, [hidden, hidden]
    conv_w: np.ndarray          # f32 [hidden·l_cache], tap-contiguous per channel


@dataclass
class AttnWeights:
    hidden: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    q_dtype: int
    k_dtype: int
    v_dtype: int
    o_dtype: int
    q: np.ndarray               # u8, [hidden, n_heads·head_dim]
    k: np.ndarray               # u8, [hidden, n_kv_heads·head_dim]
    v: np.ndarray
    o: np.ndarray               # u8, [n_heads·head_dim, hidden]
    q_norm: np.ndarray          # f32 [head_dim]
    k_norm: np.ndarray
    eps: float = RMS_EPS
    freq_base: float = ROPE_THETA

    @property
    def kv_dim(self):
        return self.n_kv_heads * self.head_dim


def conv_weights(seed, layer=0, hidden=HIDDEN, l_cache=CONV_L_CACHE, in_dtype=Q4_K, out_dtype=Q4_K):
    """Short-conv operator: Q4_K/Q6_K projections as the expert tensors; filter taps ~ N(0, 0.5)."""
    base = 100 * layer
    in_proj = quant_tensor(rng(seed, base + 11), in_dtype, hidden, 3 * hidden)
    out_proj = quant_tensor(rng(seed, base + 12), out_dtype, hidden, hidden)
    conv_w = (rng(seed, base + 13).standard_normal(hidden * l_cache, dtype=np.float32) * np.float32(0.5)).astype(np.float32)
    return ConvWeights(hidden, l_cache, in_dtype, out_dtype, in_proj, out_proj, conv_w)


def attn_weights(seed, layer=0, hidden=HIDDEN, n_heads=N_HEADS, n_kv_heads=N_KV_HEADS, head_dim=None,
                 dtypes=(Q4_K, Q4_K, Q6_K, Q4_K), freq_base=ROPE_THETA):
    """GQA attention operator: q/k/v/o in the given dtypes; q/k norm gains ~ 1 + N(0, 0.1)."""
    hd = hidden // n_heads if head_dim is None else head_dim
    base = 100 * layer
    qd, kd, vd, od = dtypes
    q = quant_tensor(rng(seed, base + 21), qd, hidden, n_heads * hd)
    k = quant_tensor(rng(seed, base + 22), kd, hidden, n_kv_heads * hd)
    v = quant_tensor(rng(seed, base + 23), vd, hidden, n_kv_heads * hd)
    o = quant_tensor(rng(seed, base + 24), od, n_heads * hd, hidden)
    g = rng(seed, base + 25)
    q_norm = (1.0 + 0.1 * g.standard_normal(hd)).astype(np.float32)
    k_norm = (1.0 + 0.1 * g.standard_normal(hd)).astype(np.float32)
    return AttnWeights(hidden, n_heads, n_kv_heads, hd, qd, kd, vd, od, q, k, v, o, q_norm, k_norm, RMS_EPS, freq_base)


def hidden_states(seed, t, hidden=HIDDEN, stream=0):
    return rng(seed, 7000 + stream).standard_normal((t, hidden), dtype=np.float32)


@dataclass
class Config:
    name: str
    tokens: int
    down_dtype: int = Q4_K
    zipf: bool = False
    layers: int = 1
    description: str = ""
    extra: dict = field(default_factory=dict)


CONFIGS = {
    1: Config("decode_t1", 1, description="decode of 1 token, Q4_K experts, unbiased router"),
    2: Config("decode_t16", 16, description="decode batch of 16 independent tokens, Q4_K experts"),
    3: Config("prefill_t512", 512, description="prefill of 512 tokens, Q4_K experts, unbiased router"),
    4: Config("prefill_t4096_zipf_q6k", 4096, down_dtype=Q6_K, zipf=True,
              description="prefill of 4096 tokens, Zipf(1.2) selection bias, Q6_K down"),
    5: Config("ffn_stack_24l_t1", 1, layers=N_LAYERS,
              description="24-layer FFN path: 2 dense + 22 MoE (down Q4_K on even, Q6_K on odd layers)"),
}


def config_layer(cfg_id, seed=0, layer=0, **kw):
    cfg = CONFIGS[cfg_id]
    bias = zipf_bias(seed) if cfg.zipf else None
    return moe_weights(seed, layer=layer, down_dtype=cfg.down_dtype, bias=bias, **kw)


def _par_map(fn, items):
    """[fn(i) for i in items] on a thread pool: every layer draws from its own seeded streams, so
    the arrays are the same in any order (numpy's generators release the GIL while filling)."""
    items = list(items)
    workers = max(1, min(len(items), os.cpu_count() or 1, 16))
    if workers == 1:
        return [fn(i) for i in items]
    with ThreadPoolExecutor(workers) as ex:
        return list(ex.map(fn, items))


def stack_layers(seed=0, hidden=HIDDEN, moe_ff=MOE_FF, dense_ff=DENSE_FF, n_experts=N_EXPERTS,
                 n_layers=N_LAYERS, n_dense=N_DENSE):
    """Config 5: layers < n_dense dense; MoE down in Q4_K on even layers, Q6_K on odd ones."""
    def one(layer):
        gain = np.ones(hidden, np.float32)
        if layer < n_dense:
            return gain, dense_weights(seed, layer, hidden, dense_ff)
        dd = Q4_K if layer % 2 == 0 else Q6_K
        return gain, moe_weights(seed, layer, hidden, moe_ff, n_experts, down_dtype=dd)

    return _par_map(one, range(n_layers))


# ---- the whole decoder (model.rs:25-31, 105-130) -------------------------------------------------
ATTENTION_LAYERS = (2, 6, 10, 14, 18, 21)   # src/config.rs:37
VOCAB = 128_000


@dataclass
class DecoderLayerWeights:
    attn_norm: np.ndarray       # f32 [hidden]
    ffn_norm: np.ndarray
    op: object                  # ConvWeights | AttnWeights
    ffn: object                 # MoeWeights | DenseWeights


@dataclass
class ModelWeights:
    hidden: int
    vocab: int
    embd_dtype: int
    token_embd: np.ndarray      # u8, [hidden, vocab]: vocab rows of hidden
    final_norm: np.ndarray      # f32 [hidden]
    layers: list
    eps: float = RMS_EPS


def model_weights(seed=0, hidden=HIDDEN, vocab=VOCAB, n_layers=N_LAYERS, n_dense=N_DENSE,
                  attention_layers=ATTENTION_LAYERS, moe_ff=MOE_FF, dense_ff=DENSE_FF, n_experts=N_EXPERTS,
                  n_heads=N_HEADS, n_kv_heads=N_KV_HEADS, embd_dtype=Q6_K):
    """LFM2.5-8B-A1B's layer schedule at any size: attention on `attention_layers`, the gated
    short conv elsewhere, dense FFN below n_dense, MoE above (down Q4_K on even layers, Q6_K on
    odd); norm gains ~ 1 + N(0, 0.05)."""
    g = rng(seed, 9100)
    gains = []
    for layer in range(n_layers):  # the norm gains share one stream: drawn in layer order
        an = (1.0 + 0.05 * g.standard_normal(hidden)).astype(np.float32)
        fn = (1.0 + 0.05 * g.standard_normal(hidden)).astype(np.float32)
        gains.append((an, fn))

    def one(layer):
        if layer in attention_layers:
            op = attn_weights(seed, layer, hidden, n_heads, n_kv_heads)
        else:
            op = conv_weights(seed, layer, hidden, in_dtype=Q4_K, out_dtype=Q6_K if layer % 2 else Q4_K)
        if layer < n_dense:
            ffn = dense_weights(seed, layer, hidden, dense_ff)
        else:
            ffn = moe_weights(seed, layer, hidden, moe_ff, n_experts, down_dtype=Q4_K if layer % 2 == 0 else Q6_K)
        return DecoderLayerWeights(gains[layer][0], gains[layer][1], op, ffn)

    layers = _par_map(one, range(n_layers))
    te = quant_tensor(rng(seed, 9101), embd_dtype, hidden, vocab)
    final = (1.0 + 0.05 * g.standard_normal(hidden)).astype(np.float32)
    return ModelWeights(hidden, vocab, embd_dtype, te, final, layers)


def model_gguf(mw, arch="lfm2moe", head_count_kv_type=None):
    """A GgufWriter holding `mw` as LFM2.5-8B-A1B's GGUF names it (model.rs:619-660: tensor names
    and [in, out] dims) with the lfm2moe.* metadata config::validate reads (config.rs:51-89).
    head_count_kv_type: the array's element type (default U32)."""
    from . import gguf as G
    w = G.GgufWriter()
    ops = [L.op for L in mw.layers]
    att = [op for op in ops if hasattr(op, "n_heads")]
    conv = [op for op in ops if hasattr(op, "conv_w")]
    moe = [L.ffn for L in mw.layers if hasattr(L.ffn, "router")]
    dense = [L.ffn for L in mw.layers if not hasattr(L.ffn, "router")]
    n_dense = sum(1 for _ in dense)
    p = arch + "."
    w.add("general.architecture", G.STRING, arch)
    for key, v in (("block_count", len(mw.layers)), ("embedding_length", mw.hidden), ("vocab_size", mw.vocab),
                   ("attention.head_count", att[0].n_heads if att else N_HEADS),
                   ("expert_count", moe[0].n_experts if moe else 0), ("expert_used_count", moe[0].n_used if moe else 0),
                   ("feed_forward_length", dense[0].ff if dense else 0),
                   ("expert_feed_forward_length", moe[0].moe_ff if moe else 0),
                   ("leading_dense_block_count", n_dense),
                   ("shortconv.l_cache", conv[0].l_cache if conv else CONV_L_CACHE)):
        w.add(p + key, G.U32, int(v))
    w.add(p + "rope.freq_base", G.F32, float(att[0].freq_base if att else ROPE_THETA))
    w.add(p + "attention.layer_norm_rms_epsilon", G.F32, float(mw.eps))
    kv = [op.n_kv_heads if hasattr(op, "n_heads") else 0 for op in ops]
    w.add(p + "attention.head_count_kv", G.ARRAY, (head_count_kv_type or G.U32, kv))

    h = mw.hidden
    w.add_tensor("token_embd.weight", (h, mw.vocab), mw.embd_dtype, mw.token_embd)
    w.add_tensor("token_embd_norm.weight", (h,), F32, mw.final_norm.astype(np.float32))
    for i, L in enumerate(mw.layers):
        b = f"blk.{i}."
        w.add_tensor(b + "attn_norm.weight", (h,), F32, L.attn_norm.astype(np.float32))
        w.add_tensor(b + "ffn_norm.weight", (h,), F32, L.ffn_norm.astype(np.float32))
        op = L.op
        if hasattr(op, "n_heads"):
            qd, kvd = op.n_heads * op.head_dim, op.n_kv_heads * op.head_dim
            w.add_tensor(b + "attn_q.weight", (h, qd), op.q_dtype, op.q)
            w.add_tensor(b + "attn_k.weight", (h, kvd), op.k_dtype, op.k)
            w.add_tensor(b + "attn_v.weight", (h, kvd), op.v_dtype, op.v)
            w.add_tensor(b + "attn_output.weight", (qd, h), op.o_dtype, op.o)
            w.add_tensor(b + "attn_q_norm.weight", (op.head_dim,), F32, op.q_norm.astype(np.float32))
            w.add_tensor(b + "attn_k_norm.weight", (op.head_dim,), F32, op.k_norm.astype(np.float32))
        else:
            w.add_tensor(b + "shortconv.in_proj.weight", (h, 3 * h), op.in_dtype, op.in_proj)
            w.add_tensor(b + "shortconv.conv.weight", (op.l_cache, h), F32, op.conv_w.astype(np.float32))
            w.add_tensor(b + "shortconv.out_proj.weight", (h, h), op.out_dtype, op.out_proj)
        f = L.ffn
        if hasattr(f, "router"):
            w.add_tensor(b + "ffn_gate_inp.weight", (h, f.n_experts), F32, f.router.astype(np.float32))
            w.add_tensor(b + "exp_probs_b.bias", (f.n_experts,), F32, f.exp_probs_b.astype(np.float32))
            w.add_tensor(b + "ffn_gate_exps.weight", (h, f.moe_ff, f.n_experts), f.gate_dtype, f.gate_exps)
            w.add_tensor(b + "ffn_up_exps.weight", (h, f.moe_ff, f.n_experts), f.up_dtype, f.up_exps)
            w.add_tensor(b + "ffn_down_exps.weight", (f.moe_ff, h, f.n_experts), f.down_dtype, f.down_exps)
        else:
            w.add_tensor(b + "ffn_gate.weight", (h, f.ff), f.gate_dtype, f.gate)
            w.add_tensor(b + "ffn_up.weight", (h, f.ff), f.up_dtype, f.up)
            w.add_tensor(b + "ffn_down.weight", (f.ff, h), f.down_dtype, f.down)
    return w
