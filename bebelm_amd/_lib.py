"""ctypes binding of libbebelm_moe.so (include/bebelm_moe.h).

The library must have been built (bebelm_amd/build.py, or __graft_entry__.build()); importing a
missing library raises instead of falling back to anything else.
"""
import ctypes
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libbebelm_moe.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "bebelm_moe.h")

(BB_OK, BB_ERR_ARG, BB_ERR_DTYPE, BB_ERR_SHAPE, BB_ERR_HIP, BB_ERR_OOM, BB_ERR_RANGE, BB_ERR_FORMAT, BB_ERR_IO,
 BB_ERR_MISSING) = range(10)
LOC_HOST, LOC_DEVICE = 0, 1

c_void_p = ctypes.c_void_p
c_size_t = ctypes.c_size_t
c_int = ctypes.c_int
c_uint32 = ctypes.c_uint32
c_float = ctypes.c_float
P = ctypes.POINTER


class BBError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"bebelm_moe error {code}: {msg}")
        self.code = code


class FusedJob(ctypes.Structure):
    _fields_ = [("dtype", c_uint32), ("w", c_void_p), ("byte_off", c_size_t), ("n_in", c_size_t),
                ("n_out", c_size_t), ("qx_q", c_void_p), ("qx_scales", c_void_p), ("qx_sums", c_void_p),
                ("x", c_void_p)]


class RouteTrace(ctypes.Structure):
    _fields_ = [("logits", c_void_p), ("sel", c_void_p), ("w", c_void_p), ("counts", c_void_p),
                ("offsets", c_void_p), ("perm", c_void_p), ("ties", c_void_p), ("margin", c_void_p)]


class LayerDesc(ctypes.Structure):
    _fields_ = [("ffn_norm", c_void_p), ("moe", c_void_p), ("dense", c_void_p)]


class DecoderLayer(ctypes.Structure):
    _fields_ = [("attn_norm", c_void_p), ("ffn_norm", c_void_p), ("conv", c_void_p), ("attn", c_void_p),
                ("moe", c_void_p), ("dense", c_void_p)]


class GgufTensorInfo(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("n_dims", c_uint32), ("dims", P(ctypes.c_uint64)),
                ("ggml_type", c_uint32), ("offset", ctypes.c_uint64), ("data_start", ctypes.c_uint64),
                ("data_len", ctypes.c_uint64)]


_SIGS = {
    "bb_last_error": (ctypes.c_char_p, []),
    "bb_version": (ctypes.c_char_p, []),
    "bb_ctx_create": (c_int, [c_int, P(c_void_p)]),
    "bb_ctx_destroy": (c_int, [c_void_p]),
    "bb_ctx_set_stream": (c_int, [c_void_p, c_void_p]),
    "bb_ctx_get_stream": (c_int, [c_void_p, P(c_void_p)]),
    "bb_ctx_synchronize": (c_int, [c_void_p]),
    "bb_ctx_profile": (c_int, [c_void_p, c_int]),
    "bb_kernel_count": (c_int, []),
    "bb_ctx_kernel_stats": (c_int, [c_void_p, c_int, P(ctypes.c_char_p), P(ctypes.c_double), P(ctypes.c_int64)]),
    "bb_ctx_reset_stats": (c_int, [c_void_p]),
    "bb_ctx_set_batched_min_entries": (c_int, [c_void_p, c_size_t]),
    "bb_tensor_upload": (c_int, [c_void_p, c_uint32, c_void_p, c_size_t, P(ctypes.c_uint64), c_int, P(c_void_p)]),
    "bb_tensor_free": (c_int, [c_void_p]),
    "bb_tensor_device_ptr": (c_int, [c_void_p, P(c_void_p)]),
    "bb_quantize_q8": (c_int, [c_void_p, c_void_p, c_size_t, c_void_p, c_void_p, c_void_p, c_int]),
    "bb_matvec": (c_int, [c_void_p, c_uint32, c_void_p, c_size_t, c_size_t, c_size_t, c_void_p, c_void_p, c_int]),
    "bb_matmul": (c_int, [c_void_p, c_uint32, c_void_p, c_size_t, c_size_t, c_size_t, c_void_p, c_size_t, c_void_p,
                          c_int]),
    "bb_matvec_fused_batch": (c_int, [c_void_p, P(FusedJob), c_size_t, c_void_p, c_int]),
    "bb_swiglu": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, c_int]),
    "bb_sigmoid_slice": (c_int, [c_void_p, c_void_p, c_size_t, c_int]),
    "bb_add_scaled": (c_int, [c_void_p, c_void_p, c_void_p, c_float, c_size_t, c_int]),
    "bb_add_assign": (c_int, [c_void_p, c_void_p, c_void_p, c_size_t, c_int]),
    "bb_rmsnorm": (c_int, [c_void_p, c_void_p, c_void_p, c_float, c_size_t, c_size_t, c_void_p, c_int]),
    "bb_logits_from_hidden": (c_int, [c_void_p, c_void_p, c_void_p, c_float, c_void_p, c_void_p, c_int]),
    "bb_moe_create": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, P(c_void_p)]),
    "bb_moe_destroy": (c_int, [c_void_p]),
    "bb_moe_forward": (c_int, [c_void_p, c_void_p, c_void_p, c_size_t, c_void_p, c_int, P(RouteTrace)]),
    "bb_moe_forward_noalloc": (c_int, [c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]),
    "bb_dense_create": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, P(c_void_p)]),
    "bb_dense_destroy": (c_int, [c_void_p]),
    "bb_dense_forward": (c_int, [c_void_p, c_void_p, c_void_p, c_size_t, c_void_p, c_int]),
    "bb_stack_create": (c_int, [c_void_p, P(LayerDesc), c_size_t, c_float, P(c_void_p)]),
    "bb_stack_destroy": (c_int, [c_void_p]),
    "bb_stack_forward": (c_int, [c_void_p, c_void_p, c_void_p, c_size_t, c_void_p, c_int]),
    "bb_conv_step": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, c_size_t, c_void_p, c_int]),
    "bb_conv_prefill": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, c_size_t, c_size_t, c_void_p,
                                c_int]),
    "bb_softmax": (c_int, [c_void_p, c_void_p, c_size_t, c_size_t, c_int]),
    "bb_attention_decode": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, c_size_t, c_size_t, c_size_t,
                                    c_void_p, c_int]),
    "bb_rope_neox": (c_int, [c_void_p, c_void_p, c_size_t, c_size_t, c_size_t, c_float, c_int]),
    "bb_conv_op_create": (c_int, [c_void_p, c_void_p, c_void_p, c_size_t, c_void_p, P(c_void_p)]),
    "bb_conv_op_destroy": (c_int, [c_void_p]),
    "bb_conv_op_forward": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p, c_int]),
    "bb_kv_cache_create": (c_int, [c_void_p, c_size_t, c_size_t, P(c_void_p)]),
    "bb_kv_cache_destroy": (c_int, [c_void_p]),
    "bb_kv_cache_length": (c_int, [c_void_p, P(c_size_t)]),
    "bb_kv_cache_read": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int]),
    "bb_kv_cache_evict_front": (c_int, [c_void_p, c_void_p, c_size_t]),
    "bb_attn_op_create": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_size_t,
                                  c_size_t, c_float, c_float, P(c_void_p)]),
    "bb_attn_op_destroy": (c_int, [c_void_p]),
    "bb_attn_op_forward": (c_int, [c_void_p, c_void_p, c_void_p, c_size_t, c_void_p, c_size_t, c_void_p, c_int]),
    "bb_model_create": (c_int, [c_void_p, c_void_p, c_void_p, P(DecoderLayer), c_size_t, c_float, P(c_void_p)]),
    "bb_model_destroy": (c_int, [c_void_p]),
    "bb_cache_create": (c_int, [c_void_p, c_void_p, c_size_t, P(c_void_p)]),
    "bb_cache_clone": (c_int, [c_void_p, c_void_p, P(c_void_p)]),
    "bb_cache_destroy": (c_int, [c_void_p]),
    "bb_cache_reset": (c_int, [c_void_p, c_void_p]),
    "bb_cache_position": (c_int, [c_void_p, P(c_size_t)]),
    "bb_cache_kv_length": (c_int, [c_void_p, P(c_size_t)]),
    "bb_cache_evict_front": (c_int, [c_void_p, c_void_p, c_size_t]),
    "bb_cache_layer_state": (c_int, [c_void_p, c_void_p, c_size_t, c_void_p, c_void_p, c_void_p, c_int]),
    "bb_model_run_layers": (c_int, [c_void_p, c_void_p, c_void_p, c_size_t, c_void_p, c_void_p, c_int]),
    "bb_model_forward_step": (c_int, [c_void_p, c_void_p, c_uint32, c_void_p, c_void_p, c_int]),
    "bb_model_absorb": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, c_size_t]),
    "bb_gguf_open": (c_int, [ctypes.c_char_p, P(c_void_p)]),
    "bb_gguf_open_bytes": (c_int, [c_void_p, c_size_t, P(c_void_p)]),
    "bb_gguf_close": (c_int, [c_void_p]),
    "bb_gguf_header": (c_int, [c_void_p, P(c_uint32), P(ctypes.c_uint64), P(ctypes.c_uint64), P(c_size_t),
                               P(c_size_t)]),
    "bb_gguf_tensor": (c_int, [c_void_p, c_size_t, P(GgufTensorInfo)]),
    "bb_gguf_find_tensor": (c_int, [c_void_p, ctypes.c_char_p, P(c_size_t)]),
    "bb_gguf_tensor_data": (c_int, [c_void_p, c_size_t, P(c_void_p), P(c_size_t)]),
    "bb_gguf_meta_key": (c_int, [c_void_p, c_size_t, P(ctypes.c_char_p)]),
    "bb_gguf_meta_type": (c_int, [c_void_p, ctypes.c_char_p, P(c_uint32), P(c_uint32), P(c_size_t)]),
    "bb_gguf_get_u32": (c_int, [c_void_p, ctypes.c_char_p, P(c_uint32)]),
    "bb_gguf_get_f32": (c_int, [c_void_p, ctypes.c_char_p, P(c_float)]),
    "bb_gguf_get_str": (c_int, [c_void_p, ctypes.c_char_p, P(c_void_p), P(c_size_t)]),
    "bb_gguf_get_u32_array": (c_int, [c_void_p, ctypes.c_char_p, P(c_uint32), c_size_t, P(c_size_t)]),
    "bb_gguf_get_str_item": (c_int, [c_void_p, ctypes.c_char_p, c_size_t, P(c_void_p), P(c_size_t)]),
    "bb_gguf_validate": (c_int, [c_void_p]),
    "bb_gguf_check_tensors": (c_int, [c_void_p, P(c_size_t)]),
    "bb_gguf_upload": (c_int, [c_void_p, c_void_p, c_size_t, P(c_void_p)]),
    "bb_model_load": (c_int, [c_void_p, c_void_p, P(c_void_p)]),
}

_lib = None


def header_symbols(path=HEADER):
    """Function names declared in include/bebelm_moe.h."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(bb_[a-z0-9_]+)\s*\(", text)))


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is not built; run `python bebelm_amd/build.py` first")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def check(rc):
    if rc != BB_OK:
        raise BBError(rc, lib().bb_last_error().decode())
    return rc
