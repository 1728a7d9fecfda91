"""bebelm_amd — MI355X-native (gfx950) sparse-MoE FFN path of maximecb/bebelm.

The product is libbebelm_moe.so (C ABI in include/bebelm_moe.h, HIP kernels in csrc/).
This package holds its ctypes binding and a host-side mirror of the reference's interface:
  bebelm_amd.model    Context, Tensor, MoeLayer (moe_ffn / moe_ffn_batch), DenseLayer, FfnStack
  bebelm_amd.kernels  quantize_q8, matvec, matmul, matvec_fused_batch, swiglu, ... mirrors
  bebelm_amd.synth    deterministic synthetic weights/inputs for the benchmark configurations
"""
from . import synth  # noqa: F401
from ._lib import BBError, LIB_PATH, header_symbols, lib  # noqa: F401

__all__ = ["synth", "BBError", "LIB_PATH", "header_symbols", "lib"]
