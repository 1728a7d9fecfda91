"""Builds libbebelm_moe.so (gfx950) in-tree from bebelm_amd/csrc/*.hip.

The library is the product: a C-ABI shared object (include/bebelm_moe.h). Flags:
  -ffp-contract=off                         no FMA contraction: f32 epilogues keep the
                                            reference's rounding sequence
  -fhip-fp32-correctly-rounded-divide-sqrt  IEEE f32 divide / sqrt (sigmoid, renorm, rmsnorm)
  -target-feature -packed-fp32-ops          no packed-FP32 instructions on this hardware pool
  -amdgpu-mfma-vgpr-form                    MFMA results in VGPRs (the GEMM epilogues read them
                                            with VALU; no accumulator-register copies)
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libbebelm_moe.so")
SOURCES = ["bb_kernels.hip", "bb_decode.hip", "bb_prefill.hip", "bb_ops.hip", "bb_api.hip", "bb_gguf.hip"]
ARCH = os.environ.get("BB_OFFLOAD_ARCH", "gfx950")


def hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if cand and (os.path.isabs(cand) and os.path.exists(cand) or not os.path.isabs(cand)):
            return cand
    return "hipcc"


def flags():
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-shared",
        "-ffp-contract=off",
        "-fhip-fp32-correctly-rounded-divide-sqrt",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-mllvm", "-amdgpu-mfma-vgpr-form",
        "-Wall",
        "-Wno-unused-function",
    ]


def build(verbose=False):
    srcs = [os.path.join(CSRC, s) for s in SOURCES if os.path.exists(os.path.join(CSRC, s))]
    tmp = LIB + ".tmp"
    cmd = [hipcc()] + flags() + srcs + ["-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("hipcc failed building libbebelm_moe.so")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
