"""The GPU's expf (bebelm_amd/csrc/bb_expf.h) against the platform expf that the reference's
f32::exp calls (activation.rs:5-13, glibc on linux-gnu).

The header is compiled as plain C next to glibc's expf and compared bit for bit over a strided
sweep of every float bit pattern, plus the inputs where an evaluation without the fused range
reduction would differ. Run with stride 1 it checks all 2^32 inputs (about a minute on 8 cores;
every one matched on this container's glibc 2.35).
"""
import os
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

# Discriminating inputs (bit patterns): the FMA-contracted and plain evaluations of the same
# steps round differently here; specials: ±0, ±inf, NaN, overflow/underflow edges, subnormal out.
SPECIAL = ["0x4202422f", "0xc27c65d9", "0x00000000", "0x80000000", "0x7f800000", "0xff800000", "0x7fc00000",
           "0x42b17217", "0x42b17218", "0xc2cff1b4", "0xc2cff1b5", "0xc2ce8ed0", "0xc2b00000", "0x3f800000"]


@pytest.fixture(scope="module")
def checker():
    d = tempfile.mkdtemp()
    exe = os.path.join(d, "expf_check")
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-I", os.path.join(ROOT, "bebelm_amd", "csrc"),
                    os.path.join(ROOT, "tests", "expf_check.c"), "-o", exe, "-lm"], check=True)
    return exe


def run(checker, stride, extra=()):
    out = subprocess.run([checker, str(stride), *extra], capture_output=True, text=True, check=True).stdout.split()
    return int(out[0]), int(out[1]), out[2]


def test_expf_matches_platform_strided(checker):
    checked, bad, first = run(checker, 997, SPECIAL)
    assert checked > 4_000_000
    assert bad == 0, f"first mismatch at {first}"


def test_expf_discriminating_inputs(checker):
    checked, bad, first = run(checker, 1 << 32, SPECIAL)
    assert bad == 0, f"first mismatch at {first}"
