import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libbebelm_moe.so on cuda:0)")
    config.addinivalue_line("markers", "slow: takes more than a few seconds on the CPU")


@pytest.fixture(scope="session")
def oracle():
    from oracle import bbo

    bbo.lib()
    return bbo


@pytest.fixture(scope="session")
def gpu_ctx():
    """One library context for every GPU test of the session (cuda:0)."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a visible GPU")
    from bebelm_amd.model import Context

    ctx = Context(0)
    yield ctx
    ctx.close()
