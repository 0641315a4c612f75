import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device")
    # build what is missing (tests load what is built; build() only when nothing is)
    need = [os.path.join(ROOT, "tierlm_amd", "libtlm_hip.so"), os.path.join(ROOT, "oracle", "liboracle.so")]
    if not all(os.path.exists(p) for p in need):
        import __graft_entry__
        __graft_entry__.build()


@pytest.fixture(scope="session")
def hip():
    """The HIP tier, initialised on cuda:0 (GPU tests only)."""
    import torch

    from tierlm_amd import quant as hq

    assert torch.cuda.is_available(), "GPU test run without a GPU"
    hq.init(0)
    return hq


@pytest.fixture(scope="session")
def dev():
    import torch
    return torch.device("cuda", 0)
