import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "tests"), os.path.join(ROOT, "x100-gemm_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def pytest_report_header(config):
    return "x100-gemm MI355X backend tests (root %s)" % ROOT


@pytest.fixture(scope="session")
def dev():
    """torch cuda device for GPU tests; fails loudly if the HIP library is not built."""
    import torch
    import x100hip
    x100hip.lib()
    assert torch.cuda.is_available(), "GPU test run without a visible GPU"
    c = x100hip.caps()
    assert c.is_gfx950, "device is %s, not gfx950" % c.arch.decode()
    return torch.device("cuda:0")
