import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line(
        "markers", "gpu: needs an MI355X (gfx950) GPU; runs the HIP kernels")


@pytest.fixture(scope="session")
def device():
    """The GPU under test. GPU tests fail (never skip) without one."""
    import torch
    assert torch.cuda.is_available(), "GPU test run without a visible GPU"
    import mini_triton_nvgpu_v1_amd as tb
    tb.lib()  # raises if the HIP library is missing: no silent fallback
    return torch.device("cuda:0")
