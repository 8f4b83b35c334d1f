import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "trellis2-cuda_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built libspconv_amd.so")


@pytest.fixture(scope="session")
def gpu():
    """The HIP library on cuda:0; a GPU test fails loudly if either is missing."""
    import torch
    import spconv_amd
    assert torch.cuda.is_available(), "gpu test without a visible GPU"
    spconv_amd.load_library()
    spconv_amd.set_stream(torch.cuda.current_stream())
    return torch.device("cuda:0")
