import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the C-ABI on cuda:0)")


@pytest.fixture(scope="session")
def torch_gpu():
    import torch
    assert torch.cuda.is_available(), "GPU test collected on a host without a GPU"
    import qw38_amd
    qw38_amd.lib()  # fail loudly if the HIP library is missing
    return torch
