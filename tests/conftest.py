import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library")


@pytest.fixture(scope="session")
def dev():
    """cuda:0 with the HIP library loaded; GPU tests fail (not skip) when the
    library is missing on a machine that has a GPU."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU in this environment")
    from kessie_amd import _lib

    _lib.load()  # raises FileNotFoundError when the .so is absent
    return torch.device("cuda:0")
