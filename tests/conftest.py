import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def gpu():
    """Return the rec_amd library handle on a machine with a GPU; fail loudly if it is missing."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU in this process")
    import rec_amd

    lib = rec_amd.library()  # raises if the HIP extension is not built
    return lib
