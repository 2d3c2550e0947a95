import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def cuda():
    """Device for GPU tests; the HIP library must be built (no fallback)."""
    import torch

    from teenyformers_amd import _lib

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    _lib.lib()  # raises if libteeny_hip.so is missing
    torch.cuda.init()
    rc = _lib.lib().teeny_init()
    assert rc == 0, f"teeny_init failed: {_lib.strerror(rc)}"
    return torch.device("cuda:0")
