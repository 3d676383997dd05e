import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (gfx950) and the built libmdl_hip.so")


@pytest.fixture(scope="session")
def device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    # The product has no fallback: a GPU box without the library is a failure.
    from mdl_amd import _lib

    _lib.lib()
    return torch.device("cuda:0")
