import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for path in (ROOT, os.path.join(ROOT, "rns-llm_amd")):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and librnsmx.so")


def gpu_ready() -> bool:
    import torch

    from rns_llm_amd import _native

    return torch.cuda.is_available() and _native.available()


@pytest.fixture(scope="session")
def backend():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from rns_llm_amd import HipRNSBackend

    # A GPU test must exercise the native library: HipRNSBackend raises
    # RuntimeError (failing the test) when librnsmx.so is missing.
    return HipRNSBackend()
