"""Shared pytest setup: markers and import paths."""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "temporal-random-walk_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP engine)")


import pytest  # noqa: E402


@pytest.fixture(autouse=True)
def _torch_runtime_first(request):
    """Before a GPU test, torch's HIP runtime is started: torch ships its own
    copy of the runtime library, and in one process it must come up before
    the engine's (which loads the system copy), or torch finds no device.
    Tests that hand torch tensors to the engine need both."""
    if request.node.get_closest_marker("gpu") is not None:
        import torch
        if torch.cuda.is_available():
            torch.zeros(1, device="cuda")
    yield
