"""pytest setup: import paths and the ``gpu`` marker.

``gpu`` tests run on the MI355X box (``pytest -m gpu``); everything else runs
on the CPU container (``pytest -m "not gpu"``).  GPU tests skip themselves
when no HIP device is visible, but never fall back to a CPU path.
"""

import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "nki-autotune_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

import pytest  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def _gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available() and torch.cuda.device_count() > 0
    except Exception:
        return False


@pytest.fixture(scope="session")
def gpu():
    """Skip unless a HIP device is present; return cuda:0."""
    if not _gpu_available():
        pytest.skip("no HIP device visible")
    import torch

    return torch.device("cuda:0")
