"""Shared test setup: import paths, the ``gpu`` marker, and device fixtures."""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

REPO_ROOT = Path(__file__).resolve().parents[1]
for entry in (REPO_ROOT, REPO_ROOT / "sglang-legolink_amd"):
    if str(entry) not in sys.path:
        sys.path.insert(0, str(entry))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def gpu_device():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no ROCm device is visible")
    from legolink_amd import _native

    _native.load_library()  # fail loudly when the HIP library is not built
    return torch.device("cuda", 0)


def report(message: str) -> None:
    """Progress line that names the case before a GPU step runs."""

    print(message, file=sys.stderr, flush=True)
