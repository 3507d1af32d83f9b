"""Shared pytest configuration: the ``gpu`` marker and repo-root imports."""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

REPO_ROOT = Path(__file__).resolve().parent.parent
if str(REPO_ROOT) not in sys.path:
    sys.path.insert(0, str(REPO_ROOT))

GOLDEN_DIR = Path(__file__).resolve().parent / "golden"


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def device():
    """The GPU under test; GPU tests require the native library (no fallback)."""

    import torch

    from crosspool_amd import _native

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible to torch")
    _native.library()  # raises NativeUnavailableError if the library was not built
    return torch.device("cuda", 0)
