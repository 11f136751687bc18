"""Shared test setup: import paths, the ``gpu`` marker, the built library."""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "costcut-infer_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X)")


@pytest.fixture(scope="session")
def built_lib() -> Path:
    """Path of libccq_hip.so; built here when missing (tests load what is built)."""
    from ccut import _build

    if not _build.LIB.exists():
        _build.build()
    return _build.LIB


@pytest.fixture(scope="session")
def gpu(built_lib):
    """A GPU device for the parity tests.  On a machine without a GPU the
    test is skipped; with a GPU, a missing or broken library is an error."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    from ccut import _lib

    _lib.lib()  # raises CcqLibraryError if unusable
    return torch.device("cuda", 0)
