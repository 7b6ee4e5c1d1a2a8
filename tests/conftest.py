"""Shared pytest configuration.

Tests marked ``gpu`` need an MI355X (gfx950) and the built library; the CPU
suite (``-m "not gpu"``) covers the oracle, host logic and the C-ABI exports.
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest
import torch

REPO_ROOT = Path(__file__).resolve().parents[1]
if str(REPO_ROOT) not in sys.path:
    sys.path.insert(0, str(REPO_ROOT))


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU and the built HIP library")


@pytest.fixture(autouse=True)
def deterministic_seed() -> None:
    torch.manual_seed(1234)


@pytest.fixture
def device() -> torch.device:
    """The GPU under test; GPU tests fail loudly when it or the library is missing."""

    if not torch.cuda.is_available():
        pytest.fail("a GPU is required for tests marked gpu")
    from tensorforge_amd import _native

    _native.library()  # raises if the gfx950 library is not built
    return torch.device("cuda", 0)
