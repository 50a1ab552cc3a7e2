"""Shared pytest setup: import paths, the ``gpu`` marker and common fixtures.

Tests marked ``gpu`` need a ROCm GPU and the built ``librwkv7_hip.so``; the
rest run on the CPU. GPU tests never read ``/root/reference``: they compare
the HIP path with the CPU oracle (``oracle/``) and the committed fixtures
under ``tests/golden/``.
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
for p in (REPO / "rwkv-tl_amd", REPO):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

GOLDEN = REPO / "tests" / "golden"


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU and the built HIP library")
    config.addinivalue_line("markers", "slow: long-running case")


@pytest.fixture(scope="session")
def manifest() -> dict:
    return json.loads((GOLDEN / "manifest.json").read_text())


@pytest.fixture(scope="session")
def golden_dir() -> Path:
    return GOLDEN


@pytest.fixture(scope="session")
def cuda():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test collected on a host without a ROCm GPU")
    return torch.device("cuda:0")
