"""Shared test setup: import paths, the ``gpu`` marker, and small helpers.

CPU tests (``-m "not gpu"``) check the oracle against the golden fixtures and
the host logic; GPU tests (``-m gpu``) compare the HIP path with the oracle.
"""
from __future__ import annotations

import json
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
PACKAGE_ROOT = ROOT / "inference-engine_amd"
GOLDEN = Path(__file__).resolve().parent / "golden"
for path in (ROOT, PACKAGE_ROOT):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP path)")


def golden(name: str) -> dict:
    return json.loads((GOLDEN / f"{name}.json").read_text())


@pytest.fixture(scope="session")
def gpu():
    """Skip unless a GPU is visible; returns the torch device."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    return torch.device("cuda", 0)
