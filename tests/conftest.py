"""Test configuration: the ``gpu`` marker and shared helpers.

``-m "not gpu"`` runs on any host (oracle, host logic, library loading);
``-m gpu`` needs an MI355X and the built ``libdionw_hip.so``.
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library")


def pytest_collection_modifyitems(config: pytest.Config, items: list[pytest.Item]) -> None:
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU on this host")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def rel_fro(a: torch.Tensor, b: torch.Tensor) -> float:
    """Relative Frobenius distance ||a - b|| / ||b|| in float64."""
    a64, b64 = a.double().cpu(), b.double().cpu()
    return float((a64 - b64).norm() / b64.norm().clamp_min(1e-300))
