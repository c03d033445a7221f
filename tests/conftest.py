"""Test tiers: ``-m "not gpu"`` runs on any host (oracle vs golden vectors, host
API, library exports); ``-m gpu`` needs an MI355X and runs the HIP parity tests."""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X / gfx950)")
    config.addinivalue_line("markers", "slow: long-running case")


def gpu_available() -> bool:
    try:
        import torch

        return bool(torch.cuda.is_available())
    except Exception:  # pragma: no cover - import failures mean no GPU
        return False
