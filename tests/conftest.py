"""Shared pytest configuration: the ``gpu`` marker and import paths."""

from __future__ import annotations

import json
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = Path(__file__).resolve().parent / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


@pytest.fixture(scope="session")
def fixtures() -> dict:
    return json.loads((GOLDEN / "reference_fixtures.json").read_text())


@pytest.fixture(scope="session")
def cuda():
    import torch

    if not torch.cuda.is_available():  # pragma: no cover - GPU box only
        pytest.skip("ROCm device required")
    return torch.device("cuda", 0)
