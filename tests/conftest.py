from __future__ import annotations

import json
import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(Path(__file__).resolve().parent))

GOLDEN = Path(__file__).resolve().parent / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: long-running test")


@pytest.fixture(scope="session")
def kats() -> dict:
    return json.loads((GOLDEN / "reference_kats.json").read_text())


@pytest.fixture
def rng() -> np.random.Generator:
    return np.random.default_rng(1234)


def gpu_available() -> bool:
    if os.environ.get("PLH_FORCE_NO_GPU"):
        return False
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:  # pragma: no cover
        return False
