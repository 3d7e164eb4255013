from __future__ import annotations

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU and the built HIP library")


def golden(name: str) -> dict[str, np.ndarray]:
    with np.load(os.path.join(GOLDEN, name), allow_pickle=False) as data:
        return {key: data[key] for key in data.files}
