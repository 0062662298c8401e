"""Shared pytest setup: the ``gpu`` marker and repository-root imports."""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line(
        "markers", "gpu: needs a real MI355X (gfx950) and the built HIP library"
    )


@pytest.fixture(scope="session")
def golden():
    import numpy as np

    data = np.load(ROOT / "tests" / "golden" / "eb_golden.npz", allow_pickle=False)
    return {key: data[key] for key in data.files}


@pytest.fixture(scope="session")
def golden_dir():
    return ROOT / "tests" / "golden"
