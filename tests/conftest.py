"""Shared pytest configuration: the ``gpu`` marker and common fixtures."""

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built extension")


@pytest.fixture(scope="session")
def golden_dir():
    return ROOT / "tests" / "golden"
