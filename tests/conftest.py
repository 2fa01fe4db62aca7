"""Shared pytest configuration: the ``gpu`` marker and common fixtures."""

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

# ASE is not installed in this image: the calculator tests run against the
# test-only stand-in under tests/ase_standin unless a real ASE is importable.
try:
    import ase  # noqa: F401
except ImportError:
    sys.path.append(str(ROOT / "tests" / "ase_standin"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built extension")


@pytest.fixture(scope="session")
def golden_dir():
    return ROOT / "tests" / "golden"
