import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import __graft_entry__ as entry  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the native HIP path)")


@pytest.fixture(autouse=True)
def _persistent_plans_by_default(monkeypatch):
    """Tests of the persistent kernel's plans (per-tile, split-K, narrow and short tiles) keep their
    shapes on that kernel: small-tile plans are off unless a test turns them on
    (tests/test_gpu_small_tiles.py forces them and checks the planner's own choice; the
    random-shape tests let the planner choose)."""
    monkeypatch.setenv("GG_SMALL", "0")


@pytest.fixture(scope="session")
def pkg():
    return entry.load_package()


@pytest.fixture(scope="session")
def oracle():
    return entry.load_oracle()
