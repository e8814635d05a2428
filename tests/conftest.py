"""Shared fixtures.  `-m gpu` tests need an MI355X; everything else runs on
the CPU (oracle, golden fixtures, host logic, C-ABI exports)."""
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

import __graft_entry__  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (gfx950) and the built HIP library")


@pytest.fixture(scope="session")
def spc():
    return __graft_entry__.load()


@pytest.fixture(scope="session")
def orc():
    import oracle

    return oracle.orc()


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")
