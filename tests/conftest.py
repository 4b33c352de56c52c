"""Test configuration: import paths, the ``gpu`` marker and shared fixtures.

CPU tests (``-m "not gpu"``) cover the oracle against the reference's golden vectors,
the host logic and the C-ABI library's exports.  GPU tests (``-m gpu``) call the
gfx950 kernels through the C ABI and compare them with the oracle.
"""

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT / "tinygrad-dx12_amd"))
sys.path.insert(0, str(ROOT / "oracle"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built kernel library")


def _gpu_available() -> bool:
    import torch

    return torch.cuda.is_available()


def pytest_collection_modifyitems(config, items):
    if any(item.get_closest_marker("gpu") for item in items) and not _gpu_available():
        skip = pytest.mark.skip(reason="no HIP GPU visible")
        for item in items:
            if item.get_closest_marker("gpu"):
                item.add_marker(skip)


@pytest.fixture(scope="session")
def dev():
    import torch

    return torch.device("cuda:0")
