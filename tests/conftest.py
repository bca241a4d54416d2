"""Shared test setup: the `gpu` marker, the package loader and the oracle."""
from __future__ import annotations

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def O():
    import oracle
    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def gdn():
    import __graft_entry__
    return __graft_entry__.load_package()


@pytest.fixture(scope="session")
def dev(gdn):
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test collected on a machine without a GPU")
    assert gdn.available(), "current device is not gfx950"
    return torch.device("cuda:0")


@pytest.fixture(autouse=True)
def _seed():
    np.random.seed(1234)
