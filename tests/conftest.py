import os
import sys

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "mamba-integer_amd")
for p in (PKG, os.path.join(REPO, "oracle"), REPO):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and libmamba_int.so")


@pytest.fixture(scope="session")
def cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from mamba_int import _lib
    _lib.load()  # a missing library is an error, not a skip
    return torch.device("cuda:0")


@pytest.fixture
def rng():
    return np.random.default_rng(12345)


def i8(rng, *shape, lo=-127, hi=127):
    return rng.integers(lo, hi + 1, size=shape, dtype=np.int8)
