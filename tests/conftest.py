"""Shared test setup: the ``gpu`` marker, the oracle build, small helpers."""
import os
import sys

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP) device")


@pytest.fixture(scope="session", autouse=True)
def _oracle_built():
    from oracle import build
    if not os.path.exists(build.LIBRARY):
        build.build()
    yield


def gpu_available() -> bool:
    return torch.cuda.is_available()


def margin_checked_seed(make, cutoff, dtype=np.float32, start=0, tries=20, margin=1e-5):
    """First seed from ``start`` whose structure has no candidate pair within ``margin``
    of the cutoff (so no rounding can move a pair across it)."""
    from oracle.nl import neighbor_list
    for seed in range(start, start + tries):
        s = make(seed)
        ei, sh, near = neighbor_list(s.pos, cutoff, s.cell, s.pbc, dtype=dtype, margin=margin)
        if near == 0:
            return seed, s, ei, sh
    raise RuntimeError("no margin-checked seed found")
