import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "aet-cnn_amd"))
sys.path.insert(0, os.path.join(ROOT, "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libach.so)")
    config.addinivalue_line("markers", "slow: long CPU oracle runs")


@pytest.fixture(scope="session")
def gpu():
    """The HIP library on a real device; fails (not skips) when either is missing."""
    import aetcnn
    lib = aetcnn.ops()
    n = lib.ach_device_count()
    assert n > 0, "no HIP device visible"
    aetcnn.check(lib.ach_set_device(0), "ach_set_device")
    return lib


@pytest.fixture(scope="session")
def oracle():
    import oracle_lib
    return oracle_lib


def rel_err(a, b):
    """Normwise relative error ||a-b||_2 / ||b||_2 (b = reference)."""
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    nb = np.linalg.norm(b)
    if nb == 0:
        return float(np.linalg.norm(a))
    return float(np.linalg.norm(a - b) / nb)
