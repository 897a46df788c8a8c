import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))
TESTS = Path(__file__).resolve().parent
if str(TESTS) not in sys.path:
    sys.path.insert(0, str(TESTS))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library on the device)")


@pytest.fixture(scope="session")
def oracle_lib():
    import oracle

    oracle.build()
    return oracle


@pytest.fixture(scope="session")
def kt():
    """The HIP library's host mirror, with a device present (fails loudly otherwise)."""
    import kotensor_amd

    if not kotensor_amd.LIBRARY_PATH.exists():
        pytest.fail("libkotensor_hip.so is not built (python -m kotensor_amd.build)")
    n = kotensor_amd.device_count()
    if n < 1:
        pytest.fail("no HIP device visible")
    print(f"[kt] devices={n} lib={kotensor_amd.LIBRARY_PATH}", flush=True)
    return kotensor_amd


def normwise_rel(actual: np.ndarray, expected: np.ndarray) -> float:
    """||actual - expected||_F / ||expected||_F (0 when both are 0)."""
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    den = np.linalg.norm(e)
    num = np.linalg.norm(a - e)
    if den == 0.0:
        return float(num)
    return float(num / den)
