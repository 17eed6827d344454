import importlib
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PKG = "mlx-server-runtime_amd"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle

    return oracle


@pytest.fixture(scope="session")
def mq():
    """The product package (directory name has dashes, so it is imported by string)."""
    return importlib.import_module(PKG)


def normwise_rel_err(y, ref):
    """max|y - ref| / max|ref| over the whole output (the matmul tolerance metric)."""
    import numpy as np

    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    denom = np.max(np.abs(ref)) if ref.size else 0.0
    if denom == 0.0:
        return float(np.max(np.abs(y - ref))) if y.size else 0.0
    return float(np.max(np.abs(y - ref)) / denom)
