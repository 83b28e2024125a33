import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C ABI)")


def load_golden(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


def rel_max_err(y, y_ref):
    """max |y - y_ref| / ||y_ref||_2 (the north-star parity measure)."""
    y = np.asarray(y, np.float64)
    y_ref = np.asarray(y_ref, np.float64)
    n = np.linalg.norm(y_ref)
    return float(np.max(np.abs(y - y_ref)) / (n if n > 0 else 1.0))


# Parity tolerance for fp32 outputs: max relative error 1e-5 of ||y||_2
# (fp32 accumulation-order differences only).
TOL = 1e-5


@pytest.fixture(scope="session")
def cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible GPU")
    import lutmac_amd
    lutmac_amd.lib()
    return torch.device("cuda:0")
