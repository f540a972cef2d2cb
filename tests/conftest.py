import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP) device and libpnfx.so")


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU in this process")
    return torch.device("cuda:0")


def golden(name):
    import numpy as np

    return np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False)


def pytest_sessionfinish(session, exitstatus):
    """Write the recorded parity ratios to $PNFX_PARITY_REPORT (JSON), if that is set."""
    path = os.environ.get("PNFX_PARITY_REPORT")
    if not path:
        return
    import json

    from tests.helpers import PARITY_LOG

    os.makedirs(os.path.dirname(os.path.abspath(path)), exist_ok=True)
    with open(path, "w") as f:
        json.dump(PARITY_LOG, f, indent=0)
