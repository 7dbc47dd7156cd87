import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = Path(__file__).parent / "golden" / "golden.npz"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def golden():
    data = np.load(GOLDEN, allow_pickle=False)
    cases = {}
    for key in data.files:
        op, dt, case, field = key.split("/")
        cases.setdefault((op, dt, case), {})[field] = data[key]
    return cases
