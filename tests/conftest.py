import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))
TESTS = Path(__file__).resolve().parent
if str(TESTS) not in sys.path:
    sys.path.insert(0, str(TESTS))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


GOLDEN = TESTS / "golden" / "reference_outputs.npz"


@pytest.fixture(scope="session")
def gold():
    """The compiled reference's outputs on the seeded fixture inputs (tests/golden/make_golden.py)."""
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}
