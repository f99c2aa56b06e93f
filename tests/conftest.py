import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT, ROOT / "oracle"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C ABI)")


@pytest.fixture(scope="session")
def backend():
    """One HIP context for the GPU tests (the library must be built)."""
    from turboqwenfare_amd.backend import HipBackend

    be = HipBackend(0)
    yield be
    be.close()


def rel_err(got, want) -> float:
    """The reference's parity metric |g - c| / max(|c|, 1)
    (backend/metal/expert.rs:309-310), maximised over elements."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    return float(np.max(np.abs(got - want) / np.maximum(np.abs(want), 1.0)))
