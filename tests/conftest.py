import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT / "echo-core_amd", ROOT / "oracle"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

GOLDEN = Path(__file__).resolve().parent / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def oc():
    from oracle import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def golden():
    return np.load(GOLDEN / "kernels_golden.npz")


@pytest.fixture(scope="session")
def hip():
    """The product library (libechohip.so) bound through its C ABI, on cuda:0."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from echohip import lib
    return lib.load()


def rel_l2(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    den = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (den if den > 0 else 1.0))
