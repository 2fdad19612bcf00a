import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line(
        "markers", "gpu: needs a real MI355X (HIP device); parity tests proper")


@pytest.fixture(scope="session")
def vectors():
    return np.load(os.path.join(GOLDEN, "ref_vectors.npz"))


@pytest.fixture(scope="session")
def scripts():
    return np.load(os.path.join(GOLDEN, "ref_scripts.npz"))


@pytest.fixture(scope="session")
def engine():
    """One HIP context for the whole GPU session (tests marked gpu)."""
    from fable5_llm_amd import engine as eng
    ctx = eng.Context(0)
    yield ctx
    ctx.close()
