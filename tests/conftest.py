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
def q9():
    """Row images and y32 of the reference's pack_ddr_rows / matvec_y32 at
    K = 4096 / 8192 / 12288 (1 / 2 / 3 scale beats per row)."""
    return np.load(os.path.join(GOLDEN, "q9_vectors.npz"))


def q9_cases(q9):
    tags = sorted({k.rsplit("_", 1)[0] for k in q9.files if k.endswith("_shape")})
    for t in tags:
        n, k, sh, stride = (int(v) for v in q9[f"{t}_shape"])
        yield dict(tag=t, N=n, K=k, sh=sh, stride=stride, w4=q9[f"{t}_w4"],
                   m=q9[f"{t}_m"], x8=q9[f"{t}_x8"], img=q9[f"{t}_img"].tobytes(),
                   y32=q9[f"{t}_y32"], y32_ext=q9[f"{t}_y32_ext"])


@pytest.fixture(scope="session")
def engine():
    """One HIP context for the whole GPU session (tests marked gpu)."""
    from fable5_llm_amd import engine as eng
    ctx = eng.Context(0)
    yield ctx
    ctx.close()
