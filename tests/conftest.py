import json
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = Path(__file__).resolve().parent / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built liboq.so")


@pytest.fixture(scope="session")
def kat():
    return json.loads((GOLDEN / "ref_kat.json").read_text())


@pytest.fixture(scope="session")
def golden():
    with np.load(GOLDEN / "ref_random.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture(scope="session")
def ctx():
    """One device context for the whole GPU session (no fallback if liboq.so is absent)."""
    import oracle_amd

    c = oracle_amd.Context(0)
    yield c
    c.close()


def hexbytes(s: str) -> np.ndarray:
    return np.frombuffer(bytes.fromhex(s), dtype=np.uint8).copy()
