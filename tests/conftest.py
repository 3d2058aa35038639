import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT, ROOT / "rlx-models_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; parity tests through the C ABI")


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle

    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def ctx():
    """One rlxq context for the whole GPU session."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import rlxq

    c = rlxq.Context(0)
    yield c
    torch.cuda.synchronize()
    c.close()


@pytest.fixture
def rng():
    return np.random.default_rng(0)


def announce(msg: str) -> None:
    """Prints the case name before a GPU step, so a fault names its case."""
    print(f"[case] {msg}", flush=True)
