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


# The batched-decode default for the LDS-staged kernel (rlxq_skinnyxl_*):
# formats Q4_1 (3), Q4_0 (2), Q8_0 (1), Q4_K (7), Q5_K (10) with K whole
# 256-element steps, up to 16 prepared rows (m for bf16 activations, 2m for
# f32), and up to 32 for Q4_1, Q4_0 and Q5_K.
XL_FORMATS = {3, 2, 1, 7, 10}


def skinny_xl_default(scheme: int, m: int, k: int, xdt: str = "bf16") -> bool:
    rows = 2 * m if xdt == "f32" else m
    return scheme in XL_FORMATS and (k // 128) % 2 == 0 and (rows <= 16 or (rows <= 32 and scheme in (3, 2, 10)))
