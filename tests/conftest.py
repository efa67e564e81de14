"""Shared test setup: import paths, the `gpu` marker, and helpers.

`-m "not gpu"` runs here (no GPU): the oracle against its golden vectors and closed forms, the
host logic, and the C-ABI library's exports and validation (no compute calls). `-m gpu` runs the
parity tests proper on an MI355X, through the C ABI.
"""
from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest

# The library's test hooks (fattn_internal_*) act only in a process that sets this before the
# library loads; the tests that compare step 2's dQ sums with step 3's use them.
os.environ.setdefault("FATTN_TEST_HOOKS", "1")

REPO = Path(__file__).resolve().parent.parent
PKG = REPO / "candle-fused-attn_amd"
for p in (str(REPO), str(PKG)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle as o
    o.lib()
    return o


@pytest.fixture(scope="session")
def cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    return torch.device("cuda:0")
