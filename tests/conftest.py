"""Shared test configuration.

Markers: ``gpu`` marks tests that need an MI355X (gfx950) device; everything
else runs on the CPU.  The native library and the oracle are loaded from the
tree; they are built only if nothing has been built yet.
"""
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "ullm-project_amd"
for p in (str(ROOT), str(PKG)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU")


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle
    if not oracle.LIB_PATH.exists():
        oracle.build()
    return oracle


@pytest.fixture(scope="session")
def uh():
    import ullm_hip
    if not ullm_hip.LIB_PATH.exists():
        import build as native_build
        native_build.build()
    return ullm_hip


@pytest.fixture(scope="session")
def gpu(uh):
    import torch
    if not torch.cuda.is_available():
        pytest.fail("gpu test selected but no GPU is visible")
    available, _, diag = uh.backend_probe()
    assert available, diag
    return torch.device("cuda:0")
