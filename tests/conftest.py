"""Shared pytest setup.

* registers the ``gpu`` marker (tests that need an MI355X);
* puts the repository root (for ``oracle``) and the package directory (for
  ``operatorlib``) on ``sys.path``;
* GPU fixtures fail loudly — never skip — when no GPU is visible, so a GPU run
  cannot pass on a silent fallback.
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
PKG = REPO / "orin-cuda-operator-library_amd"
for p in (str(REPO), str(PKG)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def device():
    import torch
    assert torch.cuda.is_available(), "GPU test selected but no HIP device is visible"
    return torch.device("cuda", 0)


@pytest.fixture(scope="session")
def lib(device):
    import operatorlib
    return operatorlib.clib()


@pytest.fixture(scope="session")
def ops(device):
    import operatorlib
    import torch
    operatorlib.load_operatorlib()
    return torch.ops.operatorlib
