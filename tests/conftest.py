import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; run with -m gpu")


@pytest.fixture(scope="session")
def oracle_lib():
    """Build (if needed) and load the oracle's C library."""
    from oracle import build as ob
    if not ob.LIB.exists():
        ob.build()
    from oracle import moe_oracle
    return moe_oracle._clib()


@pytest.fixture(scope="session")
def g5lib():
    """The product library, built in-tree (it is loaded, never called, on the CPU)."""
    from genet5_amd import _lib
    if not _lib.LIB_PATH.exists():
        from genet5_amd import build
        build.build()
    return _lib.lib()


@pytest.fixture(scope="session")
def cuda_device():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test needs a visible GPU (torch.cuda.is_available() is False)")
    name = torch.cuda.get_device_properties(0).gcnArchName
    if not name.startswith("gfx950"):
        pytest.fail(f"expected a gfx950 GPU, found {name}")
    from genet5_amd import _lib
    _lib.lib()
    return torch.device("cuda:0")
