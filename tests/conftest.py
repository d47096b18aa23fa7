import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: full-size configurations")


@pytest.fixture(scope="session")
def orc():
    import oracle
    return oracle


@pytest.fixture(scope="session")
def llk():
    """The product library (built in-tree by __graft_entry__.build())."""
    import dslcompiler_amd
    from dslcompiler_amd import _lib
    if not _lib.LIB_PATH.exists():
        from dslcompiler_amd import build
        build.build(lib_only=True)
    dslcompiler_amd.lib()
    return dslcompiler_amd


@pytest.fixture(scope="session")
def gpu(llk):
    """torch with a gfx950 device; the tests using it are marked gpu."""
    import torch
    if not torch.cuda.is_available():
        pytest.fail("gpu test selected but no GPU is visible")
    info = llk.device_info()
    assert info["status"] == 0, f"device is not gfx950: {info}"
    return torch
