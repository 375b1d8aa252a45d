import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through liblbq on the device)")


def _gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _gpu_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def oracle():
    import oracle as o
    o._load()
    return o


@pytest.fixture(scope="session")
def lbq():
    """The built HIP library (built here only if nothing is built yet)."""
    from lightbulb_amd import _lib
    if not _lib.LIB_PATH.exists():
        from lightbulb_amd import build
        build.build()
    return _lib.lib()


@pytest.fixture(scope="session")
def dev():
    import torch
    return torch.device("cuda", 0)
