import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "sched-pass_amd"), os.path.join(ROOT, "oracle"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device")


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
    for it in items:
        if "gpu" in it.keywords:
            it.add_marker(skip)


@pytest.fixture(scope="session")
def schedlib():
    """libschedpd.so, built in-tree if this checkout has none (hipcc
    cross-compiles gfx950 without a GPU)."""
    import sched_abi
    if not os.path.exists(sched_abi.LIB_PATH):
        import build_lib
        build_lib.build()
    return sched_abi.load_library()


@pytest.fixture(scope="session")
def oracle_lib():
    import oracle
    return oracle.load()
