import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = Path(__file__).resolve().parent / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")
    config.addinivalue_line("markers", "slow: long-running CPU test")


def pytest_collection_modifyitems(config, items):
    gpu_items = [i for i in items if "gpu" in i.keywords]
    if not gpu_items:
        return
    try:
        import torch

        ok = torch.cuda.is_available()
    except Exception:  # pragma: no cover
        ok = False
    if not ok:
        skip = pytest.mark.skip(reason="no GPU visible")
        for item in gpu_items:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def golden():
    return GOLDEN


@pytest.fixture(scope="session")
def oracle_lib():
    import oracle

    oracle.lib()
    return oracle
