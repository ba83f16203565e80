import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (run with -m gpu on the MI355X box)")


def _has_gpu() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:  # noqa: BLE001
        return False


def pytest_collection_modifyitems(config, items):
    if _has_gpu():
        return
    skip = pytest.mark.skip(reason="no GPU in this process")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as O
    O.lib()
    return O


@pytest.fixture(scope="session")
def dev():
    import torch
    from lockstep_amd import _capi
    _capi.load()
    torch.cuda.init()
    return torch.device("cuda", 0)


@pytest.fixture(autouse=True)
def _announce(request):
    # name the case before any GPU work so a lost box still identifies it
    if "gpu" in request.node.keywords:
        print(f"\n[gpu-case] {request.node.nodeid}", flush=True)
        sys.stdout.flush()
    yield
    if "gpu" in request.node.keywords and os.environ.get("LSMX_SYNC_EACH", "1") == "1":
        import torch
        torch.cuda.synchronize()
