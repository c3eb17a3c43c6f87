import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line('markers', 'gpu: needs a ROCm GPU (MI355X) and the built libegpt_hip.so')


def pytest_collection_modifyitems(config, items):
    import torch
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason='no ROCm GPU visible')
    for item in items:
        if 'gpu' in item.keywords:
            item.add_marker(skip)


@pytest.fixture(autouse=True)
def _announce(request):
    """Name each GPU test on stdout before it runs, so a run that dies mid-test says which one."""
    if 'gpu' in request.keywords:
        print(f'\n[gpu-test] {request.node.nodeid}', flush=True)
    yield


def pytest_sessionstart(session):
    os.environ.setdefault('HSA_ENABLE_IPC_MODE_LEGACY', '0')
