import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if REPO not in sys.path:
    sys.path.insert(0, REPO)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session", autouse=True)
def _built_oracle():
    """Build the CPU oracle if it is not built yet (the HIP library is built by
    __graft_entry__.build() / python -m orinmllm_amd.build beforehand)."""
    from oracle import oracle
    if not os.path.exists(oracle.LIB_PATH):
        oracle.build()
    yield


def pytest_collection_modifyitems(config, items):
    # On a machine without a GPU, skip GPU tests that were selected anyway.
    try:
        import torch
        have_gpu = torch.cuda.is_available()
    except Exception:
        have_gpu = False
    if have_gpu:
        return
    skip = pytest.mark.skip(reason="no GPU on this machine")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
