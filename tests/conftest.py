import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
GOLDEN = os.path.join(ROOT, "tests", "golden")
if GOLDEN not in sys.path:
    sys.path.insert(0, GOLDEN)


@pytest.fixture(autouse=True)
def _seed_global_generator():
    """Every test starts from the same state of torch's global CPU generator
    (otherwise seeded per process): default parameter initialisation and
    unseeded draws repeat from run to run."""
    import torch
    torch.manual_seed(0)
    yield


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


def pytest_collection_modifyitems(config, items):
    # GPU tests need the device; on a CPU-only host they are skipped, not failed,
    # when someone runs the whole suite without "-m".
    try:
        import torch
        has_gpu = torch.cuda.is_available()
    except Exception:  # pragma: no cover
        has_gpu = False
    if has_gpu:
        return
    skip = pytest.mark.skip(reason="no ROCm GPU on this host")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
