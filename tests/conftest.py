import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built library")


def pytest_collection_modifyitems(config, items):
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no HIP device visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def golden_dir():
    return GOLDEN


@pytest.fixture(scope="session")
def built_library():
    """The in-tree HIP library; compiled here if a fresh checkout has none."""
    from cachebridge_amd import _lib
    from cachebridge_amd.build import build_library

    if not _lib.LIB_PATH.exists():
        build_library()
    return _lib.LIB_PATH


@pytest.fixture(autouse=True)
def _single_thread_cpu():
    # Oracle arithmetic runs single-threaded so torch's vectorized kernels see
    # whole tensors (bit-stable tables and reductions), as in the reference CI.
    import torch

    prev = torch.get_num_threads()
    torch.set_num_threads(int(os.environ.get("CB_TEST_THREADS", "1")))
    yield
    torch.set_num_threads(prev)
