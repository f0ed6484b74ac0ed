import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def sampler():
    """The GPU sampler. Fails (does not skip) when the library or GPU is missing.

    torch's HIP runtime (used by the device-buffer tests for allocation) is
    brought up first, as bench.py does: it does not initialize after the
    library's runtime has claimed the device in the same process."""
    import torch

    torch.cuda.init()
    from scriptonait_amd.sampler import Sampler

    s = Sampler(0)
    yield s
    s.close()
