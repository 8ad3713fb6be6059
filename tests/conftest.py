import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = Path(__file__).resolve().parent / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libwkv.so")
    config.addinivalue_line("markers", "slow: long-running")


@pytest.fixture(scope="session")
def golden_dir() -> Path:
    return GOLDEN


@pytest.fixture(scope="session")
def cuda():
    """The GPU device for `gpu` tests; fails loudly (no silent skip) without one."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("gpu test collected on a host without a visible GPU")
    from wavelet_amd import _lib

    _lib.load()  # the HIP library must be there: no fallback path exists
    os.environ.setdefault("HIP_LAUNCH_BLOCKING", "0")
    return torch.device("cuda", 0)
