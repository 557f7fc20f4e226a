import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

# bf16-level tolerance of attention outputs against the float64 oracle
ATTN_MAX_ABS = 2e-2
ATTN_MEAN_ABS = 2e-3


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (run on the GPU box)")


def gpu_available() -> bool:
    import torch

    return torch.cuda.is_available()


@pytest.fixture(scope="session")
def device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def lib():
    from nanochat_amd.native import LIBRARY, hip_library

    if not LIBRARY.exists():
        pytest.fail(f"{LIBRARY} is not built: run python -m nanochat_amd.native (or __graft_entry__.build())")
    return hip_library()
