import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP libraries")
    config.addinivalue_line("markers", "slow: takes more than a few seconds on CPU")


def pytest_collection_modifyitems(config, items):
    # GPU tests run when selected with -m gpu; without a visible GPU they are skipped, never
    # silently passed through some other path.
    try:
        import torch

        has_gpu = torch.cuda.is_available()
    except Exception:
        has_gpu = False
    if has_gpu:
        return
    skip = pytest.mark.skip(reason="needs a GPU (torch.cuda.is_available() is False)")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def oracle_lib():
    from oracle import oracle

    return oracle


@pytest.fixture(autouse=True)
def seeded_torch():
    """Every test starts from the same torch generator state (CPU and GPU), so inputs drawn with
    torch.randn are the same on every run and a tolerance failure reproduces."""
    import torch

    torch.manual_seed(0)
