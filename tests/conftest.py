import os
import sys
from pathlib import Path

import pytest
import torch  # noqa: F401  (first: the HIP runtime libqmm.so binds to is torch's)

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "mlx-runner_amd"
for p in (ROOT, ROOT / "oracle", PKG):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if gpu_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this process")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def oracle():
    import oracle as O

    O.lib()
    return O
