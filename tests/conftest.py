"""pytest configuration: the `gpu` marker and import paths for the package and oracle."""
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
for p in (REPO / "mbr-cuda-tile_amd", REPO / "oracle", REPO / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X / gfx950) and the built libmbrt.so")


@pytest.fixture(scope="session")
def orc():
    import oracle

    if not oracle.LIB.exists():
        oracle.build()
    return oracle


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")
