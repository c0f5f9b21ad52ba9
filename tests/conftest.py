import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "qwen-native-engine_amd"
for p in (str(PKG), str(ROOT / "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs on the GPU box)")


_torch_ready = False


def pytest_runtest_setup(item):
    """torch carries its own HIP runtime; GPU tests hand torch device buffers to libqne, which works
    when torch's runtime is initialised before libqne's first HIP call."""
    global _torch_ready
    if not _torch_ready and "gpu" in item.keywords:
        import torch
        torch.cuda.init()
        _torch_ready = True


@pytest.fixture(scope="session")
def qne():
    import qne as m
    m.load_library()
    return m


@pytest.fixture(scope="session")
def oracle():
    import cpu_oracle as o
    return o
