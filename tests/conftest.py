import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "qwen-native-engine_amd"
for p in (str(PKG), str(ROOT / "oracle"), str(Path(__file__).resolve().parent)):
    if p not in sys.path:
        sys.path.insert(0, p)

# libqne.so is loaded before any test module is imported, so that it binds the HIP runtime it was
# linked against (/opt/rocm's libamdhip64.so.7) and every GPU test runs on the product's runtime.
# torch carries a second copy of that runtime; GPU tests do not import torch (their device buffers
# come from tests/devmem.py, which calls the runtime libqne bound).
import qne as _qne  # noqa: E402

try:
    _qne.load_library()
except _qne.QneError:
    pass  # not built: the tests that need it fail with the library's own message


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs on the GPU box)")


def _gpu_only(config) -> bool:
    return (config.getoption("markexpr", "") or "").strip() == "gpu"


def pytest_ignore_collect(collection_path, config):
    """Under -m gpu, files without GPU tests are not imported at all (their tests would be
    deselected anyway, and some of them import torch for their CPU references)."""
    p = Path(str(collection_path))
    if _gpu_only(config) and p.is_file() and p.suffix == ".py" and p.name.startswith("test_"):
        return "pytest.mark.gpu" not in p.read_text(encoding="utf-8")
    return None


def pytest_report_header(config):
    import devmem
    maps = devmem.mapped_hip_runtimes()
    return ["HIP runtime mapped with libqne: " + (", ".join(maps) if maps else "(none)")]


def pytest_sessionfinish(session, exitstatus):
    import devmem
    maps = devmem.mapped_hip_runtimes()
    tr = session.config.pluginmanager.get_plugin("terminalreporter")
    if tr is not None:
        tr.write_line("HIP runtime mapped at the end of the session: " + (", ".join(maps) if maps else "(none)"))


@pytest.fixture(scope="session")
def qne():
    _qne.load_library()
    return _qne


@pytest.fixture(scope="session")
def oracle():
    import cpu_oracle as o
    return o
