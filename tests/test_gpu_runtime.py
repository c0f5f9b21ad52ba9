"""The GPU tests run libqne.so on the HIP runtime it links (/opt/rocm), the runtime bench.py and
the product use: no other copy of libamdhip64 (such as the one bundled with torch) is mapped into
the test process."""
import pytest

import devmem as D
import qne as Q

pytestmark = pytest.mark.gpu


def test_only_the_rocm_hip_runtime_is_mapped():
    Q.load_library()
    D.sync()  # the runtime is initialised by now
    hip = [p for p in D.mapped_hip_runtimes() if "libamdhip64" in p]
    assert hip, "no HIP runtime mapped"
    assert all(p.startswith("/opt/rocm") for p in hip), hip
