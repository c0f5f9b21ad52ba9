"""work_deadline_s (qwen-native-engine_amd/csrc/hip_util.hpp), the host's deadline for device work of
`units` dependent steps (CPU). The host waits for a decode window, a prompt run through the token
kernel or a chain of batched steps with that deadline (the reference polls its device the same way
with a fixed timeout, kernels/src/lib.rs:399-405), so it must outlast the longest work the engine
accepts even on a device many times slower than measured, and still end a stuck single step within
about half a minute. The function is compiled from the header with g++ into a small driver."""
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "qwen-native-engine_amd" / "csrc"

DRIVER = r"""
#include <cstdio>
#include <cstdlib>
#include "hip_util.hpp"
int main(int argc, char** argv) {
    for (int i = 1; i < argc; i++) std::printf("%.9f\n", qne::work_deadline_s(std::atof(argv[i])));
    return 0;
}
"""

MAX_CONTEXT = 8192   # the largest KV capacity a test model is loaded with (4096 for the benchmark models)
MAX_PHASES = 192     # decode-program phases per token the kernel accepts (kMaxPhases, decode.hpp)
LAYERS = 28          # the 2B-shaped model


@pytest.fixture(scope="module")
def deadline(tmp_path_factory):
    d = tmp_path_factory.mktemp("deadline")
    (d / "main.cpp").write_text(DRIVER)
    exe = d / "deadline"
    r = subprocess.run(["g++", "-std=c++17", "-O1", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include", f"-I{CSRC}",
                        str(d / "main.cpp"), "-o", str(exe)], capture_output=True, text=True)
    if r.returncode != 0:
        pytest.skip("g++ / HIP headers unavailable: " + r.stderr[-300:])

    def f(*units):
        out = subprocess.run([str(exe), *map(str, units)], capture_output=True, text=True, check=True).stdout.split()
        return [float(v) for v in out]

    return f


def test_deadline_outlasts_the_longest_decode_window_and_token_prefill(deadline):
    # a window (or a prompt through the token kernel) over the whole context, every phase at 100 us:
    # about 12 times the ~8 us a phase of the 2B model takes on the critical chain
    units = MAX_CONTEXT * MAX_PHASES
    (d,) = deadline(units)
    assert d > units * 100e-6, (d, units)


def test_deadline_outlasts_the_longest_batched_decode(deadline):
    # BatchDecoder waits with 8 units per layer + 4 per step; a 64-row step of the 2B model takes
    # ~3.4 ms (~15 us per unit): allow 10 times that over every position of the context
    units = MAX_CONTEXT * (8 * LAYERS + 4)
    (d,) = deadline(units)
    assert d > MAX_CONTEXT * 34e-3, (d, units)


def test_a_stuck_single_step_still_errors_within_a_minute(deadline):
    one, none, negative = deadline(MAX_PHASES, 0, -5)
    assert 30.0 <= one < 60.0
    assert none == negative == 30.0  # no work: the fixed floor only


def test_deadline_grows_with_the_work(deadline):
    vals = deadline(0, 1, 1000, 10 ** 6, 10 ** 7)
    assert all(a < b for a, b in zip(vals, vals[1:])), vals
