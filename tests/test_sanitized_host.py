"""The host runtime under AddressSanitizer + UndefinedBehaviorSanitizer (CPU): `make asan` builds
the host sources (index.json / options parsing, validation, ABI guards) with both sanitizers, and
the ABI, format and index-fuzz tests run again in a child process against that build, with GCC's
sanitizer runtimes preloaded. Any report (heap overflow, use after free, undefined behaviour)
aborts the child and fails this test."""
import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "qwen-native-engine_amd"


def gcc_runtime(name):
    p = subprocess.run(["gcc", f"-print-file-name={name}"], capture_output=True, text=True).stdout.strip()
    return p if p and os.path.isabs(p) and os.path.exists(p) else None


def test_host_code_is_clean_under_asan_and_ubsan():
    asan, ubsan = gcc_runtime("libasan.so"), gcc_runtime("libubsan.so")
    if not asan or not ubsan:
        pytest.skip("GCC's sanitizer runtimes are not installed")
    subprocess.run(["make", "-C", str(PKG), "-j8", "asan"], check=True, capture_output=True)
    lib = PKG / "_build" / "asan" / "libqne_asan.so"
    env = dict(os.environ)
    env.update(QNE_LIBRARY=str(lib), LD_PRELOAD=f"{asan}:{ubsan}",
               ASAN_OPTIONS="detect_leaks=0:verify_asan_link_order=0:abort_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    tests = [str(ROOT / "tests" / f) for f in ("test_abi.py", "test_format.py", "test_index_fuzz.py")]
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider", *tests], env=env,
                       capture_output=True, text=True, cwd=str(ROOT), timeout=900)
    out = r.stdout[-4000:] + r.stderr[-4000:]
    assert r.returncode == 0, out
    assert "ERROR: AddressSanitizer" not in out and "runtime error" not in out, out
    assert str(lib) in r.stdout or " passed" in r.stdout
