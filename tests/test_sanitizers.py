"""The host-only code under the compilers' sanitizers, on the CPU: the engine's thread pool
(engine/src/parallel.cpp) under ThreadSanitizer and under AddressSanitizer +
UndefinedBehaviorSanitizer, the CPU oracle (oracle/oracle.cpp) under AddressSanitizer +
UndefinedBehaviorSanitizer, each driven by a program in tests/sanitize/ (recipe:
tests/sanitize/Makefile). A sanitizer report fails the run."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
MAKEFILE_DIR = os.path.join(HERE, "sanitize")


@pytest.mark.slow
def test_host_code_under_sanitizers():
    if shutil.which("g++") is None:
        pytest.skip("no g++")
    r = subprocess.run(["make", "-C", MAKEFILE_DIR, "run", "-j3"], capture_output=True, text=True,
                       timeout=600)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-4000:]
    for what in ("pool_driver: ok", "oracle_driver: ok"):
        assert what in out, out[-2000:]
    assert "WARNING: ThreadSanitizer" not in out and "ERROR: AddressSanitizer" not in out
