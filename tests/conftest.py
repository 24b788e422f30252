import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "cpp-ai-engine_amd")
TESTS = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, PKG, TESTS):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device")
    config.addinivalue_line("markers", "slow: takes more than a few seconds on the CPU")


def print_case(*parts):
    """Names the case before a GPU step, flushed, so a fault still says which one ran."""
    print("CASE:", *parts, flush=True)
