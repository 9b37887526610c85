import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU (runs through the C ABI)")


def pytest_runtest_logstart(nodeid, location):
    # Name each test on stderr before it runs, so a run that ends abruptly still shows which
    # case was on the GPU.
    if os.environ.get("SMX_TRACE_TESTS"):
        sys.stderr.write(f"[start] {nodeid}\n")
        sys.stderr.flush()
