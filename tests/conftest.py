import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tinyllama.c_amd"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device)")


def _flush_case(item):
    # name the case before any GPU work so a crash still identifies it
    print(f"\n[case] {item.nodeid}", flush=True)


@pytest.hookimpl(tryfirst=True)
def pytest_runtest_setup(item):
    if "gpu" in item.keywords:
        _flush_case(item)
