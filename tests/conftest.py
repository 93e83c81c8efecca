"""Shared test configuration.

``gpu`` tests need a real MI355X and the built ``libyufhip.so``; everything
else runs on the CPU (oracle checks, host logic, ABI symbol checks).
"""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


@pytest.fixture(scope="session")
def golden_dir():
    return GOLDEN


@pytest.fixture
def wkv_kernel(request, monkeypatch):
    """Force the per-token VALU WKV-7 kernel ("serial") or the chunked MFMA one
    ("chunked"); the library reads YUF_WKV7_KERNEL at each launch."""
    monkeypatch.setenv("YUF_WKV7_KERNEL", request.param)
    return request.param
