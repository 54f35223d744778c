"""Shared pytest setup.

Markers: ``gpu`` - needs a real MI355X (HIP device) and the built ``libmpk.so``.
CPU tests never launch a kernel.
"""

from __future__ import annotations

import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if REPO not in sys.path:
    sys.path.insert(0, REPO)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: test needs a HIP GPU (MI355X) and the built libmpk.so")


def _ensure_library_built() -> None:
    from tiktoktechjam2026_amd import build

    if not os.path.exists(build.LIB_PATH):
        build.build(verbose=True)


@pytest.fixture(scope="session")
def hip_device():
    """The GPU device for ``gpu`` tests; fails (not skips) when no GPU is visible."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("gpu test collected but no HIP device is visible")
    _ensure_library_built()
    torch.backends.cuda.matmul.allow_tf32 = False
    torch.backends.cudnn.allow_tf32 = False
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def built_library():
    _ensure_library_built()
    from tiktoktechjam2026_amd import _lib

    return _lib.load()
