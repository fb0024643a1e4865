"""Shared pytest set-up.

Markers: ``gpu`` tests need an MI355X (run on the GPU box with ``-m gpu``);
everything else runs on the CPU. GPU tests call the HIP library through its
C ABI and compare with the CPU oracle (oracle/), which is the checker only.
"""
from __future__ import annotations

import ctypes as C
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU and the built libgpu_engine.so")


@pytest.fixture(scope="session")
def ora():
    from oracle import oracle as O

    O.lib()
    return O


@pytest.fixture(scope="session")
def lib():
    """The gfx950 library, initialised on device 0. Fails (never skips) when
    the library or the GPU is missing: a GPU test must run the HIP path."""
    from neurogrid_amd import _lib

    L = _lib.load()
    n = C.c_int(0)
    rc = L.cuda_get_device_count(C.byref(n))
    if rc != 0 or n.value < 1:
        pytest.fail("no GPU visible to the HIP runtime; gpu tests need a gfx950 device")
    assert L.cuda_init(0) == 0
    return L
