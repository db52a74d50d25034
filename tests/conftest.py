"""Shared fixtures: the oracle (test infrastructure), the compiled reference
routines when built, and the product package on sys.path."""
from __future__ import annotations

import ctypes
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "citlali-llm-engine_amd")
if PKG not in sys.path:
    sys.path.insert(0, PKG)
for _p in (os.path.join(ROOT, "tests"), os.path.join(ROOT, "oracle")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

from oracle_binding import Oracle, RefLib  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the C ABI on cuda:0)")


@pytest.fixture(scope="session")
def orc() -> Oracle:
    return Oracle()


@pytest.fixture(scope="session")
def ref() -> RefLib:
    r = RefLib.try_load()
    if r is None:
        pytest.skip("oracle/_ref (the compiled reference routines) is not built")
    return r


@pytest.fixture(scope="session")
def synth():
    """Seeded synthetic inputs (host only, no GPU)."""
    from pycitlali import synth as s
    return s


@pytest.fixture(scope="session")
def hip():
    """The product library on a GPU; fails loudly if the build is missing."""
    import pycitlali
    lib = pycitlali.load()
    n = ctypes.c_int(0)
    pycitlali.check(lib.citlali_hip_device_count(ctypes.byref(n)))
    assert n.value >= 1, "no HIP device visible"
    pycitlali.check(lib.citlali_hip_init(0))
    return pycitlali


def tol_ok(got, ref, atol=2e-3, rtol=1e-2):
    """The north-star bar for float results: |got - ref| <= atol + rtol*|ref|."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return np.abs(got - ref) <= atol + rtol * np.abs(ref)
