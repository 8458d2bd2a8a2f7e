"""Shared fixtures.  GPU tests are marked `gpu`; everything else runs on CPU."""
from __future__ import annotations

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import __graft_entry__  # noqa: E402
from oracle import oracle as _oracle  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X)")


@pytest.fixture(scope="session")
def ipus():
    module = __graft_entry__.import_package()
    module.load_library()
    return module


@pytest.fixture(scope="session")
def oracle():
    _oracle.lib()
    return _oracle


@pytest.fixture(scope="session")
def ctx(ipus):
    context = ipus.Context(0)
    yield context
    context.close()


def max_rel(got, want) -> float:
    """Normwise max-rel: max|y - r| / max|r| (the gating error metric)."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    denom = float(np.max(np.abs(want))) if want.size else 1.0
    return float(np.max(np.abs(got - want))) / (denom if denom > 0 else 1.0) if want.size else 0.0


def ref_style_ok(got, want, atol=0.03, rtol=0.03) -> bool:
    """The reference's per-element check |y - r| <= atol + rtol |r| with its
    default atol = rtol = 0.03 (crates/ipu-tests/src/main.rs:47-53)."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    return bool(np.all(np.abs(got - want) <= atol + rtol * np.abs(want)))


def fp16_close(got, want, tol=1e-2) -> bool:
    """fp16 parity: normwise max-rel <= tol (the gating metric) and the
    reference's own per-element tolerance."""
    return max_rel(got, want) <= tol and ref_style_ok(got, want)
