"""Shared test setup: import paths, the `gpu` marker, common fixtures."""
from __future__ import annotations

import os
import sys
from pathlib import Path

import numpy as np
import pytest

REPO = Path(__file__).resolve().parent.parent
PKG = REPO / "llm.rs_amd"
for p in (str(REPO), str(PKG)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def orc():
    import oracle
    oracle.lib()
    # the GPU hosts give one GPU's job 16 cores, whatever os.cpu_count() says
    oracle.set_threads(int(os.environ.get("ORACLE_THREADS", str(min(16, os.cpu_count() or 1)))))
    return oracle


@pytest.fixture(scope="session")
def hip():
    """The GPU backend, initialised once per session (gpu tests only)."""
    import llmrs_hip
    llmrs_hip.init(0)
    return llmrs_hip


@pytest.fixture
def rng():
    return np.random.default_rng(20260000)


def rel_close(got, want, rtol=1e-3, atol=1e-4):
    """Per-kernel parity bar: |got - want| <= atol + rtol * |want| elementwise."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    err = np.abs(got - want)
    lim = atol + rtol * np.abs(want)
    bad = err > lim
    return (not bad.any()), (float(err.max()) if err.size else 0.0), int(bad.sum())
