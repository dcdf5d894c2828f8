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


# The greedy-stream bar: the GPU's stream equals the oracle's for the first
# min(min_steps, length) steps (the parity bar's 64 identical steps), with no
# allowance; after that it may only part at a step whose oracle top1-top2
# logit margin is below NEAR_TIE (a near-tie that f32 summation-order
# differences can flip).
NEAR_TIE = 2e-3


def check_stream(gpu, ref, margins, min_steps=64):
    """Steps on which the streams agree; asserts the bar above."""
    gpu, ref = np.asarray(gpu), np.asarray(ref)
    mism = np.nonzero(gpu != ref)[0]
    if mism.size == 0:
        return len(ref)
    i = int(mism[0])
    around = f"gpu {gpu[max(0, i - 2):i + 3]} oracle {ref[max(0, i - 2):i + 3]}"
    assert i >= min(min_steps, len(ref)), (
        f"greedy stream diverged at step {i}, before step {min(min_steps, len(ref))} "
        f"(oracle margin {margins[i]:.4g}): {around}")
    assert margins[i] < NEAR_TIE, f"greedy stream diverged at step {i} with oracle margin {margins[i]:.4g}: {around}"
    return i


_M64 = (1 << 64) - 1


def splitmix64(seed: int, n: int) -> int:
    """Output n (1-based) of the SplitMix64 stream seeded with `seed`."""
    z = (seed + n * 0x9E3779B97F4A7C15) & _M64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & _M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & _M64
    return z ^ (z >> 31)


def sample_u(seed: int, pos: int) -> float:
    """The draw after the token at position `pos`: 24 bits of output pos+1."""
    return float(np.float32((splitmix64(seed, pos + 1) >> 40) / float(1 << 24)))
