"""The device exponential (exact_math.h) compiled for the host, against the
host libm's expf over every float bit pattern.

SiLU and softmax in the reference call f32::exp (layer.rs:75-79,
cpu.rs:410-413), glibc's expf on x86-64 Linux.  exact_math.h restates its
double-precision evaluation; the same source is compiled into the gfx950
kernels with contraction off, so equality here over all 2^32 inputs, plus
test_gpu_exact.py's device-vs-host comparison, pins the kernels' exp.
"""
from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent
CSRC = HERE.parent / "llm.rs_amd" / "csrc"


def build_checker(tmp_path: Path) -> Path:
    exe = tmp_path / "expf_check"
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-fopenmp", f"-I{CSRC}", "-o", str(exe),
                    str(HERE / "native" / "expf_check.cpp")], check=True)
    return exe


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
@pytest.mark.timeout(600)
def test_exact_expf_equals_host_expf_everywhere(tmp_path):
    exe = build_checker(tmp_path)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()
    checked, mismatches = int(out[1]), int(out[3])
    # every non-NaN pattern: 2^32 minus the 2 * (2^23 - 1) NaNs
    assert checked == (1 << 32) - 2 * ((1 << 23) - 1)
    assert mismatches == 0, " ".join(out)
