"""The no-allocation matmul_transposed entry point (llmrs_matmul_transposed_
noalloc) against llmrs_matmul_transposed: equal outputs, bit for bit, on
two calls in a row through the C ABI, the second with a smaller input (the
fixed scratch keeps the first call's contents); sizes beyond the scratch
are rejected; f32 and single-row inputs, which need no scratch, also match.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
F32 = np.float32


def _case(hip, rng, m, n, k, wtype):
    be = hip.HipBackend()
    a = rng.normal(0, 1, (m, k)).astype(F32)
    if wtype == "q8_0":
        qs, sc = hip.synth_q8(20260011, m + n + k, n, k, 2e-4, 3.5e-4)
        w = hip.Tensor.from_q8_0(qs, sc, n, k)
    elif wtype == "f32":
        w = hip.Tensor.from_numpy(rng.uniform(-1, 1, (n, k)).astype(F32))
    else:
        qs, sc = hip.synth_q4(20260012, m + n + k, n, k, 0.003, 0.006)
        w = hip.Tensor.from_q4(qs, sc, n, k)
    ta = hip.Tensor.from_numpy(a)
    want = be.matmul_transposed(ta, w).data()
    out = hip.Tensor.zeros((m, n))
    be.matmul_transposed_noalloc(ta, w, out)
    got = out.data()
    assert got.shape == want.shape
    assert np.array_equal(got, want), f"{int(np.sum(got != want))} of {got.size} outputs differ"


@pytest.mark.parametrize("wtype", ["q4_0", "q8_0"])
def test_noalloc_matches_twice_second_smaller(hip, rng, wtype):
    # 1000 x 4096: 4.6 MiB of codes and scales in the scratch; then 37 rows
    _case(hip, rng, 1000, 4096, 4096, wtype)
    _case(hip, rng, 37, 1000, 1024, wtype)


def test_noalloc_single_row_and_f32(hip, rng):
    _case(hip, rng, 1, 4096, 4096, "q4_0")
    _case(hip, rng, 1, 512, 2048, "q4_0")
    _case(hip, rng, 8, 64, 128, "f32")


def test_noalloc_rejects_beyond_scratch_and_bad_out(hip, rng):
    be = hip.HipBackend()
    k = 8192
    qs, sc = hip.synth_q4(5, 6, 64, k, 0.003, 0.006)
    w = hip.Tensor.from_q4(qs, sc, 64, k)
    m = 2048  # 2048 * 8192 * 1.125 bytes = 18 MiB > 16 MiB
    a = hip.Tensor.from_numpy(np.zeros((m, k), F32))
    with pytest.raises(hip.LlmrsError) as e:
        be.matmul_transposed_noalloc(a, w, hip.Tensor.zeros((m, 64)))
    assert e.value.code == hip.E_RANGE
    with pytest.raises(hip.LlmrsError) as e:
        be.matmul_transposed_noalloc(hip.Tensor.from_numpy(np.zeros((4, k), F32)), w, hip.Tensor.zeros((4, 63)))
    assert e.value.code == hip.E_INVALID
