"""C ABI checks that need no GPU: the library loads, exports every function
declared in include/llmrs_hip.h, rejects bad calls with error codes, and the
seeded synthetic generator is deterministic with the stated distributions."""
from __future__ import annotations

import ctypes as C
import re
from pathlib import Path

import numpy as np
import pytest

import llmrs_hip as lh

HEADER = Path(__file__).resolve().parent.parent / "include" / "llmrs_hip.h"


def declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\*?(llmrs_\w+)\s*\(", text, re.M)))


def test_every_declared_symbol_is_exported():
    names = declared()
    assert len(names) >= 40
    so = C.CDLL(str(lh.LIB_PATH))
    for n in names:
        assert hasattr(so, n), n
    assert set(names) == set(lh.EXPORTED)


def test_device_and_name():
    assert lh.lib().llmrs_device() == lh.Device.Hip
    assert lh.lib().llmrs_name() == b"Hip"


def test_calls_before_init_fail_cleanly():
    rc = lh.lib().llmrs_sync()
    if rc == 0:
        pytest.skip("a context is already initialised in this process")
    assert rc == lh.E_NOINIT
    assert b"llmrs_init" in lh.lib().llmrs_last_error()


def test_bad_device_is_an_error():
    rc = lh.lib().llmrs_init(99, None)
    assert rc < 0
    assert lh.lib().llmrs_last_error()


def test_synth_q4_deterministic_and_uniform():
    a_qs, a_sc = lh.synth_q4(20260002, 21, 64, 4096, 0.003, 0.006, threads=3)
    b_qs, b_sc = lh.synth_q4(20260002, 21, 64, 4096, 0.003, 0.006, threads=1)
    assert np.array_equal(a_qs, b_qs) and np.array_equal(a_sc, b_sc)
    codes = np.concatenate([a_qs & 15, a_qs >> 4])
    hist = np.bincount(codes, minlength=16) / codes.size
    assert np.all(np.abs(hist - 1 / 16) < 0.005)
    assert a_sc.min() >= 0.003 - 1e-6 and a_sc.max() <= 0.006 + 1e-6
    # fp16-exact scales
    assert np.array_equal(a_sc.astype(np.float16).astype(np.float32), a_sc)
    c_qs, _ = lh.synth_q4(20260002, 22, 64, 4096, 0.003, 0.006)
    assert not np.array_equal(a_qs, c_qs)


def test_synth_q8_range():
    qs, sc = lh.synth_q8(20260001, 5, 32, 2048, 2e-4, 3.5e-4)
    assert qs.min() == -127 and qs.max() == 127
    assert abs(qs.astype(np.float64).mean()) < 0.5
    assert sc.min() >= 2e-4 - 1e-7 and sc.max() <= 3.5e-4 + 1e-7
    assert np.array_equal(sc.astype(np.float16).astype(np.float32), sc)


def test_synth_normal_and_tokens():
    x = lh.synth_normal(1, 2, 200001, 1.0, 0.02)
    assert abs(x.mean() - 1.0) < 1e-3 and abs(x.std() - 0.02) < 1e-3
    t = lh.synth_tokens(20260002, 3, 512, 128256)
    assert t.min() >= 0 and t.max() < 128256 and len(set(t.tolist())) > 500
    assert np.array_equal(t, lh.synth_tokens(20260002, 3, 512, 128256))


@pytest.mark.parametrize("field,value", [
    ("max_seq", 1 << 20),   # 8 KV heads x 2^20 positions x 128 x 2 B: a 2 GiB K cache per layer
    ("head_dim", 96),
    ("n_kv_heads", 3),      # 8 query heads over 3 KV heads
])
def test_model_config_rejected_before_any_device_call(field, value):
    """llmrs_model_create validates the configuration before touching a
    device, so bad shapes fail with LLMRS_E_INVALID here, without a GPU."""
    from llmrs_hip import DType, synthetic as syn
    cfg = syn.tiny(DType.Q4_0, DType.F16, head_dim=128, n_heads=8, n_kv_heads=8).config(4096)
    setattr(cfg, field, value)
    h = C.c_void_p()
    rc = lh.lib().llmrs_model_create(C.byref(cfg), C.byref(h))
    assert rc == lh.E_INVALID, (rc, lh.lib().llmrs_last_error())
    assert not h.value
