"""Batched decode (llmrs_batch_*): B sequences of one model decoding together.

The reference decodes one sequence; a row's values in its layer code depend
only on that row and its own cache (layer.rs:175-333).  Bars: each slot's
logits within 1e-2 of the oracle's forward over that slot's sequence and its
greedy stream identical to the oracle's for the first 64 steps (a slot whose
stream parts earlier at a near-tie makes the test an expected failure that
names it; parting anywhere else fails); a slot's logits bit-identical
whichever other sequences share the batch; every slot at its own position."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import NEAR_TIE, check_stream
from llmrs_hip import DType, HipBatch, synthetic as syn

pytestmark = pytest.mark.gpu

SPECS = [
    syn.tiny(DType.Q4_0, DType.F16, head_dim=128, n_heads=8, n_kv_heads=2, ffn=1024, seed=21),
    syn.tiny(DType.Q8_0, DType.F32, head_dim=64, n_heads=4, n_kv_heads=2, ffn=512, seed=22),
    syn.tiny(DType.Q4, DType.F16, head_dim=64, n_heads=8, n_kv_heads=1, ffn=512, seed=23),
]


def prompts(spec, B, seed=5):
    rng = np.random.default_rng(seed)
    return [rng.integers(0, spec.vocab, int(rng.integers(1, 20))).astype(np.int32) for _ in range(B)]


@pytest.mark.parametrize("mode", ["gemv", "skinny", "prefill"])
@pytest.mark.parametrize("spec", SPECS, ids=lambda s: s.name)
def test_batch_streams_vs_oracle(hip, orc, spec, mode, monkeypatch):
    """The three linear-layer paths: the row-batched decode GEMV (the
    default up to 4 sequences), the skinny GEMM (up to 64) and the prefill
    GEMM."""
    monkeypatch.setenv("LLMRS_BATCH_GEMM", mode)
    w = syn.make_weights(spec)
    gm = hip.HipModel(spec.config(128))
    syn.load_model(gm, w)
    om = orc.OracleModel.from_spec(spec, max_seq=128)
    om.load(w)
    B, steps = 5, 72
    ps = prompts(spec, B)
    bt = HipBatch(gm, B)
    for s, p in enumerate(ps):
        bt.begin(s, p)
    bt.decode_steps(steps - 1)
    lg = bt.logits()
    early = []
    for s, p in enumerate(ps):
        toks = bt.tokens(s, p.size + steps)
        assert np.array_equal(toks[:p.size], p)
        gen = toks[p.size:]
        ref, margins = om.generate(p, steps)
        # the last step's logits against the oracle's forward over the same sequence
        olg, _ = om.forward(toks[:-1], 0)
        assert np.max(np.abs(lg[s] - olg)) < 1e-2, f"slot {s}"
        mism = np.nonzero(gen != ref)[0]
        if mism.size and mism[0] < 64 and margins[mism[0]] < NEAR_TIE:
            early.append(f"slot {s} at step {mism[0]} (oracle margin {margins[mism[0]]:.2g})")
        else:
            check_stream(gen, ref, margins)
    bt.close()
    gm.close()
    if early:
        # measured on MI355X: tiny-Q8_0-F32 (all three paths) parts at step 36
        # (margin 0.002), tiny-Q4-F16 on the skinny GEMM at step 22 (0.0017)
        pytest.xfail("fast kernels: greedy stream parts from the oracle before step 64 at a near-tie: "
                     + "; ".join(early))


def test_batch_rows_independent(hip, orc):
    spec = SPECS[0]
    w = syn.make_weights(spec)
    gm = hip.HipModel(spec.config(96))
    syn.load_model(gm, w)
    ps = prompts(spec, 4, seed=9)
    out = {}
    for B in (4, 1):
        bt = HipBatch(gm, B)
        for s in range(B):
            bt.begin(s, ps[s])
        bt.decode_steps(20)
        out[B] = (bt.logits(), [bt.tokens(s, ps[s].size + 21) for s in range(B)])
        bt.close()
    assert np.array_equal(out[4][0][0], out[1][0][0]), "slot 0's logits depend on the other slots"
    assert np.array_equal(out[4][1][0], out[1][1][0])
    # a slot restarted with another prompt keeps the others unchanged
    bt = HipBatch(gm, 2)
    bt.begin(0, ps[0])
    bt.begin(1, ps[1])
    bt.decode_steps(5)
    a = bt.tokens(0, ps[0].size + 6)
    bt.begin(1, ps[2])
    bt.decode_steps(5)
    b0 = bt.tokens(0, ps[0].size + 11)
    assert np.array_equal(b0[:a.size], a)
    assert np.array_equal(b0, out[4][1][0][:b0.size])
    bt.close()
    gm.close()


@pytest.mark.parametrize("kv", [DType.F16, DType.F32], ids=["f16", "f32"])
def test_batch_xcd_local(hip, kv, monkeypatch):
    """LLMRS_ATTN_LOCAL=1 gives the batch bit-identical logits and streams."""
    spec = syn.tiny(DType.Q4_0, kv, head_dim=64, n_heads=16, n_kv_heads=8, ffn=512, seed=24)
    w = syn.make_weights(spec)
    ps = prompts(spec, 3, seed=11)
    out = {}
    for mode in ("0", "1"):
        monkeypatch.setenv("LLMRS_ATTN_LOCAL", mode)
        gm = hip.HipModel(spec.config(128))
        syn.load_model(gm, w)
        bt = HipBatch(gm, 3)
        for s, p in enumerate(ps):
            bt.begin(s, p)
        bt.decode_steps(40)
        out[mode] = (bt.logits(), [bt.tokens(s, p.size + 41) for s, p in enumerate(ps)])
        bt.close()
        gm.close()
    assert np.array_equal(out["0"][0], out["1"][0])
    for a, b in zip(out["0"][1], out["1"][1]):
        assert np.array_equal(a, b)


def test_batch_errors(hip):
    spec = SPECS[1]
    gm = hip.HipModel(spec.config(32))
    syn.load_model(gm, syn.make_weights(spec))
    bt = HipBatch(gm, 2)
    with pytest.raises(hip.LlmrsError):
        bt.decode_steps(1)  # slots not begun
    bt.begin(0, [1, 2, 3])
    bt.begin(1, [4])
    with pytest.raises(hip.LlmrsError):
        bt.begin(2, [1])
    with pytest.raises(hip.LlmrsError):
        bt.decode_steps(40)  # beyond max_seq
    bt.decode_steps(3)
    with pytest.raises(hip.LlmrsError):
        bt.tokens(0, 3 + 5)  # more than produced
    bt.close()
    with pytest.raises(hip.LlmrsError):
        HipBatch(gm, 0)
    gm.close()


@pytest.mark.timeout(900)
@pytest.mark.parametrize("B", [16, 64])
def test_batch_8b_widths(hip, orc, B):
    """Two 8B-width layers with the full 128256-row lm_head, B sequences of
    1-20 prompt tokens decoding 16 greedy steps on the skinny GEMM (its
    8B-width launches, the ones the benchmark times): every slot's stream
    identical to the oracle's for all 16 steps and its last logits within
    1e-2."""
    spec = syn.with_sizes(syn.WORKLOADS[2], n_layers=2)
    steps = 16
    w = syn.make_weights(spec)
    gm = hip.HipModel(spec.config(64))
    syn.load_model(gm, w)
    om = orc.OracleModel.from_spec(spec, max_seq=64)
    om.load(w)
    ps = prompts(spec, B, seed=B)
    bt = HipBatch(gm, B)
    for s, p in enumerate(ps):
        bt.begin(s, p)
    bt.decode_steps(steps - 1)
    lg = bt.logits()
    worst = 0.0
    for s, p in enumerate(ps):
        toks = bt.tokens(s, p.size + steps)
        ref, margins = om.generate(p, steps)
        check_stream(toks[p.size:], ref, margins, min_steps=steps)
        olg, _ = om.forward(toks[:-1], 0)
        worst = max(worst, float(np.max(np.abs(lg[s] - olg))))
    print(f"\nRAW batch of {B} at 8B widths: {steps}/{steps} identical steps in every slot; "
          f"last logits max-abs error {worst:.3g}", flush=True)
    assert worst < 1e-2
    bt.close()
    gm.close()


def test_model_free_refused_while_a_batch_lives(hip):
    """A batch holds its model's weights: freeing the model first is
    refused (LLMRS_E_INVALID) and works once the batch is freed."""
    spec = SPECS[0]
    gm = hip.HipModel(spec.config(32))
    syn.load_model(gm, syn.make_weights(spec))
    bt = HipBatch(gm, 2)
    with pytest.raises(hip.LlmrsError) as e:
        gm.close()
    assert e.value.code == hip.E_INVALID and "batch" in str(e.value)
    bt.close()
    gm.close()
