"""The device sampler (sample.hip) against the oracle's restatement of the
token loop's sampling (src/main.rs:192-305).

Bar: every draw is the oracle's, or lies within the rounding of the
reference's f32 running sums of a boundary (orc_sample's acceptance: the
device sums probabilities exactly in fixed point, the reference in f32 in
walk order); most draws are identical.  U is bit-exact to the SplitMix64
stream.  Model level: each token a sampled generation produced is what the
sampler gives on that step's decode logits (recomputed by an eager step at
the same position), and the oracle accepts it; an end-of-sequence id stops
the run; greedy decoding comes back unchanged afterwards."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import sample_u
from llmrs_hip import DType, LlmrsError, Sampling, sample_logits, synthetic as syn

pytestmark = pytest.mark.gpu

VOCAB = 128256

CASES = [  # (logit scale, temperature, top_p, penalty, window)
    (1.0, 1.0, 1.0, 1.0, 0),     # flat: roulette over all ids
    (1.0, 0.8, 0.9, 1.2, 64),    # the reference's defaults (main.rs:42-58)
    (4.0, 0.8, 0.9, 1.2, 64),
    (4.0, 1.0, 0.5, 1.3, 0),
    (8.0, 1.5, 0.95, 1.2, 16),
    (8.0, 0.7, 1.0, 1.1, 64),    # peaked roulette
    (2.0, 1.0, 0.0, 1.0, 0),     # top_p 0: the most probable id
    (0.05, 1.0, 0.9, 1.0, 0),    # every p below 1e-5: all ids are candidates
]


def check_draws(orc, lg, hist, case, seed, positions):
    scale, t, top_p, pen, win = case
    s = Sampling.make(temperature=t, top_p=top_p, repeat_penalty=pen, penalty_window=win, seed=seed)
    same = 0
    for pos in positions:
        tok, u = sample_logits(lg, hist, s, pos)
        assert u == sample_u(seed, pos), (pos, u)
        want, ok = orc.sample(lg, hist, pen, t, top_p, win, u, tok)
        assert ok, f"case {case} position {pos}: device {tok}, oracle {want}, u {u}"
        same += tok == want
    return same


@pytest.mark.parametrize("case", CASES, ids=lambda c: "s{}-t{}-p{}-r{}-w{}".format(*c))
def test_sampler_vs_oracle(hip, orc, case):
    rng = np.random.default_rng(int(case[0] * 100) + int(case[2] * 10))
    lg = (rng.standard_normal(VOCAB) * case[0]).astype(np.float32)
    hist = rng.integers(0, VOCAB, 300).astype(np.int32)
    hist[-10:] = np.argsort(-lg)[:10]  # penalise some of the most probable ids
    positions = range(0, 400, 5)
    same = check_draws(orc, lg, hist, case, 20260101, positions)
    # over nearly flat distributions the reference's f32 running sums drift
    # across several ids, so fewer draws are identical
    frac = 0.5 if case[0] <= 1.0 else 0.9
    assert same >= frac * len(positions), f"only {same} of {len(positions)} draws identical"


@pytest.mark.parametrize("vocab", [1, 7, 1000, 4097, 262144])
def test_sampler_vocab_sizes(hip, orc, vocab):
    rng = np.random.default_rng(vocab)
    lg = (rng.standard_normal(vocab) * 3).astype(np.float32)
    hist = rng.integers(0, vocab, 50).astype(np.int32)
    for case in [(3.0, 0.8, 0.9, 1.2, 64), (3.0, 1.0, 1.0, 1.0, 0)]:
        check_draws(orc, lg, hist, case, 7, range(0, 60, 3))


@pytest.mark.parametrize("top_p", [0.3, 0.5, 0.95, 1.0])
def test_sampler_ties(hip, orc, top_p):
    # six distinct logits over the whole vocabulary: the cut and the draw
    # land inside groups of ~21000 exactly equal probabilities, taken in
    # index order.  The reference's f32 running sum drifts by hundreds of
    # ids over such a group (each addition of the same small p rounds the
    # same way), so the bar is acceptance alone.
    rng = np.random.default_rng(int(top_p * 100))
    lg = (rng.integers(0, 6, VOCAB) * 0.7).astype(np.float32)
    check_draws(orc, lg, np.zeros(0, np.int32), (1.0, 1.0, top_p, 1.0, 0), 11, range(0, 200, 5))
    # four tied ids far above the rest: the top-p walk over them keeps its
    # f32 sums exact, so every draw is the reference's (the roulette also
    # walks the 4996 small probabilities in index order: nearly every one)
    lg = np.zeros(5000, np.float32)
    lg[[17, 400, 401, 4999]] = 12.0
    positions = range(40)
    same = check_draws(orc, lg, np.zeros(0, np.int32), (1.0, 1.0, top_p, 1.0, 0), 12, positions)
    assert same >= len(positions) - (2 if top_p >= 1.0 else 0)


def test_sampler_history_edges(hip, orc):
    rng = np.random.default_rng(5)
    lg = (rng.standard_normal(5000) * 4).astype(np.float32)
    top = np.argsort(-lg)[:8].astype(np.int32)
    case = (4.0, 1.0, 0.9, 2.0, 4)
    check_draws(orc, lg, np.zeros(0, np.int32), case, 3, range(20))      # empty history
    check_draws(orc, lg, top, case, 3, range(20))                         # window < history
    check_draws(orc, lg, top[:2], case, 3, range(20))                     # window > history
    check_draws(orc, lg, np.array([-5, 5000, 10 ** 6, top[0]], np.int32), case, 3, range(20))  # ids out of range
    check_draws(orc, lg, np.repeat(top[:3], 50), case, 3, range(20))      # repeated ids


def test_sampler_rejects(hip):
    lg = np.zeros(16, np.float32)
    with pytest.raises(LlmrsError):
        sample_logits(lg, [], Sampling.make(temperature=0.0), 0)
    with pytest.raises(LlmrsError):
        sample_logits(lg, [], Sampling.make(top_p=float("nan")), 0)
    with pytest.raises(LlmrsError):
        sample_logits(np.zeros(262145, np.float32), [], Sampling.make(), 0)


SPEC = syn.tiny(DType.Q4_0, DType.F16, head_dim=128, n_heads=8, n_kv_heads=2, ffn=1024, vocab=1000)


def test_sampled_generation(hip, orc, monkeypatch):
    gm = hip.HipModel(SPEC.config(128))
    w = syn.make_weights(SPEC)
    syn.load_model(gm, w)
    prompt = syn.prompt(SPEC)
    greedy = gm.generate(prompt, 48)
    s = Sampling.make(temperature=0.9, top_p=0.9, repeat_penalty=1.2, penalty_window=16, seed=99, eos=())
    gm.set_sampling(s)
    steps = 64
    out = gm.generate(prompt, steps)
    assert out.size == steps and gm.produced() == (steps, False)
    assert np.array_equal(out, gm.generate(prompt, steps)), "a seeded run must repeat"
    seq = np.concatenate([prompt, out]).astype(np.int32)
    n0 = prompt.size
    # each draw against the decode logits of its position (an eager step over
    # the cache the run left, which holds the same rows)
    monkeypatch.setenv("LLMRS_PREFILL", "0")
    same = 0
    for j in range(steps):
        p = n0 - 1 + j
        lg, _, _ = gm.forward(seq[p:p + 1], p)
        hist = seq[:p + 1]
        tok, u = sample_logits(lg, hist, s, p)
        assert tok == out[j], f"step {j}: generation drew {out[j]}, the sampler on its logits {tok}"
        want, ok = orc.sample(lg, hist, s.repeat_penalty, s.temperature, s.top_p, s.penalty_window, u, tok)
        assert ok, f"step {j}: device {tok}, oracle {want}"
        same += tok == want
    assert same >= steps - 3
    assert len(set(out.tolist())) > 8, "sampling should not collapse to a few ids"
    # an end-of-sequence id ends the run before it is appended
    k = next(j for j in range(8, steps) if out[j] not in out[:j])
    gm.set_sampling(Sampling.make(temperature=0.9, top_p=0.9, repeat_penalty=1.2, penalty_window=16, seed=99,
                                  eos=(int(out[k]),)))
    stopped = gm.generate(prompt, steps)
    assert np.array_equal(stopped, out[:k]) and gm.produced() == (k, True)
    # greedy again
    gm.set_sampling(None)
    assert np.array_equal(gm.generate(prompt, 48), greedy)
