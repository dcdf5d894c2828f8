"""The oracle's restatement of the token loop's sampling (src/main.rs:
192-305), pinned on the CPU: hand-derived known answers, the inverse CDF of
the truncated distribution in float64, the penalty's sign and once-per-id
rule and its window, the all-below-threshold fallback, the acceptance test
used against the device sampler, and the SplitMix64 stream against its
published vectors."""
from __future__ import annotations

import math

import numpy as np
import pytest

from conftest import sample_u, splitmix64


def test_splitmix64_published_vectors():
    # the first outputs of SplitMix64 seeded with 1234567 (Vigna's splitmix64.c)
    want = [6457827717110365317, 3203168211198807973, 9817491932198370423,
            4593380528125082431, 16408922859458223821]
    assert [splitmix64(1234567, n) for n in range(1, 6)] == want
    u = sample_u(1234567, 0)
    assert u == (6457827717110365317 >> 40) / 2.0 ** 24 and 0.0 <= u < 1.0


def test_known_answers(orc):
    # p = [1/7, 2/7, 4/7]; descending order ids 2, 1, 0
    lg = np.log(np.array([1.0, 2.0, 4.0], np.float32))
    s = lambda u, top_p, **kw: orc.sample(lg, [], kw.get("pen", 1.0), kw.get("t", 1.0), top_p,
                                          kw.get("win", 0), u)[0]
    # top_p 0.5: 4/7 > 0.5 already, only id 2
    assert {s(u, 0.5) for u in (0.0, 0.3, 0.99)} == {2}
    # top_p 0.8: cut after 2 ids (6/7 > 0.8), r = u * 6/7: id 2 while u <= 2/3
    assert s(0.6, 0.8) == 2 and s(0.7, 0.8) == 1 and s(0.999, 0.8) == 1
    # roulette in index order: id 0 while u <= 1/7, id 1 while u <= 3/7
    assert s(0.1, 1.0) == 0 and s(0.2, 1.0) == 1 and s(0.4, 1.0) == 1 and s(0.5, 1.0) == 2
    # top_p 0 keeps the most probable id
    assert s(0.9, 0.0) == 2
    # temperature 0.5 squares the ratios: p = [1, 4, 16] / 21; roulette
    assert s(1 / 21 - 1e-3, 1.0, t=0.5) == 0 and s(1 / 21 + 1e-3, 1.0, t=0.5) == 1
    assert s(5 / 21 + 1e-3, 1.0, t=0.5) == 2


def test_penalty_rules(orc):
    greedy = lambda lg, hist, pen, win=0: orc.sample(np.array(lg, np.float32), hist, pen, 1.0, 0.0, win, 0.5)[0]
    # positive logits divided once per distinct id: 1.0 / 2 = 0.5 > 0.4
    # (twice would give 0.25 < 0.4)
    assert greedy([1.0, 0.4], [0, 0, 0], 2.0) == 0
    assert greedy([1.0, 0.6], [0], 2.0) == 1
    # negative logits multiplied: -1 * 2 = -2 < -1.5
    assert greedy([-1.0, -1.5], [0], 2.0) == 1
    # penalty <= 1 leaves the logits alone
    assert greedy([1.0, 0.6], [0], 1.0) == 0
    assert greedy([1.0, 0.6], [0], 0.5) == 0
    # window: only the last `win` entries count
    assert greedy([1.0, 0.6], [0, 1], 2.0, win=1) == 0  # only id 1 penalised
    assert greedy([1.0, 0.6], [1, 0], 2.0, win=1) == 1  # only id 0 penalised
    assert greedy([1.0, 0.6], [0, 1], 2.0, win=0) == 0  # both: 0.5 > 0.3


def inverse_cdf(lg, hist, pen, t, top_p, win, u):
    """float64 nucleus / roulette draw from the definitions: the id whose
    interval of the walk's running sum holds u * total, and the distance of
    the draw from the interval's ends relative to the total."""
    l = np.array(lg, np.float64)
    if pen > 1.0:
        h = list(hist)[-win:] if 0 < win < len(hist) else list(hist)
        for i in set(h):
            l[i] = l[i] * pen if l[i] < 0 else l[i] / pen
    if abs(t - 1.0) > 1e-6:
        l = l / t
    p = np.exp(l - l.max())
    p /= p.sum()
    if top_p < 1.0:
        idx = np.nonzero(p > 1e-5)[0]
        if idx.size == 0:
            idx = np.arange(p.size)
        order = idx[np.argsort(-p[idx], kind="stable")]
        cs = np.cumsum(p[order])
        cut = int(np.argmax(cs > top_p)) if (cs > top_p).any() else order.size - 1
        order = order[: cut + 1]
    else:
        order = np.arange(p.size)
    cs = np.cumsum(p[order])
    r = u * cs[-1]
    k = min(int(np.searchsorted(cs, r)), order.size - 1)
    lo = cs[k - 1] if k else 0.0
    return int(order[k]), min(r - lo, cs[k] - r) / cs[-1], (abs(cs - top_p).min() if top_p < 1 else 1.0)


@pytest.mark.parametrize("vocab,scale", [(50, 1.0), (50, 4.0), (3000, 2.0), (3000, 6.0)])
def test_inverse_cdf(orc, vocab, scale):
    rng = np.random.default_rng(vocab * 10 + int(scale))
    lg = (rng.standard_normal(vocab) * scale).astype(np.float32)
    hist = rng.integers(0, vocab, 40)
    checked = 0
    for pen, t, top_p, win in [(1.0, 1.0, 1.0, 0), (1.2, 0.8, 0.9, 16), (1.3, 1.5, 0.5, 0), (1.2, 0.8, 1.0, 64)]:
        for u in rng.random(60):
            want, dist, cut_dist = inverse_cdf(lg, hist, pen, t, top_p, win, float(np.float32(u)))
            if dist < 1e-4 or cut_dist < 1e-4:
                continue  # within the reference's f32 rounding of a boundary
            got, ok = orc.sample(lg, hist, pen, t, top_p, win, np.float32(u), want)
            assert got == want and ok, (pen, t, top_p, win, u)
            checked += 1
    assert checked > 150


def test_all_below_threshold_fallback(orc):
    # 200000 equal logits: p = 5e-6 <= 1e-5 everywhere, so every id is a
    # candidate; ties keep index order, the cut ends near 0.5 (the f32
    # running sums of 1e5 terms drift by a few hundredths of a percent)
    lg = np.zeros(200000, np.float32)
    for u in (0.1, 0.5, 0.9):
        got, _ = orc.sample(lg, [], 1.0, 1.0, 0.5, 0, u)
        assert abs(got - u * 100000) < 200, (u, got)
    # with one id above the threshold only that one is a candidate
    lg[123] = 20.0
    assert {orc.sample(lg, [], 1.0, 1.0, 0.5, 0, u)[0] for u in (0.0, 0.5, 0.99)} == {123}


def test_acceptance_is_tight(orc):
    """The check of another implementation's draw takes a neighbour across a
    boundary only when the draw sits on that boundary (a mistake planted in
    the candidate id is caught)."""
    lg = np.log(np.array([1.0, 2.0, 4.0], np.float32))
    # u = 2/3 at top_p 0.8 is the 2 | 1 boundary: both accepted
    u = np.float32(2 / 3)
    tok, _ = orc.sample(lg, [], 1.0, 1.0, 0.8, 0, u)
    assert tok in (1, 2)
    assert orc.sample(lg, [], 1.0, 1.0, 0.8, 0, u, 1)[1] and orc.sample(lg, [], 1.0, 1.0, 0.8, 0, u, 2)[1]
    # away from it, only the right id; never the id outside the cut
    assert orc.sample(lg, [], 1.0, 1.0, 0.8, 0, 0.3, 2)[1]
    assert not orc.sample(lg, [], 1.0, 1.0, 0.8, 0, 0.3, 1)[1]
    assert not orc.sample(lg, [], 1.0, 1.0, 0.8, 0, 0.99, 0)[1]
    # roulette: 0.5 lies inside id 2's interval (3/7, 1]
    assert orc.sample(lg, [], 1.0, 1.0, 1.0, 0, 0.5, 2)[1]
    assert not orc.sample(lg, [], 1.0, 1.0, 1.0, 0, 0.5, 1)[1]
    assert math.isclose(3 / 7, 0.428571, rel_tol=1e-5)
