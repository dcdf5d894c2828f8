"""Pins the oracle's layer / model / token-loop composition on CPU.

Restates the reference's own model tests (src/core/layer.rs:430-489) at model
level and adds invariants of the reference arithmetic:
  * batched prefill == sequential decode, bit for bit;
  * GQA by K/V row duplication (loader.rs:62-98) == true GQA, bit for bit;
  * an independent float64 restatement of the whole model (numpy_ref).
"""
from __future__ import annotations

import numpy as np
import pytest

import numpy_ref as ref
from llmrs_hip import DType, synthetic as syn


def _oracle(orc, spec, max_seq=None):
    w = syn.make_weights(spec)
    m = orc.OracleModel.from_spec(spec, max_seq=max_seq)
    m.load(w)
    return m, w


@pytest.fixture(scope="module")
def tiny_q4(orc):
    spec = syn.tiny(DType.Q4_0, DType.F32, head_dim=64, prompt=6, decode=10)
    return spec, *_oracle(orc, spec)


def test_causality(orc, tiny_q4):
    """layer.rs:430-464: row 0 does not depend on later tokens (bit-exact)."""
    spec, _, w = tiny_q4
    a, _ = _oracle(orc, spec)
    b, _ = _oracle(orc, spec)
    la, ta = a.forward([11, 22], 0, all_rows=True, trace=True)
    lb, tb = b.forward([11, 999], 0, all_rows=True, trace=True)
    assert np.array_equal(la[0], lb[0])
    assert np.array_equal(ta[0], tb[0])
    assert not np.array_equal(la[1], lb[1])


def test_kv_cache_update(orc, tiny_q4):
    """layer.rs:466-489: K at pos 0 after the first call, pos 1 after the second."""
    spec, _, _ = tiny_q4
    m, _ = _oracle(orc, spec)
    m.forward([5], 0)
    k, _ = m.kv_read(0, 0, 0, 2)
    assert np.any(k[0] != 0) and not np.any(k[1] != 0)
    m.forward([6], 1)
    k, _ = m.kv_read(0, 0, 0, 2)
    assert np.any(k[1] != 0)


def test_prefill_equals_sequential_decode(orc, tiny_q4):
    spec, _, _ = tiny_q4
    toks = syn.prompt(spec)
    a, _ = _oracle(orc, spec)
    batched, _ = a.forward(toks, 0)
    b, _ = _oracle(orc, spec)
    for i, t in enumerate(toks):
        seq, _ = b.forward([t], i)
    assert np.array_equal(batched, seq)
    ka, va = a.kv_read(1, 1, 0, len(toks))
    kb, vb = b.kv_read(1, 1, 0, len(toks))
    assert np.array_equal(ka, kb) and np.array_equal(va, vb)


def test_gqa_duplication_equals_true_gqa(orc, tiny_q4):
    """The reference duplicates K/V rows per query head; same logits."""
    spec, m_gqa, w = tiny_q4
    rep = spec.n_heads // spec.n_kv_heads
    hd, H = spec.head_dim, spec.hidden
    from dataclasses import replace
    full = replace(spec, n_kv_heads=spec.n_heads)
    m_full = orc.OracleModel.from_spec(full)
    m_full.set_embedding(w.embed)
    m_full.set_norm(-1, 2, w.final_norm)
    m_full.set_linear_q4(-1, 7, *w.lm_head)
    for l in range(spec.n_layers):
        m_full.set_norm(l, 0, w.norms[l][0])
        m_full.set_norm(l, 1, w.norms[l][1])
        for s, (qs, sc) in w.linears[l].items():
            if s in (1, 2):  # k, v: repeat each KV head's rows n_rep times
                qs2 = qs.reshape(spec.n_kv_heads, hd, H // 2)
                sc2 = sc.reshape(spec.n_kv_heads, hd, H // 32)
                qs = np.repeat(qs2, rep, axis=0).reshape(-1)
                sc = np.repeat(sc2, rep, axis=0).reshape(-1)
            m_full.set_linear_q4(l, s, qs, sc)
    toks = syn.prompt(spec)
    m2, _ = _oracle(orc, spec)
    a, _ = m2.forward(toks, 0)
    b, _ = m_full.forward(toks, 0)
    assert np.array_equal(a, b)


def _deq_weights(spec, w):
    deq = ref.dequant_q8 if spec.weight == DType.Q8_0 else ref.dequant_q4
    names = {0: "q", 1: "k", 2: "v", 3: "o", 4: "gate", 5: "up", 6: "down"}
    layers = []
    for l in range(spec.n_layers):
        d = {"norm0": w.norms[l][0], "norm1": w.norms[l][1]}
        for s, (qs, sc) in w.linears[l].items():
            d[names[s]] = deq(qs, sc, *spec.shape(s))
        layers.append(d)
    n, k = spec.shape(7)
    return {"embed": w.embed, "final_norm": w.final_norm, "lm_head": deq(*w.lm_head, n, k),
            "layers": layers}


@pytest.mark.parametrize("weight,kv,hd", [(DType.Q4_0, DType.F32, 64), (DType.Q8_0, DType.F16, 128)])
def test_model_vs_float64_restatement(orc, weight, kv, hd):
    spec = syn.tiny(weight, kv, head_dim=hd, prompt=5)
    m, w = _oracle(orc, spec)
    toks = syn.prompt(spec)
    got, _ = m.forward(toks, 0)
    dims = (spec.n_layers, spec.hidden, spec.n_heads, spec.n_kv_heads, spec.head_dim, spec.ffn, spec.rms_eps)
    kv_round = (lambda a: a.astype(np.float16).astype(np.float64)) if kv == DType.F16 else None
    want = ref.model_forward64(dims, _deq_weights(spec, w), toks, kv_round)
    scale = np.max(np.abs(want))
    assert np.max(np.abs(got - want)) <= 1e-2 * scale
    assert np.corrcoef(got, want)[0, 1] > 0.9999
    assert int(np.argmax(got)) == int(np.argmax(want)) or np.sort(want)[-1] - np.sort(want)[-2] < 1e-2 * scale


def test_generate_matches_forward_loop(orc, tiny_q4):
    spec, _, _ = tiny_q4
    m, _ = _oracle(orc, spec)
    toks = syn.prompt(spec)
    out, margins = m.generate(toks, 6)
    m2, _ = _oracle(orc, spec)
    ids = list(toks)
    lg, _ = m2.forward(ids, 0)
    for s in range(6):
        t, _ = orc.argmax(lg)
        assert t == out[s]
        ids.append(t)
        lg, _ = m2.forward([t], len(ids) - 1)
    assert np.all(margins >= 0)


def test_arch_switch_is_off_by_default_and_restores(orc, tiny_q4):
    """The aarch64 restatement is test-only: the default (x86) build is
    bit-identical before and after switching, and the aarch64 build moves
    the logits by rounding-level amounts only on this Q4 model."""
    spec, _, w = tiny_q4
    toks = syn.prompt(spec)

    def run(arch):
        orc.set_arch(arch)
        try:
            m = orc.OracleModel.from_spec(spec)
            m.load(w)
            return m.forward(toks, 0)[0]
        finally:
            orc.set_arch(0)

    base = run(0)
    other = run(1)
    assert np.array_equal(base, run(0))
    assert np.max(np.abs(other - base)) < 1e-2


def test_attention_f64_switch_matches_float64_closed_form(orc):
    """orc_set_attn_f64: the attention of given projections with float64
    sums equals a float64 numpy attention on the same rotated query and
    cached rows (to the final f32 rounding); the default f32 path stays
    within f32 rounding of it."""
    spec = syn.tiny(DType.Q4_0, DType.F32, head_dim=64, n_layers=1, n_heads=4, n_kv_heads=2)
    om = orc.OracleModel.from_spec(spec, max_seq=40)
    rng = np.random.default_rng(5)
    hd, nq, nkv, pos = 64, 4, 2, 30
    k = rng.normal(0, 1, (nkv, pos, hd)).astype(np.float32)
    v = rng.normal(0, 1, (nkv, pos, hd)).astype(np.float32)
    for g in range(nkv):
        om.kv_write(0, g, 0, k[g], v[g])
    qkv = rng.normal(0, 1, (nq + 2 * nkv) * hd).astype(np.float32)
    f32 = om.attention(0, qkv, pos)[0]
    orc.set_attn_f64(True)
    try:
        f64 = om.attention(0, qkv, pos)[0]
    finally:
        orc.set_attn_f64(False)
    kc = np.stack([om.kv_read(0, g, 0, pos + 1)[0] for g in range(nkv)]).astype(np.float64)
    vc = np.stack([om.kv_read(0, g, 0, pos + 1)[1] for g in range(nkv)]).astype(np.float64)
    scale = np.float64(np.float32(1.0) / np.sqrt(np.float32(hd)))
    for h in range(nq):
        q = orc.rope_inplace(qkv[h * hd:(h + 1) * hd][None], pos)[0].astype(np.float64)
        s = kc[h // 2] @ q * scale
        p = np.exp(s - s.max())
        want = (p @ vc[h // 2]) / p.sum()
        got = f64[h * hd:(h + 1) * hd]
        assert np.max(np.abs(got - want)) <= 2 * np.spacing(np.abs(want).astype(np.float32)).max()
        assert np.max(np.abs(f32[h * hd:(h + 1) * hd] - want)) < 1e-5
