"""The reference-order decode step (llmrs_model_set_exact) against the CPU
oracle, bit for bit.

The oracle restates the reference's x86-64 build, whose f32 sum orders these
kernels follow (exact.hip).  Bars, none with a tolerance:

* the device exponential equals the host libm's expf on every input tried;
* every intermediate of a decoder layer - RMSNorm codes and scales, Q|K|V
  rows, ctx and its codes, the appended K/V rows, O + residual, the SwiGLU
  product and its codes, down + residual - equals the oracle's on the same
  inputs;
* model runs: the residual stream entering every layer, the final logits
  and the greedy stream equal the oracle's, every step (no near-tie
  allowance).  The parity bar (logits within 1e-2, 64 identical
  greedy steps) is asserted on its own besides, on the 1B Q4_0, 1B Q8_0,
  8B and 70B-width workloads.
"""
from __future__ import annotations

import numpy as np
import pytest

from llmrs_hip import DType, W_DOWN, W_GATE, W_K, W_O, W_Q, W_UP, W_V, synthetic as syn
from llmrs_hip import synth_normal
from test_gpu_kernels import fill_cache, gemv, layer_models

pytestmark = pytest.mark.gpu
F32 = np.float32


def same(got, want, what):
    got, want = np.asarray(got), np.asarray(want)
    assert got.shape == want.shape, f"{what}: shape {got.shape} vs {want.shape}"
    if got.dtype == F32:
        # bit patterns, except that +0 and -0 compare equal (the reference's
        # f32 sums start from +0, the order of two zero terms is not pinned)
        diff = (got.view(np.int32) != want.view(np.int32)) & ~((got == 0) & (want == 0))
    else:
        diff = got != want
    n = int(np.count_nonzero(diff))
    if n:
        i = int(np.flatnonzero(diff)[0])
        raise AssertionError(f"{what}: {n} of {got.size} values differ, first at {i}: "
                             f"{got.ravel()[i]!r} vs {want.ravel()[i]!r}")


def test_device_expf_is_glibc(hip, orc):
    """The exponential of the SiLU and softmax kernels against the host
    libm's expf: every 257th float bit pattern (all exponents, both signs,
    the overflow and underflow edges), a dense walk over the softmax range
    [-104, 0] and special values."""
    pats = np.arange(0, 1 << 32, 257, dtype=np.uint64).astype(np.uint32)
    dense = np.arange(0x80000000, 0xC2D00000, 61, dtype=np.uint64).astype(np.uint32)  # -0 .. -104
    x = np.concatenate([pats, dense]).view(F32)
    special = np.array([0.0, -0.0, np.inf, -np.inf, 88.0, 88.72283, 88.72284, -87.33655, -103.27893,
                        -103.972084, -103.97208, 1e-30, -1e-30, 0.5, -0.5, 1.0, -1.0], F32)
    x = np.concatenate([x[~np.isnan(x)], special])
    same(hip.probe_expf(x), orc.expf(x), "expf")


def check_exact_layer(hip, orc, spec, pos, steps=2):
    """One decoder layer at `pos` (cache below it N(0,1)) in the exact
    mode, `steps` positions in a row: every intermediate equals the
    oracle's reference arithmetic on the same inputs."""
    gm, om, w = layer_models(hip, orc, spec, pos + steps)
    gm.set_exact(True)
    assert gm.decode_plan()["exact"]
    if pos:
        fill_cache(gm, om, spec, pos)
    L, (n_in, n_post) = w.linears[0], w.norms[0]
    eps = spec.rms_eps
    for i in range(steps):
        p = pos + i
        x = synth_normal(spec.seed, 70 + i, spec.hidden, 0.0, 1.0)
        pr = gm.probe_decode_layer(0, p, x)
        oq, od = orc.quantize_row_q8_0(orc.rms_norm(x[None], n_in, eps)[0])
        same(pr["xq"], oq, "input RMSNorm codes")
        same(pr["xd"], od, "input RMSNorm scales")
        qkv = np.concatenate([gemv(orc, spec, oq, od, L[s])[0] for s in (W_Q, W_K, W_V)])
        same(pr["qkv"], qkv, "Q|K|V rows")
        ctx = om.attention(0, qkv, p)[0]
        same(pr["ctx"], ctx, "attention ctx")
        cq, cd = orc.quantize_row_q8_0(ctx)
        same(pr["ctx_q"], cq, "ctx codes")
        same(pr["ctx_d"], cd, "ctx scales")
        for g in range(spec.n_kv_heads):
            for a, b in zip(gm.kv_read(0, g, p, 1), om.kv_read(0, g, p, 1)):
                same(a, b, f"appended K/V row of KV head {g}")
        h = orc.add_assign(gemv(orc, spec, cq, cd, L[W_O])[0], x)
        same(pr["h"], h, "O + residual")
        hq, hd = orc.quantize_row_q8_0(orc.rms_norm(h[None], n_post, eps)[0])
        same(pr["hq"], hq, "post-attention RMSNorm codes")
        same(pr["hd"], hd, "post-attention RMSNorm scales")
        m = orc.silu_mul(gemv(orc, spec, hq, hd, L[W_GATE])[0], gemv(orc, spec, hq, hd, L[W_UP])[0])
        same(pr["m"], m, "SwiGLU product")
        mq, md = orc.quantize_row_q8_0(m)
        same(pr["m_q"], mq, "SwiGLU codes")
        same(pr["m_d"], md, "SwiGLU scales")
        same(pr["out"], orc.add_assign(gemv(orc, spec, mq, md, L[W_DOWN])[0], h), "down + residual")
    # the head: final RMSNorm codes and the lm_head logits and argmax
    x = synth_normal(spec.seed, 99, spec.hidden, 0.0, 1.0)
    xq, xd, lg, nxt = gm.probe_head(x)
    oq, od = orc.quantize_row_q8_0(orc.rms_norm(x[None], w.final_norm, eps)[0])
    same(xq, oq, "final RMSNorm codes")
    same(xd, od, "final RMSNorm scales")
    olg = gemv(orc, spec, oq, od, w.lm_head)[0]
    same(lg, olg, "logits")
    assert nxt == orc.argmax(olg)[0]
    gm.close()


LAYERS = [
    (syn.tiny(DType.Q4_0, DType.F32, head_dim=64), 0),
    (syn.tiny(DType.Q4_0, DType.F16, head_dim=128, n_heads=8, n_kv_heads=2, ffn=1024), 37),
    (syn.tiny(DType.Q8_0, DType.F16, head_dim=64, n_heads=8, n_kv_heads=1), 300),
    (syn.tiny(DType.Q8_0, DType.F32, head_dim=128, n_heads=8, n_kv_heads=8), 9),
    (syn.tiny(DType.Q4, DType.F16, head_dim=128, n_heads=16, n_kv_heads=2, ffn=1024, seed=11), 70),
    # the 1B (Q8_0, f16) and 8B widths with their contexts
    (syn.tiny(DType.Q8_0, DType.F16, head_dim=64, n_layers=1, n_heads=32, n_kv_heads=8, ffn=8192,
              vocab=4096, seed=20260001), 159),
    (syn.tiny(DType.Q4_0, DType.F16, head_dim=128, n_layers=1, n_heads=32, n_kv_heads=8, ffn=14336,
              vocab=4096, seed=20260002), 700),
]


@pytest.mark.parametrize("spec,pos", LAYERS, ids=lambda v: getattr(v, "name", str(v)))
def test_exact_layer_kernels(hip, orc, spec, pos):
    check_exact_layer(hip, orc, spec, pos)


@pytest.mark.parametrize("spec", [LAYERS[0][0], LAYERS[5][0], LAYERS[6][0]], ids=lambda s: s.name)
def test_exact_norm_fold_rows(hip, orc, spec):
    """The exact RMSNorm folds its sum of squares by chunks, each from a
    window of start values around the exact sum before it, and folds a
    chunk in order when the sequential total falls outside the window.  Rows
    whose sequential fold drifts far from the exact sum (equal squares, a
    heavy tail, a sparse row, sums that overflow to infinity) take that
    fallback; on every row the final RMSNorm's codes and scales and the
    logits equal the oracle's sequential arithmetic."""
    gm, om, w = layer_models(hip, orc, spec, 4)
    gm.set_exact(True)
    n, eps = spec.hidden, spec.rms_eps
    rng = np.random.default_rng(20261202)
    g = rng.standard_normal(n)
    sparse = np.zeros(n)
    sparse[::7] = 1.5
    rows = {
        "normal": g,
        "constant 0.3": np.full(n, 0.3),
        "constant 1": np.ones(n),
        "heavy tail": g * rng.exponential(1.0, n) ** 3,
        "sparse": sparse,
        "one outlier": np.where(np.arange(n) == n // 3, 4.0e3, g),
        "overflow": np.full(n, 3.0e18),
        "zero": np.zeros(n),
    }
    for name, x in rows.items():
        x = x.astype(F32)
        xq, xd, lg, nxt = gm.probe_head(x)
        oq, od = orc.quantize_row_q8_0(orc.rms_norm(x[None], w.final_norm, eps)[0])
        same(xq, oq, f"final RMSNorm codes, {name} row")
        same(xd, od, f"final RMSNorm scales, {name} row")
        same(lg, gemv(orc, spec, oq, od, w.lm_head)[0], f"logits, {name} row")
    gm.close()


@pytest.mark.parametrize("spec,pos", [LAYERS[1], LAYERS[6]], ids=lambda v: getattr(v, "name", str(v)))
def test_exact_attention_fold_equal_keys(hip, orc, spec, pos):
    """Cached keys k0, -k0, then 0.5 k0 on every other row of a KV head: one
    of the first two scores exceeds the repeated one, so the softmax
    denominator holds a long run of equal terms below 1, whose sequential sum
    drifts from the exact sum and takes the in-order fallback of the chunked
    fold.  ctx and its codes equal the oracle's."""
    gm, om, w = layer_models(hip, orc, spec, pos + 1)
    gm.set_exact(True)
    for g in range(spec.n_kv_heads):
        k, v = syn.prefill_kv(syn.with_sizes(spec, prefilled=pos), 0, g)
        k0 = k[0].copy()
        k = np.repeat((0.5 * k0)[None], pos, axis=0).astype(k.dtype)
        k[0], k[1] = k0, -k0
        gm.kv_write(0, g, 0, k, v)
        om.kv_write(0, g, 0, k, v)
    L, (n_in, _) = w.linears[0], w.norms[0]
    x = synth_normal(spec.seed, 71, spec.hidden, 0.0, 1.0)
    pr = gm.probe_decode_layer(0, pos, x)
    oq, od = orc.quantize_row_q8_0(orc.rms_norm(x[None], n_in, spec.rms_eps)[0])
    qkv = np.concatenate([gemv(orc, spec, oq, od, L[s])[0] for s in (W_Q, W_K, W_V)])
    same(pr["qkv"], qkv, "Q|K|V rows")
    ctx = om.attention(0, qkv, pos)[0]
    same(pr["ctx"], ctx, "attention ctx")
    cq, cd = orc.quantize_row_q8_0(ctx)
    same(pr["ctx_q"], cq, "ctx codes")
    same(pr["ctx_d"], cd, "ctx scales")
    gm.close()


@pytest.mark.timeout(900)
def test_exact_layer_kernels_70b_widths(hip, orc):
    """The 70B widths (Q|K|V 10240 x 8192, gate|up 57344 x 8192, down 8192 x
    28672, 8 query heads per KV head) at position 8192 of a pre-filled
    f16 cache."""
    spec = syn.tiny(DType.Q4_0, DType.F16, head_dim=128, n_layers=1, n_heads=64, n_kv_heads=8, ffn=28672,
                    vocab=2048, seed=20260004)
    check_exact_layer(hip, orc, spec, 8192, steps=1)


def exact_model(hip, orc, spec, max_seq=None, weights=None, exact=True):
    w = weights or syn.make_weights(spec)
    gm = hip.HipModel(spec.config(max_seq))
    syn.load_model(gm, w)
    gm.set_exact(exact)
    om = orc.OracleModel.from_spec(spec, max_seq=max_seq)
    om.load(w)
    return gm, om, w


def identical_steps(gpu, ref):
    mism = np.nonzero(np.asarray(gpu) != np.asarray(ref))[0]
    return int(mism[0]) if mism.size else len(ref)


TINY = [
    syn.tiny(DType.Q4_0, DType.F32, head_dim=64),
    syn.tiny(DType.Q4_0, DType.F16, head_dim=128, n_heads=8, n_kv_heads=2, ffn=1024),
    syn.tiny(DType.Q8_0, DType.F16, head_dim=128, n_heads=4, n_kv_heads=1),
    syn.tiny(DType.Q8_0, DType.F32, head_dim=64, n_heads=8, n_kv_heads=8),
    syn.tiny(DType.Q4, DType.F16, head_dim=128, n_heads=8, n_kv_heads=2, ffn=1024, seed=11),
]


@pytest.mark.parametrize("spec", TINY, ids=lambda s: s.name)
def test_exact_tiny_models(hip, orc, spec):
    """Residual trace, logits and an 80-step greedy stream equal the
    oracle's; the prompt split at position 5 (cache below taken as filled)
    gives the same logits."""
    gm, om, w = exact_model(hip, orc, spec, max_seq=96)
    toks = syn.prompt(spec)
    lg, nxt, tr = gm.forward(toks, 0, trace=True)
    olg, otr = om.forward(toks, 0, all_rows=False, trace=True)
    same(tr, otr, "residual trace")
    same(lg, olg, "logits")
    assert nxt == orc.argmax(olg)[0]
    gtoks = gm.generate(toks, 80)
    otoks, _ = om.generate(toks, 80)
    assert identical_steps(gtoks, otoks) == 80, (gtoks[:12], otoks[:12])
    gs, _, _ = exact_model(hip, orc, spec, max_seq=96, weights=w)
    gs.forward(toks[:5], 0, logits=False)
    lg2, _, _ = gs.forward(toks[5:], 5)
    same(lg2, lg, "logits of the split prompt")


def run_workload(hip, orc, spec, steps):
    """Prompt logits and a greedy stream of `steps` tokens, GPU (exact
    mode) against the oracle; returns (max-abs logit error, identical
    steps)."""
    print(f"\n{spec.name} ({spec.prompt}+{steps}), reference-order kernels: building", flush=True)
    gm, om, _ = exact_model(hip, orc, spec)
    toks = syn.prompt(spec)
    lg, _, _ = gm.forward(toks, 0)
    olg, _ = om.forward(toks, 0)
    err = float(np.max(np.abs(lg - olg)))
    gtoks = gm.generate(toks, steps)
    otoks, margins = om.generate(toks, steps)
    n = identical_steps(gtoks, otoks)
    print(f"{spec.name}: prompt logits max-abs error {err:.3g} (bit-identical: "
          f"{np.array_equal(lg.view(np.int32), olg.view(np.int32))}); {n}/{steps} identical greedy steps; "
          f"min oracle margin {margins.min():.4g}", flush=True)
    same(lg, olg, "prompt logits")
    gm.close()
    return err, n


@pytest.mark.timeout(900)
@pytest.mark.parametrize("index,prompt_len,steps", [(0, 32, 128), (1, 32, 128), (2, 512, 64)],
                         ids=["1b-q4_0-f32kv", "1b-q8_0-f16kv", "8b-q4_0-f16kv"])
def test_exact_workload_parity_bar(hip, orc, index, prompt_len, steps):
    """The parity bar on the full-size workloads (1B Q4_0 and
    Q8_0 at 32+128, 8B at its 512-token prompt + 64 steps) with the
    reference-order kernels: logits within 1e-2 (here: equal) and every
    greedy step identical, with no near-tie allowance."""
    spec = syn.with_sizes(syn.WORKLOADS[index], prompt=prompt_len, decode=steps)
    err, n = run_workload(hip, orc, spec, steps)
    assert err < 1e-2
    assert n == steps and n >= 64


@pytest.mark.timeout(900)
def test_exact_prefill_8b_2048(hip, orc):
    """The 2048-token prompt workload through two 8B-width layers and the
    full lm_head, one batched forward on the reference-order kernels: the
    residual stream of every row and the last row's logits equal the
    oracle's batched forward."""
    spec = syn.with_sizes(syn.WORKLOADS[3], n_layers=2, prompt=2048, decode=0)
    print("\n8B-width 2-layer model, 2048-token prompt, reference-order kernels: building", flush=True)
    gm, om, _ = exact_model(hip, orc, spec, max_seq=2048)
    toks = syn.prompt(spec)
    lg, nxt, tr = gm.forward(toks, 0, trace=True)
    olg, otr = om.forward(toks, 0, all_rows=False, trace=True)
    same(tr, otr, "residual trace")
    same(lg, olg, "logits")
    assert nxt == orc.argmax(olg)[0]
    print("RAW exact 8B 2-layer 2048-token prefill: trace and logits bit-identical", flush=True)


@pytest.mark.timeout(1200)
def test_exact_70b_widths_4_layers_long_context(hip, orc):
    """Four 70B-width layers (hidden 8192, 64 query / 8 KV heads, FFN 28672)
    with the full 128256-row lm_head, decoding 16 greedy steps from 8192
    pre-filled f16 positions: every step's logits equal the oracle's and the
    streams are identical; the HIP-graph run from the same position repeats
    the stream."""
    spec = syn.with_sizes(syn.WORKLOADS[4], n_layers=4, decode=16)
    print(f"\n{spec.name} x4 layers: building", flush=True)
    gm, om, _ = exact_model(hip, orc, spec)
    for l in range(spec.n_layers):
        for g in range(spec.n_kv_heads):
            k, v = syn.prefill_kv(spec, l, g)
            gm.kv_write(l, g, 0, k, v)
            om.kv_write(l, g, 0, k, v)
    tok = syn.prompt(spec)[:1]
    ids, oids = [], []
    nxt = int(tok[0])
    for s in range(spec.decode):
        pos = spec.prefilled + s
        lg, _, _ = gm.forward([nxt], pos)
        olg, _ = om.forward([nxt], pos)
        same(lg, olg, f"logits at step {s}")
        nxt = int(np.argmax(lg))
        ids.append(nxt)
        oids.append(orc.argmax(olg)[0])
    print(f"70B widths x4: {identical_steps(ids, oids)}/{spec.decode} identical greedy steps, logits "
          f"bit-identical every step", flush=True)
    assert ids == oids
    for l in range(spec.n_layers):
        for g in range(spec.n_kv_heads):
            gm.kv_write(l, g, 0, *syn.prefill_kv(spec, l, g))
    gm.begin(tok, start_pos=spec.prefilled)
    gm.decode_steps(spec.decode - 1)
    run = gm.tokens(spec.prefilled + spec.decode + 1)[spec.prefilled + 1:]
    assert list(run) == ids


def test_exact_sampling_and_mode_switch(hip, orc):
    """Sampling reads the exact logits (each draw the oracle sampler's on
    them), and switching the mode off and on again restores the fast and
    the exact streams."""
    spec = TINY[1]
    gm, om, w = exact_model(hip, orc, spec, max_seq=96)
    toks = syn.prompt(spec)
    exact_ids = gm.generate(toks, 24)
    gm.set_exact(False)
    fast = hip.HipModel(spec.config(96))
    syn.load_model(fast, w)
    assert list(gm.generate(toks, 24)) == list(fast.generate(toks, 24))
    gm.set_exact(True)
    assert list(gm.generate(toks, 24)) == list(exact_ids)
    s = hip.Sampling.make(temperature=0.8, top_p=0.9, repeat_penalty=1.1, penalty_window=16, seed=5, eos=())
    gm.set_sampling(s)
    drawn = gm.generate(toks, 12)
    assert len(drawn) == 12
    hist = [int(t) for t in toks]
    olg, _ = om.forward(toks, 0)
    for t in drawn:  # each step's logits are the oracle's; the draw is the sampler's on them
        got, _ = hip.sample_logits(olg, np.array(hist, np.int32), s, len(hist) - 1)
        assert got == int(t)
        hist.append(int(t))
        olg, _ = om.forward([int(t)], len(hist) - 1)
