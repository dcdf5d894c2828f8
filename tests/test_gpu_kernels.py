"""Per-kernel parity of the decode and prefill kernels on their own inputs.

Every kernel of one decoder layer runs through the test probes
(llmrs_model_probe_*), which copy back each intermediate the kernels
produce; the oracle then evaluates the reference arithmetic of that one
kernel on the GPU's own inputs, so a kernel is judged alone, not through
the layers before it.  Bars:

* f32 outputs of the decode GEMVs and the decode attention:
  |gpu - oracle| <= 1e-4 + 1e-3 |oracle| (only the f32 summation order
  differs; the integer block sums are exact).
* prefill GEMMs: bit-exact (the int8 MFMA GEMM keeps the reference's block
  loop order and roundings, cpu.rs:910-937), the SwiGLU product included
  (its epilogue calls the device restatement of glibc's expf).
* Q8_0 codes a kernel builds from its own f32 values (ctx, m): equal to the
  reference quantiser's (cpu.rs:724-743) on those values, bit for bit.
* Q8_0 codes of RMSNorm rows built inside a GEMV prologue: equal, or one
  step apart where the reference's x*inv lies within 8 ulps of a .5 midpoint
  (the sum of squares is added in another order, so x*s*w can move by an
  ulp or two); scales within the rounding error of the reference's own
  sequential sum of squares (measured against float64 per row).
* decode attention: also no further from float64 sums than the
  reference's sequential f32 sums.
* K/V rows written by the kernels: bit-exact (RoPE tables are the
  reference's own f32 values, rotation in the reference's order, IEEE
  round-to-nearest-even to f16).
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import rel_close
from llmrs_hip import DType, W_DOWN, W_GATE, W_K, W_LM_HEAD, W_O, W_Q, W_UP, W_V, synthetic as syn
from llmrs_hip import synth_normal

pytestmark = pytest.mark.gpu
F32 = np.float32


def check_norm_codes(orc, gq, gd, x, w, eps, ulps=8):
    """Prologue codes of RMSNorm(x) against the reference's: returns the
    number of one-step differences, each at a rounding midpoint.

    The scales d = amax(x*s*w)/127 carry the RMSNorm factor s = 1/rms, whose
    sum of squares the reference adds in sequence (cpu.rs:381) and the GPU
    as a tree: they may differ by the reference's own rounding error of that
    sum (measured here against float64; the tree's own error is below 1e-6
    relative), halved by the square root, plus a few roundings.  The codes
    x*s*w/d do not depend on s beyond rounding."""
    x = np.asarray(x, F32)
    y = orc.rms_norm(x[None], w, eps)[0]
    oq, od = orc.quantize_row_q8_0(y)
    sq = (x * x).astype(F32)
    ss_seq = float(np.cumsum(sq, dtype=F32)[-1])       # the reference's sequential f32 sum
    ss = float(np.sum(x.astype(np.float64) ** 2))
    rel = 0.5 * (abs(ss_seq - ss) / ss + 1e-6) + 4 * 2.0 ** -24
    drel = np.abs(gd.astype(np.float64) - od) / np.maximum(od.astype(np.float64), 1e-38)
    assert np.all(drel <= rel), f"scales: max relative difference {drel.max():.3g} > {rel:.3g}"
    diff = gq.astype(np.int32) - oq.astype(np.int32)
    bad = np.nonzero(diff)[0]
    if bad.size:
        assert np.all(np.abs(diff[bad]) == 1), f"codes differ by {np.abs(diff[bad]).max()} steps"
        inv = (F32(1.0) / od[bad // 32]).astype(F32)
        p = np.abs((y[bad] * inv).astype(F32))
        dist = np.abs(p - np.floor(p) - 0.5)
        lim = ulps * np.spacing(p)
        assert np.all(dist <= lim), (
            f"code step away from a midpoint: element {bad[np.argmax(dist - lim)]}, "
            f"|x*inv| = {p[np.argmax(dist - lim)]!r}")
    return int(bad.size)


def check_own_codes(orc, q, d, v):
    """Codes a kernel derived from its own f32 output v: exactly the
    reference quantiser's."""
    oq, od = orc.quantize_row_q8_0(np.asarray(v, F32))
    assert np.array_equal(q, oq), f"{int(np.sum(q != oq))} codes differ"
    assert np.array_equal(d.view(np.int32), od.view(np.int32)), "scales differ"


def assert_close(got, want, what):
    ok, err, nbad = rel_close(got, want)
    assert ok, f"{what}: max abs err {err:.3g}, {nbad} outside 1e-4 + 1e-3 |ref|"


def layer_models(hip, orc, spec, max_seq):
    """A GPU model and an oracle model with the same layer-0 and head
    weights (no embedding: the probes feed rows directly)."""
    w = syn.make_weights(spec, embed=False)
    gm = hip.HipModel(spec.config(max_seq))
    syn.load_model(gm, w)
    om = orc.OracleModel.from_spec(spec, max_seq=max_seq)
    om.load(w)
    return gm, om, w


def fill_cache(gm, om, spec, npos):
    for g in range(spec.n_kv_heads):
        k, v = syn.prefill_kv(syn.with_sizes(spec, prefilled=npos), 0, g)
        gm.kv_write(0, g, 0, k, v)
        om.kv_write(0, g, 0, k, v)


def gemv(orc, spec, xq, xd, arrs):
    qs, sc = arrs
    n = sc.size * 32 // xq.shape[-1]
    return orc.gemv_codes(xq, xd, qs, sc, n, q8w=spec.weight == DType.Q8_0)


def exact_attention(om, orc, qkv, pos):
    """The oracle's attention with float64 sums (rounded once to f32)."""
    orc.set_attn_f64(True)
    try:
        return om.attention(0, qkv, pos)
    finally:
        orc.set_attn_f64(False)


def check_decode_attention(gm, om, orc, spec, pr, pos):
    """ctx against the oracle's attention on the GPU's projections, ctx
    codes against the quantiser, the appended K/V rows bit-exact; and the
    GPU's ctx no further from float64 sums than the reference's sequential
    f32 sums are (online softmax and split partial sums)."""
    ctx = om.attention(0, pr["qkv"], pos)[0]
    assert_close(pr["ctx"], ctx, "attention ctx")
    exact = exact_attention(om, orc, pr["qkv"], pos)[0].astype(np.float64)
    e_gpu = np.linalg.norm(pr["ctx"] - exact)
    e_ref = np.linalg.norm(ctx - exact)
    assert e_gpu <= e_ref, f"GPU attention {e_gpu:.3g} from float64 sums, the reference {e_ref:.3g}"
    check_own_codes(orc, pr["ctx_q"], pr["ctx_d"], pr["ctx"])
    for g in range(spec.n_kv_heads):
        gk, gv = gm.kv_read(0, g, pos, 1)
        ok_, ov = om.kv_read(0, g, pos, 1)
        assert np.array_equal(gk, ok_) and np.array_equal(gv, ov), f"new K/V row of KV head {g}"


# (workload, pre-filled positions): the 1B Q4_0/f32-KV and Q8_0/f16-KV, 8B
# and 70B layer widths with every GEMV shape of the workloads, the full
# 128256-row lm_head included.  The 70B case decodes at position 8192, where
# the matrix-core attention runs 32 splits x 4 waves with 2-3 tiles per wave
# (the long-context layout of the 70B workload).
DECODE_CASES = [(0, 300), (1, 300), (2, 700), (4, 8192)]


@pytest.mark.timeout(900)
@pytest.mark.parametrize("index,pos", DECODE_CASES, ids=lambda v: str(v))
def test_decode_layer_kernels(hip, orc, index, pos):
    base = syn.WORKLOADS[index]
    spec = syn.with_sizes(base, n_layers=1, prefilled=0, prompt=1, decode=1)
    max_seq = pos + 2
    print(f"\n{base.name} layer widths, decode at position {pos}", flush=True)
    gm, om, w = layer_models(hip, orc, spec, max_seq)
    fill_cache(gm, om, spec, pos)
    L = w.linears[0]
    x = synth_normal(spec.seed, 99, spec.hidden, 0.0, 1.0)
    pr = gm.probe_decode_layer(0, pos, x)
    eps = spec.rms_eps

    # Q|K|V GEMV: RMSNorm + Q8_0 prologue, then the block loop (layer.rs:177-179)
    flips = check_norm_codes(orc, pr["xq"], pr["xd"], x, w.norms[0][0], eps)
    qkv = np.concatenate([gemv(orc, spec, pr["xq"], pr["xd"], L[s])[0] for s in (W_Q, W_K, W_V)])
    assert_close(pr["qkv"], qkv, "Q|K|V GEMV")
    # decode attention (layer.rs:216-299)
    check_decode_attention(gm, om, orc, spec, pr, pos)
    # O GEMV + residual (layer.rs:329-332,386)
    h = (gemv(orc, spec, pr["ctx_q"], pr["ctx_d"], L[W_O])[0] + x).astype(F32)
    assert_close(pr["h"], h, "O GEMV + residual")
    # gate|up GEMV: RMSNorm + Q8_0 prologue, SwiGLU and Q8_0 of m (layer.rs:37-89)
    flips += check_norm_codes(orc, pr["hq"], pr["hd"], pr["h"], w.norms[0][1], eps)
    g = gemv(orc, spec, pr["hq"], pr["hd"], L[W_GATE])[0]
    u = gemv(orc, spec, pr["hq"], pr["hd"], L[W_UP])[0]
    assert_close(pr["m"], orc.silu_mul(g, u), "gate|up GEMV + SwiGLU")
    check_own_codes(orc, pr["m_q"], pr["m_d"], pr["m"])
    # down GEMV + residual (layer.rs:93-96,403)
    out = (gemv(orc, spec, pr["m_q"], pr["m_d"], L[W_DOWN])[0] + pr["h"]).astype(F32)
    assert_close(pr["out"], out, "down GEMV + residual")
    # final RMSNorm + lm_head GEMV + greedy argmax (model.rs:39-47)
    xq, xd, lg, nxt = gm.probe_head(pr["out"])
    flips += check_norm_codes(orc, xq, xd, pr["out"], w.final_norm, eps)
    assert_close(lg, gemv(orc, spec, xq, xd, w.lm_head)[0], "lm_head GEMV")
    assert nxt == int(np.argmax(lg)), "argmax partials + final reduction"
    print(f"{base.name}: every kernel within its bar; {flips} prologue codes one step apart at midpoints",
          flush=True)


# Decode attention with forced split and tile-stream counts from 700 cached
# positions (22 tiles of 32): every split and stream walks at least two
# tiles, so the next-tile prefetch, the online-softmax rescale across tiles
# and the new row on a later tile of its split (position 700 is tile 21)
# all run.  Two steps in a row, and the second step repeated: equal inputs
# give bit-identical outputs (a split that read stale LDS once made them
# differ run to run).
# (tile streams or waves, splits): tile streams per workgroup of the vector
# kernel (f32 caches: 1 or 4), tile waves per workgroup of the matrix-core
# kernel (f16: 1, 4 or 8).  At position 700 (22 tiles) one tile wave runs
# 22, 11 or 8 tiles with 1, 2 or 3 splits, four run 6 or 3 per wave with 1
# or 2 splits, eight run 3 or 1-2 with 1 or 2 splits, and 7 or 64 splits
# leave waves and whole splits without a tile.
ATTN_LAYOUTS = [(1, 1), (1, 2), (1, 3), (4, 1), (4, 2), (1, 7), (1, 64), (4, 7), (8, 1), (8, 2), (8, 7)]


@pytest.mark.parametrize("kv", [DType.F16, DType.F32], ids=["f16", "f32"])
@pytest.mark.parametrize("head_dim", [128, 64])
@pytest.mark.parametrize("nkv", [2, 8], ids=["kv2", "kv8"])
@pytest.mark.parametrize("streams,splits", ATTN_LAYOUTS, ids=lambda v: str(v))
def test_decode_attention_layouts(hip, orc, kv, head_dim, nkv, streams, splits, monkeypatch):
    """Query heads per KV head: 2 (nkv = 8) and 8 (nkv = 2)."""
    if kv == DType.F32 and streams == 8:
        pytest.skip("the vector kernel runs 1 or 4 tile streams")
    monkeypatch.setenv("LLMRS_ATTN_STREAMS" if kv == DType.F32 else "LLMRS_ATTN_WAVES", str(streams))
    monkeypatch.setenv("LLMRS_ATTN_SPLITS", str(splits))
    pos = 700
    spec = syn.tiny(DType.Q4_0, kv, head_dim=head_dim, n_layers=1, n_heads=16, n_kv_heads=nkv, ffn=512,
                    seed=31 + head_dim)
    gm, om, _ = layer_models(hip, orc, spec, pos + 3)
    fill_cache(gm, om, spec, pos)
    x = synth_normal(spec.seed, 98, spec.hidden, 0.0, 1.0)
    pr = gm.probe_decode_layer(0, pos, x)
    check_decode_attention(gm, om, orc, spec, pr, pos)
    x2 = synth_normal(spec.seed, 97, spec.hidden, 0.0, 1.0)
    pr2 = gm.probe_decode_layer(0, pos + 1, x2)
    check_decode_attention(gm, om, orc, spec, pr2, pos + 1)
    again = gm.probe_decode_layer(0, pos + 1, x2)
    assert np.array_equal(again["ctx"], pr2["ctx"]), "attention is not deterministic"


# The split combine's batches: the live splits (those holding a tile) are
# read 8, 16 or 32 at a time, and past 32 in further batches of 32 whose
# weights come from lanes 32-63 of the first (max, sum) load.  (splits, pos):
# 12 live of 12 at 700 positions (22 tiles), 40 of 40 and 47 of 64 at 1500
# (47 tiles).
COMBINE_CASES = [(12, 700), (40, 1500), (64, 1500)]


@pytest.mark.parametrize("kv", [DType.F16, DType.F32], ids=["f16", "f32"])
@pytest.mark.parametrize("head_dim", [128, 64])
@pytest.mark.parametrize("splits,pos", COMBINE_CASES, ids=lambda v: str(v))
def test_decode_attention_combine_batches(hip, orc, kv, head_dim, splits, pos, monkeypatch):
    """head_dim 128: two dims per lane in the combine (8-byte partial
    loads); 64: one (4-byte loads)."""
    monkeypatch.setenv("LLMRS_ATTN_STREAMS" if kv == DType.F32 else "LLMRS_ATTN_WAVES", "1")
    monkeypatch.setenv("LLMRS_ATTN_SPLITS", str(splits))
    spec = syn.tiny(DType.Q4_0, kv, head_dim=head_dim, n_layers=1, n_heads=32, n_kv_heads=8, ffn=512, seed=43)
    gm, om, _ = layer_models(hip, orc, spec, pos + 3)
    assert gm.decode_plan()["nsplit"] == splits
    fill_cache(gm, om, spec, pos)
    x = synth_normal(spec.seed, 96, spec.hidden, 0.0, 1.0)
    pr = gm.probe_decode_layer(0, pos, x)
    check_decode_attention(gm, om, orc, spec, pr, pos)


@pytest.mark.parametrize("kv", [DType.F16, DType.F32], ids=["f16", "f32"])
@pytest.mark.parametrize("head_dim", [128, 64])
@pytest.mark.parametrize("waves,splits", [(1, 1), (4, 2), (8, 7), (1, 64), (8, 32), (4, 7)], ids=lambda v: str(v))
def test_decode_attention_xcd_local(hip, orc, kv, head_dim, waves, splits, monkeypatch):
    """LLMRS_ATTN_LOCAL=1 (8 KV heads: a head's splits on one XCD, partials
    and tickets through its L2) gives ctx and codes bit-identical to the
    device-scope exchange, within the oracle's bar.  (waves, splits): tile
    waves of the matrix-core kernel, tile streams (1 or 4) of the f32 one."""
    if kv == DType.F32 and waves == 8:
        pytest.skip("the vector kernel runs 1 or 4 tile streams")
    monkeypatch.setenv("LLMRS_ATTN_STREAMS" if kv == DType.F32 else "LLMRS_ATTN_WAVES", str(waves))
    monkeypatch.setenv("LLMRS_ATTN_SPLITS", str(splits))
    pos = 700
    spec = syn.tiny(DType.Q4_0, kv, head_dim=head_dim, n_layers=1, n_heads=32, n_kv_heads=8, ffn=512,
                    seed=41 + head_dim)
    x = synth_normal(spec.seed, 98, spec.hidden, 0.0, 1.0)
    got = {}
    for mode in ("0", "1"):
        monkeypatch.setenv("LLMRS_ATTN_LOCAL", mode)
        gm, om, _ = layer_models(hip, orc, spec, pos + 3)
        fill_cache(gm, om, spec, pos)
        got[mode] = []
        for p in (pos, pos + 1):
            got[mode].append(gm.probe_decode_layer(0, p, x))
            if mode == "1":
                check_decode_attention(gm, om, orc, spec, got[mode][-1], p)
        gm.close()
    for a, b in zip(got["0"], got["1"]):
        for key in ("ctx", "ctx_q", "ctx_d"):
            assert np.array_equal(a[key], b[key]), f"{key} differs with the XCD-local exchange"


def check_prefill_layer(hip, orc, spec, start, M):
    """Every prefill kernel of one layer on M rows at positions start..:
    GEMMs bit-exact on the GPU's own operands (the tile GEMM, or for up to
    64 rows the skinny GEMM's exact launches)."""
    def same(got, want, what):
        assert np.array_equal(got, want), f"{what} not bit-exact"
    gm, om, w = layer_models(hip, orc, spec, start + M)
    if start:
        fill_cache(gm, om, spec, start)
    L = w.linears[0]
    H, eps = spec.hidden, spec.rms_eps
    x = synth_normal(spec.seed, 96, M * H, 0.0, 1.0).reshape(M, H)
    pr = gm.probe_prefill_layer(0, start, x)
    flips = 0
    for i in range(M):
        flips += check_norm_codes(orc, pr["xq"][i], pr["xd"][i], x[i], w.norms[0][0], eps)
    qkv = np.concatenate([gemv(orc, spec, pr["xq"], pr["xd"], L[s]) for s in (W_Q, W_K, W_V)], axis=1)
    same(pr["qkv"], qkv, "Q|K|V GEMM")
    ctx = om.attention(0, pr["qkv"], start)
    assert_close(pr["ctx"], ctx, "causal attention ctx")
    exact = exact_attention(om, orc, pr["qkv"], start).astype(np.float64)
    print(f"\nprefill attention, distance from float64 sums: GPU {np.linalg.norm(pr['ctx'] - exact):.3g}, "
          f"reference {np.linalg.norm(ctx - exact):.3g}", flush=True)
    for i in range(M):
        check_own_codes(orc, pr["ctx_q"][i], pr["ctx_d"][i], pr["ctx"][i])
    for g in range(spec.n_kv_heads):
        gk, gv = gm.kv_read(0, g, start, M)
        ok_, ov = om.kv_read(0, g, start, M)
        assert np.array_equal(gk, ok_) and np.array_equal(gv, ov), f"K/V rows of KV head {g}"
    h = (gemv(orc, spec, pr["ctx_q"], pr["ctx_d"], L[W_O]) + x).astype(F32)
    same(pr["h"], h, "O GEMM + residual")
    for i in range(M):
        flips += check_norm_codes(orc, pr["hq"][i], pr["hd"][i], pr["h"][i], w.norms[0][1], eps)
    g = gemv(orc, spec, pr["hq"], pr["hd"], L[W_GATE])
    u = gemv(orc, spec, pr["hq"], pr["hd"], L[W_UP])
    m = orc.silu_mul(g, u)
    same(pr["m"], m, "gate|up GEMM + SwiGLU")
    for i in range(M):
        check_own_codes(orc, pr["m_q"][i], pr["m_d"][i], pr["m"][i])
    out = (gemv(orc, spec, pr["m_q"], pr["m_d"], L[W_DOWN]) + pr["h"]).astype(F32)
    same(pr["out"], out, "down GEMM + residual")
    return flips


@pytest.mark.timeout(900)
def test_prefill_layer_kernels_8b_2048(hip, orc):
    """One 2048-token prefill chunk at the 8B widths (the 2048-token prefill
    workload's GEMMs: Q|K|V 6144 x 4096, O 4096 x 4096, gate|up 28672 x 4096
    with the SwiGLU epilogue, down 4096 x 14336 with the residual epilogue,
    16 token tiles, so the XCD-grouped tile order runs over many groups)."""
    spec = syn.with_sizes(syn.WORKLOADS[3], n_layers=1, vocab=1024, prompt=2048, decode=0)
    flips = check_prefill_layer(hip, orc, spec, 0, 2048)
    print(f"\n8B prefill layer, M = 2048: GEMMs bit-exact; {flips} prologue codes one step apart", flush=True)


@pytest.mark.timeout(900)
def test_prefill_layer_kernels_ragged_after_cache(hip, orc):
    """A ragged 700-row chunk at start_pos 300 at the 1B widths with Q8_0
    weights and an f16 cache: partial token and row tiles, causal attention
    over pre-filled positions, the head_dim-64 matrix-core attention."""
    spec = syn.with_sizes(syn.WORKLOADS[1], n_layers=1, vocab=1024, prompt=700, decode=0)
    check_prefill_layer(hip, orc, spec, 300, 700)


@pytest.mark.parametrize("index,start,M", [(3, 0, 24), (1, 300, 40), (2, 0, 5), (4, 0, 64)],
                         ids=["8b-24", "1b_q8-40-after-cache", "8b-5", "70b-64"])
def test_prefill_layer_kernels_short(hip, orc, index, start, M):
    """Prompts of up to 64 rows: the linear layers on the skinny GEMM's
    exact launches (one, two and four 16-token tiles), Q4_0 and Q8_0
    weights, the 70B widths, after a filled cache."""
    spec = syn.with_sizes(syn.WORKLOADS[index], n_layers=1, vocab=1024, prompt=M, decode=0, prefilled=0)
    check_prefill_layer(hip, orc, spec, start, M)
