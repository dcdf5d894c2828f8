"""Weight-file loaders: llmrs_model_load_safetensors (Loader::load_model,
src/core/loader.rs:100-198, with Tensor::quantize_q4, tensor.rs:102-167) and
llmrs_model_load_gguf (no reference counterpart).

A loaded model must equal the model built by uploading the same weights
through the C-ABI (bit-identical logits and tokens): the safetensors path
against the oracle's restatement of quantize_q4, the GGUF path against the
Q4_0 / Q8_0 blocks it was written from.  The loaded model is also held to
the oracle (1e-2 logits, identical greedy stream).  Malformed files are
rejected with LLMRS_E_FORMAT before any device work, so those tests run on
the CPU."""
from __future__ import annotations

import ctypes as C
import struct

import numpy as np
import pytest

import weight_files as wf
from conftest import check_stream
from llmrs_hip import DType, synthetic as syn

E_FORMAT, E_NOINIT = -8, -4


def tiny(weight, kv=DType.F16, **kw):
    base = dict(head_dim=64, n_layers=2, n_heads=4, n_kv_heads=2, ffn=256, vocab=384, prompt=6, decode=12, seed=41)
    base.update(kw)
    return syn.tiny(weight, kv, **base)


def f32_weights(spec):
    """Float weights of `spec` in the Hugging Face names (rows x cols)."""
    H, seed = spec.hidden, spec.seed
    t = {"model.embed_tokens.weight": syn.synth_normal(seed, 0, spec.vocab * H, 0.0, 0.02).reshape(spec.vocab, H),
         "model.norm.weight": syn.synth_normal(seed, 1, H, 1.0, 0.02),
         "lm_head.weight": syn.synth_normal(seed, 2, spec.vocab * H, 0.0, 0.05).reshape(spec.vocab, H)}
    names = {syn.W_Q: "self_attn.q_proj", syn.W_K: "self_attn.k_proj", syn.W_V: "self_attn.v_proj",
             syn.W_O: "self_attn.o_proj", syn.W_GATE: "mlp.gate_proj", syn.W_UP: "mlp.up_proj",
             syn.W_DOWN: "mlp.down_proj"}
    for l in range(spec.n_layers):
        p = f"model.layers.{l}."
        t[p + "input_layernorm.weight"] = syn.synth_normal(seed, syn.layer_tid(l, 0), H, 1.0, 0.02)
        t[p + "post_attention_layernorm.weight"] = syn.synth_normal(seed, syn.layer_tid(l, 8), H, 1.0, 0.02)
        for s, nm in names.items():
            n, k = spec.shape(s)
            t[p + nm + ".weight"] = syn.synth_normal(seed, syn.layer_tid(l, 1 + s), n * k, 0.0, 0.05).reshape(n, k)
    return t, names


def upload_f32(model_or_oracle, orc, spec, t, names, tied=False):
    """The same weights through the C-ABI (or into the oracle), quantised by
    the oracle's quantize_q4."""
    m = model_or_oracle
    m.set_embedding(t["model.embed_tokens.weight"])
    m.set_norm(-1, syn.N_FINAL, t["model.norm.weight"])
    head = t["model.embed_tokens.weight"] if tied else t["lm_head.weight"]
    m.set_linear_q4(-1, syn.W_LM_HEAD, *orc.quantize_q4(head))
    for l in range(spec.n_layers):
        p = f"model.layers.{l}."
        m.set_norm(l, syn.N_INPUT, t[p + "input_layernorm.weight"])
        m.set_norm(l, syn.N_POST, t[p + "post_attention_layernorm.weight"])
        for s, nm in names.items():
            m.set_linear_q4(l, s, *orc.quantize_q4(t[p + nm + ".weight"]))


def same_model(a, b, toks, steps):
    la, na, _ = a.forward(toks, 0)
    lb, nb, _ = b.forward(toks, 0)
    assert np.array_equal(la, lb) and na == nb, f"logits differ by {np.max(np.abs(la - lb))}"
    ga, gb = a.generate(toks, steps), b.generate(toks, steps)
    assert np.array_equal(ga, gb)
    return la, ga


# ---- CPU: malformed files ---------------------------------------------------

def load_rc(hip_lib, fn, path):
    """(return code, message).  A file that parses reaches model creation,
    which needs an initialised device: LLMRS_E_NOINIT on the CPU (0, with
    the model freed again, where a device is up)."""
    h = C.c_void_p()
    rc = getattr(hip_lib, fn)(str(path).encode(), None, C.byref(h))
    msg = hip_lib.llmrs_last_error().decode()
    if rc == 0:
        hip_lib.llmrs_model_free(h)
        rc = E_NOINIT
    return rc, msg


@pytest.fixture(scope="module")
def hlib():
    import llmrs_hip
    return llmrs_hip.lib()


def gguf_q4_file(path, spec, w, embed_f16=True, mix=False, drop=None, arch="llama"):
    """A GGUF file of synthetic Q4_0 (or Q8_0) weights `w` of `spec`."""
    H, hd, V = spec.hidden, spec.head_dim, spec.vocab
    q8 = spec.weight == DType.Q8_0
    emb = w.embed.astype(np.float16) if embed_f16 else w.embed.astype(np.float32)
    ts = [("token_embd.weight", wf.F16 if embed_f16 else wf.F32, [H, V], emb.tobytes())]
    names = {syn.W_Q: "attn_q", syn.W_K: "attn_k", syn.W_V: "attn_v", syn.W_O: "attn_output",
             syn.W_GATE: "ffn_gate", syn.W_UP: "ffn_up", syn.W_DOWN: "ffn_down"}

    def lin(qs, sc, n, k, rope):
        rows = wf.rope_permute_rows(n, hd) if rope else np.arange(n)
        if q8:
            return wf.Q8_0, wf.q8_to_ggml(np.asarray(qs).reshape(n, k)[rows], np.asarray(sc).reshape(n, k // 32)[rows])
        return wf.Q4_0, wf.q4_ref_to_ggml(np.asarray(qs).reshape(n, k // 2)[rows], np.asarray(sc).reshape(n, k // 32)[rows])

    for l in range(spec.n_layers):
        ts.append((f"blk.{l}.attn_norm.weight", wf.F32, [H], w.norms[l][0].astype(np.float32).tobytes()))
        ts.append((f"blk.{l}.ffn_norm.weight", wf.F32, [H], w.norms[l][1].astype(np.float32).tobytes()))
        for s, nm in names.items():
            n, k = spec.shape(s)
            t, raw = lin(*w.linears[l][s], n, k, s in (syn.W_Q, syn.W_K))
            if mix and l == 1 and s == syn.W_DOWN:  # one weight in the other format
                t = wf.Q8_0 if t == wf.Q4_0 else wf.Q4_0
                raw = bytes((n * k // 32) * (34 if t == wf.Q8_0 else 18))
            ts.append((f"blk.{l}.{nm}.weight", t, [k, n], raw))
    ts.append(("output_norm.weight", wf.F32, [H], w.final_norm.astype(np.float32).tobytes()))
    t, raw = lin(*w.lm_head, V, H, False)
    ts.append(("output.weight", t, [H, V], raw))
    if drop:
        ts = [x for x in ts if x[0] != drop]
    meta = wf.gguf_meta(spec)
    meta["general.architecture"] = arch
    wf.write_gguf(path, meta, ts)


def test_gguf_rejects_malformed_files(tmp_path, hlib):
    spec = tiny(DType.Q4_0)
    w = syn.make_weights(spec)
    good = tmp_path / "m.gguf"
    gguf_q4_file(good, spec, w)
    rc, msg = load_rc(hlib, "llmrs_model_load_gguf", good)
    assert rc == E_NOINIT, msg  # parsed; creating the model needs the device
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"GGML" + good.read_bytes()[4:])
    assert load_rc(hlib, "llmrs_model_load_gguf", bad)[0] == E_FORMAT
    bad.write_bytes(good.read_bytes()[:200])
    rc, msg = load_rc(hlib, "llmrs_model_load_gguf", bad)
    assert rc == E_FORMAT and ("truncated" in msg or "beyond" in msg), msg
    gguf_q4_file(bad, spec, w, arch="gpt2")
    rc, msg = load_rc(hlib, "llmrs_model_load_gguf", bad)
    assert rc == E_FORMAT and "architecture" in msg, msg
    gguf_q4_file(bad, spec, w, mix=True)
    rc, msg = load_rc(hlib, "llmrs_model_load_gguf", bad)
    assert rc == E_FORMAT and "mix" in msg, msg
    gguf_q4_file(bad, spec, w, drop="blk.1.ffn_up.weight")
    rc, msg = load_rc(hlib, "llmrs_model_load_gguf", bad)
    assert rc == E_FORMAT and "ffn_up" in msg, msg
    assert load_rc(hlib, "llmrs_model_load_gguf", tmp_path / "missing.gguf")[0] == E_FORMAT
    # crafted sizes: every bound is checked without wrapping, and unsupported
    # tensor types are refused before any device work (E_FORMAT, not the
    # E_NOINIT that creating the model on this host would give)
    raw = good.read_bytes()
    bad.write_bytes(raw[:24] + struct.pack("<Q", (1 << 64) - 8) + raw[32:])  # first key's length
    rc, msg = load_rc(hlib, "llmrs_model_load_gguf", bad)
    assert rc == E_FORMAT and "truncated" in msg, msg
    name = b"output.weight"
    at = raw.index(struct.pack("<Q", len(name)) + name) + 8 + len(name)  # nd, ne[2], type, offset
    ne_pos, type_pos, off_pos = at + 4, at + 4 + 16, at + 4 + 16 + 4

    def patched(pos, fmt, value):
        return raw[:pos] + struct.pack(fmt, value) + raw[pos + struct.calcsize(fmt):]
    for off in ((1 << 64) - 16, 1 << 63, len(raw)):
        bad.write_bytes(patched(off_pos, "<Q", off))
        rc, msg = load_rc(hlib, "llmrs_model_load_gguf", bad)
        assert rc == E_FORMAT and "beyond" in msg, (off, msg)
    bad.write_bytes(raw[:ne_pos] + struct.pack("<QQ", 1 << 40, 1 << 40) + raw[ne_pos + 16:])
    rc, msg = load_rc(hlib, "llmrs_model_load_gguf", bad)
    assert rc == E_FORMAT and "larger than the file" in msg, msg
    bad.write_bytes(patched(type_pos, "<I", 14))  # Q6_K, as common llama.cpp Q4_0 files store output.weight
    rc, msg = load_rc(hlib, "llmrs_model_load_gguf", bad)
    assert rc == E_FORMAT and "output.weight" in msg and "type 14" in msg, msg


def test_safetensors_rejects_malformed_files(tmp_path, hlib):
    spec = tiny(DType.Q4)
    t, _ = f32_weights(spec)
    d = tmp_path / "ck"
    wf.write_checkpoint(d, wf.hf_config(spec), t)
    rc, msg = load_rc(hlib, "llmrs_model_load_safetensors", d)
    assert rc == E_NOINIT, msg
    raw = (d / "model.safetensors").read_bytes()
    (d / "model.safetensors").write_bytes(struct.pack("<Q", len(raw)) + raw[8:])
    rc, msg = load_rc(hlib, "llmrs_model_load_safetensors", d)
    assert rc == E_FORMAT and "header" in msg, msg
    (d / "model.safetensors").write_bytes(raw[:8] + b"x" + raw[9:])
    assert load_rc(hlib, "llmrs_model_load_safetensors", d)[0] == E_FORMAT
    (d / "model.safetensors").write_bytes(raw)
    (d / "config.json").write_text("{\"hidden_size\": 64}")
    rc, msg = load_rc(hlib, "llmrs_model_load_safetensors", d)
    assert rc == E_FORMAT and "num_hidden_layers" in msg, msg
    # a header nested far deeper than any real one is refused, not recursed into
    deep = b'{"a":' + b"[" * 100000 + b"]" * 100000 + b"}"
    (d / "model.safetensors").write_bytes(struct.pack("<Q", len(deep)) + deep)
    rc, msg = load_rc(hlib, "llmrs_model_load_safetensors", d)
    assert rc == E_FORMAT and "deep" in msg, msg
    (d / "config.json").unlink()
    assert load_rc(hlib, "llmrs_model_load_safetensors", d)[0] == E_FORMAT


def test_writers_round_trip(tmp_path):
    """The test writers against independent readers: safetensors' own numpy
    loader for F32 checkpoints, bf16 rounding against float64 arithmetic."""
    from safetensors.numpy import load_file
    spec = tiny(DType.Q4)
    t, _ = f32_weights(spec)
    wf.write_checkpoint(tmp_path, wf.hf_config(spec), t)
    back = load_file(str(tmp_path / "model.safetensors"))
    assert set(back) == set(t) and all(np.array_equal(back[k], t[k]) for k in t)
    # ties to even: 1 + 2^-8 lies halfway between 1 and 1 + 2^-7
    x = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -2.5e-3, 1.0 + 2 ** -8 + 2 ** -9], np.float32)
    b = wf.from_bf16_bits(wf.to_bf16_bits(x))
    assert b[:3].tolist() == [1.0, 1.0, 1.0 + 2 ** -6] and b[4] == 1.0 + 2 ** -7
    assert abs(float(b[3]) + 2.5e-3) <= 2.5e-3 * 2 ** -8
    rows = wf.rope_permute_rows(8, 4)  # two heads of 4: rows 0,2,1,3 within each
    assert rows.tolist() == [0, 2, 1, 3, 4, 6, 5, 7]


# ---- GPU: loaded models equal uploaded ones ---------------------------------

@pytest.mark.gpu
@pytest.mark.parametrize("dtype,tied,shards", [("F32", False, 1), ("BF16", False, 3), ("F32", True, 2)],
                         ids=["f32", "bf16-shards", "f32-tied"])
def test_load_safetensors(tmp_path, hip, orc, dtype, tied, shards):
    spec = tiny(DType.Q4)
    t, names = f32_weights(spec)
    if tied:
        del t["lm_head.weight"]
    wf.write_checkpoint(tmp_path, wf.hf_config(spec), t, dtype=dtype, shards=shards)
    if dtype == "BF16":
        t = {k: wf.from_bf16_bits(wf.to_bf16_bits(v)).reshape(np.shape(v)) for k, v in t.items()}
    max_seq = spec.prompt + spec.decode + 4
    loaded = hip.HipModel.load_safetensors(tmp_path, max_seq=max_seq, kv=DType.F16)
    assert loaded.cfg.vocab == spec.vocab and loaded.cfg.weight_dtype == DType.Q4
    direct = hip.HipModel(spec.config(max_seq))
    upload_f32(direct, orc, spec, t, names, tied)
    toks = syn.prompt(spec)
    lg, gen = same_model(loaded, direct, toks, spec.decode)
    om = orc.OracleModel.from_spec(spec, max_seq=max_seq)
    upload_f32(om, orc, spec, t, names, tied)
    olg, _ = om.forward(toks, 0)
    assert np.max(np.abs(lg - olg)) < 1e-2
    if not tied:  # the tied N(0, 0.02) embedding gives logits of std ~0.3: near-ties within the 1e-2 bar
        check_stream(gen, *om.generate(toks, spec.decode))


@pytest.mark.gpu
@pytest.mark.parametrize("weight", [DType.Q4_0, DType.Q8_0], ids=["q4_0", "q8_0"])
def test_load_gguf(tmp_path, hip, orc, weight):
    """Q4_0 / Q8_0 blocks taken as they are; Q and K rows un-permuted from
    llama.cpp's order (a wrong permutation changes every logit)."""
    spec = tiny(weight)
    w = syn.make_weights(spec)
    w.embed = w.embed.astype(np.float16).astype(np.float32)  # the file holds it in f16
    path = tmp_path / "m.gguf"
    gguf_q4_file(path, spec, w)
    max_seq = spec.prompt + spec.decode + 4
    loaded = hip.HipModel.load_gguf(path, max_seq=max_seq, kv=DType.F16)
    assert loaded.cfg.weight_dtype == weight and loaded.cfg.n_kv_heads == spec.n_kv_heads
    direct = hip.HipModel(spec.config(max_seq))
    syn.load_model(direct, w)
    toks = syn.prompt(spec)
    lg, gen = same_model(loaded, direct, toks, spec.decode)
    om = orc.OracleModel.from_spec(spec, max_seq=max_seq)
    om.load(w)
    olg, _ = om.forward(toks, 0)
    assert np.max(np.abs(lg - olg)) < 1e-2
    check_stream(gen, *om.generate(toks, spec.decode))
