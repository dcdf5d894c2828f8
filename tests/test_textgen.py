"""Text front-end (llmrs_hip.textgen): the reference's command-line token
loop (src/main.rs:28-58 arguments, :105-111 tokenizer, :128-327 loop,
:315-317 per-token text, :330-340 timings) over a loaded checkpoint.

The tokenizer is the `tokenizers` library at the version the reference pins
(0.22.2), so its encode/decode are the reference's own; the tests pin what
the front-end does with them: special tokens added on encode and skipped on
decode, the end-of-sequence ids, the arguments' defaults, and - on the GPU -
that the streamed ids and text equal the device generation's for the same
seed, from a safetensors checkpoint through the loader to text."""
from __future__ import annotations

import numpy as np
import pytest

import weight_files as wf
from llmrs_hip import LLAMA3_EOS, Sampling, synthetic as syn
from llmrs_hip import textgen


@pytest.fixture(scope="module")
def tok_path(tmp_path_factory):
    p = tmp_path_factory.mktemp("tok") / "tokenizer.json"
    wf.write_tokenizer(p, 1000)
    return p


def test_tokenizer_conventions(tok_path):
    tok = textgen.load_tokenizer(tok_path)
    ids = tok.encode("Hello world, the model reads", add_special_tokens=True).ids
    assert ids[0] == tok.token_to_id("<|begin_of_text|>")
    assert tok.decode(ids, skip_special_tokens=True) == "Hello world, the model reads"
    # per-token text (main.rs:315-317): byte-level tokens carry their spaces
    assert "".join(tok.decode([i], skip_special_tokens=True) for i in ids) == "Hello world, the model reads"
    assert tok.decode([ids[0]], skip_special_tokens=True) == ""
    assert textgen.eos_ids(tok) == (tok.token_to_id("<|end_of_text|>"), tok.token_to_id("<|eot_id|>"))


def test_eos_fallback_is_the_references():
    class NoSpecials:
        def token_to_id(self, t):
            return None
    assert textgen.eos_ids(NoSpecials()) == LLAMA3_EOS == (128001, 128009)


def test_argument_defaults():
    a = textgen.build_parser().parse_args([])
    assert (a.model, a.tokenizer, a.prompt, a.steps) == ("models/model.safetensors", "models/tokenizer.json",
                                                         "Hello world", 200)
    assert (a.repeat_penalty, a.penalty_window, a.temperature, a.top_p) == (1.2, 64, 0.8, 0.9)


SPEC = syn.tiny(syn.DType.Q4, syn.DType.F16, head_dim=64, n_layers=2, n_heads=4, n_kv_heads=2, ffn=256,
                vocab=1000, seed=43)


@pytest.fixture(scope="module")
def checkpoint(tmp_path_factory, tok_path):
    import test_loader as tl
    d = tmp_path_factory.mktemp("ckpt")
    t, _ = tl.f32_weights(SPEC)
    wf.write_checkpoint(d, wf.hf_config(SPEC), t, dtype="BF16")
    return d


@pytest.mark.gpu
def test_text_generation_matches_device_stream(hip, checkpoint, tok_path):
    tok = textgen.load_tokenizer(tok_path)
    model = textgen.load_model(checkpoint, max_seq=256)
    s = Sampling.make(seed=7, eos=textgen.eos_ids(tok))
    gen = textgen.TextGenerator(model, tok, s)
    streamed = []
    g = gen.generate("Hello world, the model reads", 40, on_text=streamed.append)
    assert g.prompt_ids == tok.encode("Hello world, the model reads", add_special_tokens=True).ids
    assert 0 < len(g.ids) <= 40 and (g.stopped or len(g.ids) == 40)
    # the same run through the device loop alone
    model.set_sampling(s)
    direct = model.generate(np.asarray(g.prompt_ids, np.int32), 40)
    assert list(direct) == g.ids
    assert streamed == [tok.decode([i], skip_special_tokens=True) for i in g.ids]
    assert g.text == "".join(streamed)
    assert g.ttft_ms >= 0 and g.tbt_ms >= 0 and g.total_s > 0
    # greedy: the model's argmax stream
    gen_g = textgen.TextGenerator(model, tok, None)
    gg = gen_g.generate("the cache grows", 24)
    assert gg.ids == list(model.generate(np.asarray(gg.prompt_ids, np.int32), 24))
    # an end-of-sequence id stops the loop before it is emitted
    k = next((j for j in range(3, len(g.ids)) if g.ids[j] not in g.ids[:j]), None)
    if k is not None:
        s2 = Sampling.make(seed=7, eos=(g.ids[k],))
        g2 = textgen.TextGenerator(model, tok, s2).generate("Hello world, the model reads", 40)
        assert g2.stopped and g2.ids == g.ids[:k]
    with pytest.raises(ValueError):
        gen.generate("x " * 300, 10)  # beyond max_seq
    model.close()


@pytest.mark.gpu
def test_command_line(hip, checkpoint, tok_path, capsys):
    argv = ["-m", str(checkpoint), "-t", str(tok_path), "-p", "blocks of thirty two", "-n", "16",
            "--seed", "3", "--max-seq", "128"]
    assert textgen.main(argv) == 0
    r = capsys.readouterr()
    assert "--- Output ---" in r.out and "TTFT Time" in r.err and "TBT Time" in r.err
    # the same text through the generator
    tok = textgen.load_tokenizer(tok_path)
    model = textgen.load_model(checkpoint, max_seq=128)
    g = textgen.TextGenerator(model, tok, Sampling.make(seed=3, eos=textgen.eos_ids(tok))).generate(
        "blocks of thirty two", 16)
    out = r.out.split("--- Output ---\n", 1)[1].split("\n--------------", 1)[0]
    assert out == "blocks of thirty two" + g.text
    model.close()
    # a --config other than the one beside the weights is refused
    assert textgen.main(argv + ["-c", str(tok_path)]) == 2
