"""Writers of the weight files the loaders read, for tests: safetensors
checkpoints (config.json + model.safetensors or shards with an index) and
GGUF files (version 3, llama architecture).  The tensors come from the
synthetic generators; these writers only lay them out."""
from __future__ import annotations

import json
import struct
from pathlib import Path

import numpy as np

# ---- safetensors ------------------------------------------------------------

def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even f32 -> bf16 bit patterns."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return r.astype(np.uint16)


def from_bf16_bits(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


def _st_blob(tensors: dict, dtype: str) -> bytes:
    header, blobs, off = {}, [], 0
    for name, arr in tensors.items():
        a = np.asarray(arr, np.float32)
        raw = to_bf16_bits(a).tobytes() if dtype == "BF16" else np.ascontiguousarray(a).tobytes()
        header[name] = {"dtype": dtype, "shape": list(a.shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    header["__metadata__"] = {"format": "pt"}
    h = json.dumps(header).encode()
    h += b" " * (-len(h) % 8)
    return struct.pack("<Q", len(h)) + h + b"".join(blobs)


def write_checkpoint(dirpath: Path, config: dict, tensors: dict, dtype: str = "F32", shards: int = 1) -> None:
    """config.json plus model.safetensors (shards == 1) or `shards` files
    with model.safetensors.index.json."""
    dirpath.mkdir(parents=True, exist_ok=True)
    (dirpath / "config.json").write_text(json.dumps(config))
    names = list(tensors)
    if shards == 1:
        (dirpath / "model.safetensors").write_bytes(_st_blob(tensors, dtype))
        return
    weight_map = {}
    for s in range(shards):
        part = names[s::shards]
        fname = f"model-{s + 1:05d}-of-{shards:05d}.safetensors"
        (dirpath / fname).write_bytes(_st_blob({n: tensors[n] for n in part}, dtype))
        weight_map.update({n: fname for n in part})
    (dirpath / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": weight_map}))


def hf_config(spec) -> dict:
    return {"hidden_size": spec.hidden, "num_hidden_layers": spec.n_layers,
            "num_attention_heads": spec.n_heads, "num_key_value_heads": spec.n_kv_heads,
            "intermediate_size": spec.ffn, "vocab_size": spec.vocab, "rms_norm_eps": spec.rms_eps,
            "rope_theta": spec.rope_theta, "architectures": ["LlamaForCausalLM"]}

# ---- GGUF -------------------------------------------------------------------

GGUF_MAGIC = 0x46554747
F32, F16, Q4_0, Q8_0, BF16 = 0, 1, 2, 8, 30
_U32, _F32, _STR = 4, 6, 8


def _gstr(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _kv(key: str, value) -> bytes:
    if isinstance(value, str):
        return _gstr(key) + struct.pack("<I", _STR) + _gstr(value)
    if isinstance(value, float):
        return _gstr(key) + struct.pack("<If", _F32, value)
    return _gstr(key) + struct.pack("<II", _U32, int(value))


def q4_ref_to_ggml(qs: np.ndarray, scales: np.ndarray) -> bytes:
    """Reference CpuQ4 rows (byte i = e[2i] | e[2i+1] << 4, f32 scales that
    fp16 holds exactly) as ggml Q4_0 blocks (fp16 d, qs[j] = e[j] | e[j+16] << 4)."""
    q = np.asarray(qs, np.uint8).reshape(-1, 16)
    e = np.empty((q.shape[0], 32), np.uint8)
    e[:, 0::2] = q & 15
    e[:, 1::2] = q >> 4
    d = np.asarray(scales, np.float32).reshape(-1).astype(np.float16)
    assert np.array_equal(d.astype(np.float32), np.asarray(scales, np.float32).reshape(-1)), "scale not fp16"
    blk = np.empty((q.shape[0], 18), np.uint8)
    blk[:, 0:2] = d.view(np.uint8).reshape(-1, 2)
    blk[:, 2:] = e[:, :16] | (e[:, 16:] << 4)
    return blk.tobytes()


def q8_to_ggml(qs: np.ndarray, scales: np.ndarray) -> bytes:
    q = np.asarray(qs, np.int8).reshape(-1, 32)
    d = np.asarray(scales, np.float32).reshape(-1).astype(np.float16)
    assert np.array_equal(d.astype(np.float32), np.asarray(scales, np.float32).reshape(-1)), "scale not fp16"
    blk = np.empty((q.shape[0], 34), np.uint8)
    blk[:, 0:2] = d.view(np.uint8).reshape(-1, 2)
    blk[:, 2:] = q.view(np.uint8)
    return blk.tobytes()


def rope_permute_rows(n_rows: int, head_dim: int) -> np.ndarray:
    """Source (rotate-half) row of every GGUF row of a Q or K matrix:
    llama.cpp stores row h * hd/2 + j of a head at 2j + h."""
    half = head_dim // 2
    g = np.arange(n_rows)
    head, i = g // head_dim, g % head_dim
    return head * head_dim + (i % 2) * half + i // 2


def write_gguf(path: Path, meta: dict, tensors: list, alignment: int = 32) -> None:
    """tensors: (name, ggml type, ne list with ne[0] innermost, raw bytes)."""
    out = [struct.pack("<IIQQ", GGUF_MAGIC, 3, len(tensors), len(meta))]
    out += [_kv(k, v) for k, v in meta.items()]
    offs, off = [], 0
    for _, _, _, raw in tensors:
        offs.append(off)
        off += len(raw) + (-len(raw) % alignment)
    for (name, t, ne, _), o in zip(tensors, offs):
        out.append(_gstr(name) + struct.pack("<I", len(ne)) + struct.pack(f"<{len(ne)}Q", *ne) + struct.pack("<IQ", t, o))
    head = b"".join(out)
    head += b"\0" * (-len(head) % alignment)
    body = b"".join(raw + b"\0" * (-len(raw) % alignment) for _, _, _, raw in tensors)
    Path(path).write_bytes(head + body)


def gguf_meta(spec) -> dict:
    return {"general.architecture": "llama", "general.alignment": 32,
            "llama.block_count": spec.n_layers, "llama.embedding_length": spec.hidden,
            "llama.attention.head_count": spec.n_heads, "llama.attention.head_count_kv": spec.n_kv_heads,
            "llama.feed_forward_length": spec.ffn,
            "llama.attention.layer_norm_rms_epsilon": float(spec.rms_eps),
            "llama.rope.freq_base": float(spec.rope_theta)}


# ---- tokenizer ----------------------------------------------------------------

_WORDS = ("the model reads every weight once per token and the cache grows by one row "
          "a prompt goes in and text comes out while the device keeps its state resident "
          "blocks of thirty two codes share one scale the matrix cores add the products "
          "hello world sampling draws one id from the nucleus of the distribution").split()


def write_tokenizer(path, vocab_size: int) -> None:
    """A byte-level BPE tokenizer (as Llama 3's) with vocab_size ids, trained
    on a fixed synthetic corpus; specials <|begin_of_text|> (added in front
    of every encoding), <|end_of_text|>, <|eot_id|>."""
    from tokenizers import Tokenizer, decoders, models, pre_tokenizers, processors, trainers
    tok = Tokenizer(models.BPE())
    tok.pre_tokenizer = pre_tokenizers.ByteLevel(add_prefix_space=False)
    tok.decoder = decoders.ByteLevel()
    specials = ["<|begin_of_text|>", "<|end_of_text|>", "<|eot_id|>"]
    trainer = trainers.BpeTrainer(vocab_size=vocab_size, special_tokens=specials, show_progress=False,
                                  initial_alphabet=pre_tokenizers.ByteLevel.alphabet())
    rng = np.random.default_rng(1234)
    corpus = [" ".join(rng.choice(_WORDS, 12)) + f" {i} {i * 37 % 1000}" for i in range(3000)]
    tok.train_from_iterator(corpus, trainer)
    bos = tok.token_to_id("<|begin_of_text|>")
    tok.post_processor = processors.TemplateProcessing(single="<|begin_of_text|> $A",
                                                       special_tokens=[("<|begin_of_text|>", bos)])
    tok.save(str(path))
