"""Text front-end of the resident HIP model: the reference's command-line
token loop with real prompts and text output.

Mirrors src/main.rs: the arguments and their defaults (main.rs:28-58), the
tokenizer (`tokenizers` 0.22.2, the crate version the reference pins;
Tokenizer::from_file and encode(prompt, add_special_tokens=true),
main.rs:105-111), the loop of `steps` iterations - the whole prompt first,
then one token per step (main.rs:128-138) - with sampling and the
end-of-sequence stop on the device (main.rs:192-310), each produced id
decoded on its own with skip_special_tokens=true and printed as it arrives
(main.rs:315-325), and the closing timings (main.rs:330-340: total, TTFT,
TBT = (total - TTFT) / tokens in whole milliseconds).

The model comes from a Hugging Face checkpoint directory (config.json plus
safetensors), a .safetensors file with config.json beside it, or a GGUF file.

    python -m llmrs_hip.textgen -m models/ -t models/tokenizer.json -p "Hello world"
"""
from __future__ import annotations

import argparse
import sys
import time
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

from . import DType, HipModel, LLAMA3_EOS, MAX_EOS, Sampling

# The reference's end-of-sequence ids are Llama 3's (main.rs:121); a tokenizer
# that defines these tokens gives their ids (the same numbers for Llama 3).
EOS_TOKENS = ("<|end_of_text|>", "<|eot_id|>")


def load_tokenizer(path):
    from tokenizers import Tokenizer
    return Tokenizer.from_file(str(path))


def eos_ids(tokenizer) -> tuple[int, ...]:
    ids = tuple(i for i in (tokenizer.token_to_id(t) for t in EOS_TOKENS) if i is not None)
    return ids or LLAMA3_EOS


def load_model(path, max_seq: int = 0, kv: DType = DType.F16) -> HipModel:
    """A checkpoint directory or .safetensors file, or a .gguf file."""
    p = Path(path)
    if p.suffix == ".gguf":
        return HipModel.load_gguf(p, max_seq=max_seq, kv=kv)
    return HipModel.load_safetensors(p, max_seq=max_seq, kv=kv)


@dataclass
class Generation:
    prompt_ids: list[int]
    ids: list[int] = field(default_factory=list)  # produced, end-of-sequence id excluded
    text: str = ""
    stopped: bool = False                          # an end-of-sequence id ended the run
    total_s: float = 0.0
    ttft_ms: int = 0
    tbt_ms: int = 0


class TextGenerator:
    """Prompt in, text out, over a resident model and a tokenizer."""

    def __init__(self, model: HipModel, tokenizer, sampling: Sampling | None = None):
        self.model = model
        self.tokenizer = tokenizer
        self.sampling = sampling
        model.set_sampling(sampling)

    def encode(self, prompt: str) -> list[int]:
        ids = self.tokenizer.encode(prompt, add_special_tokens=True).ids  # main.rs:108-111
        if not ids:
            raise ValueError("the prompt encodes to no tokens")
        vocab = self.model.cfg.vocab
        bad = [i for i in ids if i >= vocab]
        if bad:
            raise ValueError(f"token ids {bad[:4]} beyond the model's vocabulary of {vocab}")
        return ids

    def generate(self, prompt: str, steps: int, on_text=None) -> Generation:
        """Up to `steps` ids (the first from the prompt); `on_text(word)` is
        called with each id's text as it arrives."""
        ids = self.encode(prompt)
        n0 = len(ids)
        if n0 + steps > self.model.cfg.max_seq:
            raise ValueError(f"prompt ({n0}) + steps ({steps}) exceed the model's {self.model.cfg.max_seq} positions")
        g = Generation(prompt_ids=ids)
        if steps == 0:
            return g
        t0 = time.perf_counter()
        self.model.begin(np.asarray(ids, np.int32))
        words = []
        ttft = 0.0
        done = 0  # iterations of the reference loop run (the prompt is the first)
        while True:
            done += 1
            produced, stopped = self.model.produced()
            if produced > len(g.ids):
                tok = int(self.model.tokens(n0 + produced)[-1])
                word = self.tokenizer.decode([tok], skip_special_tokens=True)  # main.rs:315-317
                if not g.ids:
                    ttft = time.perf_counter() - t0
                g.ids.append(tok)
                words.append(word)
                if on_text:
                    on_text(word)
            if stopped:
                g.stopped = True
                break
            if done >= steps:
                break
            self.model.decode_steps(1)
        g.total_s = time.perf_counter() - t0
        g.text = "".join(words)
        g.ttft_ms = int(ttft * 1e3)
        g.tbt_ms = int((g.total_s - ttft) * 1e3) // len(g.ids) if g.ids else 0
        return g


def build_parser() -> argparse.ArgumentParser:
    """main.rs:28-58's arguments and defaults, plus the seed, greedy and
    KV options this backend adds."""
    ap = argparse.ArgumentParser(description="Text generation on the MI355X backend (src/main.rs's loop)")
    ap.add_argument("-m", "--model", default="models/model.safetensors",
                    help="checkpoint directory, .safetensors file (config.json beside it) or .gguf file")
    ap.add_argument("-c", "--config", default=None,
                    help="config.json; it must be the one beside the weights (the loader reads that one)")
    ap.add_argument("-t", "--tokenizer", default="models/tokenizer.json")
    ap.add_argument("-p", "--prompt", default="Hello world")
    ap.add_argument("-n", "--steps", type=int, default=200)
    ap.add_argument("-r", "--repeat-penalty", type=float, default=1.2)
    ap.add_argument("-w", "--penalty-window", type=int, default=64)
    ap.add_argument("--temperature", type=float, default=0.8)
    ap.add_argument("--top-p", type=float, default=0.9)
    ap.add_argument("--seed", type=int, default=None, help="draws repeat for a given seed (default: from the clock)")
    ap.add_argument("--greedy", action="store_true", help="argmax instead of sampling")
    ap.add_argument("--max-seq", type=int, default=0, help="KV positions (0: 2048, as the reference)")
    ap.add_argument("--kv", choices=("f16", "f32"), default="f16")
    return ap


def main(argv=None) -> int:
    args = build_parser().parse_args(argv)

    model_path = Path(args.model)
    if args.config is not None and model_path.suffix != ".gguf":
        beside = (model_path if model_path.is_dir() else model_path.parent) / "config.json"
        if Path(args.config).resolve() != beside.resolve():
            print(f"textgen: the loader reads {beside}; --config {args.config} differs", file=sys.stderr)
            return 2
    t0 = time.perf_counter()
    model = load_model(model_path, max_seq=args.max_seq, kv=DType.F16 if args.kv == "f16" else DType.F32)
    tok = load_tokenizer(args.tokenizer)
    print(f"[textgen] model and tokenizer loaded in {time.perf_counter() - t0:.2f}s", file=sys.stderr)
    sampling = None
    if not args.greedy:
        seed = args.seed if args.seed is not None else time.time_ns()
        sampling = Sampling.make(temperature=args.temperature, top_p=args.top_p,
                                 repeat_penalty=args.repeat_penalty, penalty_window=args.penalty_window,
                                 seed=seed, eos=eos_ids(tok)[:MAX_EOS])
    gen = TextGenerator(model, tok, sampling)
    print("\n--- Output ---")
    print(args.prompt, end="", flush=True)
    g = gen.generate(args.prompt, args.steps, on_text=lambda w: print(w, end="", flush=True))
    print("\n--------------")
    print(f"[textgen] Total Time: {g.total_s:.2f}s", file=sys.stderr)
    print(f"[textgen] TTFT Time: {g.ttft_ms}ms", file=sys.stderr)
    print(f"[textgen] TBT Time: {g.tbt_ms}ms", file=sys.stderr)
    print(f"[textgen] tokens: {len(g.ids)}{' (end of sequence)' if g.stopped else ''}", file=sys.stderr)
    model.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
