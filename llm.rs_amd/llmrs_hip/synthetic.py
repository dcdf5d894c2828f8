"""Seeded synthetic Llama-shaped models (benchmark and test inputs).

Shapes and distributions of the five workloads the backend is measured on,
plus small shapes for parity tests.  Weights are produced by the
counter-based generator of the C library (``llmrs_synth_*``), so every
consumer - the GPU model, the CPU oracle, the benchmark - sees identical
arrays for a given (seed, tensor id).

Tensor ids: embedding 0, final norm 1, lm_head 2, prompt 3, pre-filled-KV
first token 4; layer l uses 16 + 16*l + {input norm 0, q 1, k 2, v 3, o 4,
gate 5, up 6, down 7, post norm 8, K pre-fill 9, V pre-fill 10}.
"""
from __future__ import annotations

from dataclasses import dataclass, field, replace

import numpy as np

from . import (DType, ModelConfig, N_FINAL, N_INPUT, N_POST, W_DOWN, W_GATE, W_K,
               W_LM_HEAD, W_O, W_Q, W_UP, W_V, synth_normal, synth_q4, synth_q8,
               synth_tokens)

Q4_SCALE = (0.003, 0.006)
Q8_SCALE = (2e-4, 3.5e-4)
SLOTS = (W_Q, W_K, W_V, W_O, W_GATE, W_UP, W_DOWN)


@dataclass(frozen=True)
class Spec:
    name: str
    n_layers: int
    hidden: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    ffn: int
    vocab: int
    weight: DType
    kv: DType
    prompt: int
    decode: int
    prefilled: int = 0       # positions of N(0,1) K/V written before decoding
    seed: int = 20260000
    rms_eps: float = 1e-5
    rope_theta: float = 500000.0

    @property
    def max_seq(self) -> int:
        return self.prefilled + self.prompt + self.decode

    def config(self, max_seq: int | None = None) -> ModelConfig:
        return ModelConfig(self.n_layers, self.hidden, self.n_heads, self.n_kv_heads,
                           self.head_dim, self.ffn, self.vocab, max_seq or self.max_seq,
                           self.rms_eps, self.rope_theta, int(self.weight), int(self.kv))

    def shape(self, slot: int) -> tuple[int, int]:
        H, hd, nq, nkv, F = self.hidden, self.head_dim, self.n_heads, self.n_kv_heads, self.ffn
        return {W_Q: (nq * hd, H), W_K: (nkv * hd, H), W_V: (nkv * hd, H), W_O: (H, nq * hd),
                W_GATE: (F, H), W_UP: (F, H), W_DOWN: (H, F), W_LM_HEAD: (self.vocab, H)}[slot]

    def linear_bytes(self) -> float:
        """Algorithmic weight bytes streamed per decoded token."""
        per = 18.0 / 32 if self.weight != DType.Q8_0 else 34.0 / 32
        if self.weight == DType.Q4:
            per = 20.0 / 32
        n = sum(np.prod(self.shape(s)) for s in SLOTS) * self.n_layers + np.prod(self.shape(W_LM_HEAD))
        return float(n) * per


# The five measured workloads (seed = 20260000 + index).
WORKLOADS = {
    0: Spec("llama-1b-q4_0-f32kv", 16, 2048, 32, 8, 64, 8192, 128256, DType.Q4_0, DType.F32, 32, 128),
    1: Spec("llama-1b-q8_0-f16kv", 16, 2048, 32, 8, 64, 8192, 128256, DType.Q8_0, DType.F16, 32, 128,
            seed=20260001),
    2: Spec("llama-8b-q4_0-f16kv", 32, 4096, 32, 8, 128, 14336, 128256, DType.Q4_0, DType.F16, 512, 256,
            seed=20260002),
    3: Spec("llama-8b-q4_0-prefill2048", 32, 4096, 32, 8, 128, 14336, 128256, DType.Q4_0, DType.F16,
            2048, 0, seed=20260003),
    4: Spec("llama-70b-q4_0-f16kv-ctx8192", 80, 8192, 64, 8, 128, 28672, 128256, DType.Q4_0, DType.F16,
            1, 64, prefilled=8192, seed=20260004),
}


def tiny(weight: DType = DType.Q4_0, kv: DType = DType.F32, head_dim: int = 64, n_layers: int = 2,
         n_heads: int = 4, n_kv_heads: int = 2, ffn: int = 512, vocab: int = 1000, prompt: int = 8,
         decode: int = 8, seed: int = 7) -> Spec:
    """A small model with the workload seed scheme, for parity tests."""
    return Spec(f"tiny-{weight.name}-{kv.name}-hd{head_dim}", n_layers, n_heads * head_dim, n_heads,
                n_kv_heads, head_dim, ffn, vocab, weight, kv, prompt, decode, seed=seed)


def layer_tid(layer: int, j: int) -> int:
    return 16 + 16 * layer + j


@dataclass
class Weights:
    """Host arrays of one synthetic model in the reference formats."""
    spec: Spec
    embed: np.ndarray
    final_norm: np.ndarray
    lm_head: tuple
    norms: list = field(default_factory=list)     # [(input, post)] per layer
    linears: list = field(default_factory=list)   # [{slot: (qs, scales)}] per layer


def linear(spec: Spec, tid: int, slot: int, threads: int = 0):
    n, k = spec.shape(slot)
    if spec.weight == DType.Q8_0:
        return synth_q8(spec.seed, tid, n, k, *Q8_SCALE, threads=threads)
    return synth_q4(spec.seed, tid, n, k, *Q4_SCALE, threads=threads)


def make_weights(spec: Spec, threads: int = 0, embed: bool = True) -> Weights:
    """Every tensor of `spec` (embed=False leaves the embedding table out:
    None, for probes that feed layer inputs directly)."""
    H = spec.hidden
    w = Weights(spec,
                embed=(synth_normal(spec.seed, 0, spec.vocab * H, 0.0, 0.02, threads).reshape(spec.vocab, H)
                       if embed else None),
                final_norm=synth_normal(spec.seed, 1, H, 1.0, 0.02, threads),
                lm_head=linear(spec, 2, W_LM_HEAD, threads))
    for l in range(spec.n_layers):
        w.norms.append((synth_normal(spec.seed, layer_tid(l, 0), H, 1.0, 0.02, threads),
                        synth_normal(spec.seed, layer_tid(l, 8), H, 1.0, 0.02, threads)))
        w.linears.append({s: linear(spec, layer_tid(l, 1 + s), s, threads) for s in SLOTS})
    return w


def prompt(spec: Spec) -> np.ndarray:
    return synth_tokens(spec.seed, 3, spec.prompt, spec.vocab)


def prefill_kv(spec: Spec, layer: int, kv_head: int, threads: int = 0):
    """N(0,1) K and V rows [prefilled][head_dim] of one layer / KV head."""
    n = spec.prefilled * spec.head_dim
    tk = layer_tid(layer, 9) * 64 + kv_head
    tv = layer_tid(layer, 10) * 64 + kv_head
    return (synth_normal(spec.seed, tk, n, 0.0, 1.0, threads).reshape(spec.prefilled, spec.head_dim),
            synth_normal(spec.seed, tv, n, 0.0, 1.0, threads).reshape(spec.prefilled, spec.head_dim))


def load_model(model, w: Weights) -> None:
    """Upload every tensor of `w` into a HipModel."""
    spec = w.spec
    if w.embed is not None:
        model.set_embedding(w.embed)
    model.set_norm(-1, N_FINAL, w.final_norm)
    put = model.set_linear_q8_0 if spec.weight == DType.Q8_0 else model.set_linear_q4
    put(-1, W_LM_HEAD, *w.lm_head)
    for l in range(spec.n_layers):
        model.set_norm(l, N_INPUT, w.norms[l][0])
        model.set_norm(l, N_POST, w.norms[l][1])
        for s in SLOTS:
            put(l, s, *w.linears[l][s])


def stream_model(model, spec: Spec, threads: int = 0) -> None:
    """Generate and upload tensor by tensor (bounded host memory)."""
    H = spec.hidden
    model.set_embedding(synth_normal(spec.seed, 0, spec.vocab * H, 0.0, 0.02, threads))
    model.set_norm(-1, N_FINAL, synth_normal(spec.seed, 1, H, 1.0, 0.02, threads))
    put = model.set_linear_q8_0 if spec.weight == DType.Q8_0 else model.set_linear_q4
    put(-1, W_LM_HEAD, *linear(spec, 2, W_LM_HEAD, threads))
    for l in range(spec.n_layers):
        model.set_norm(l, N_INPUT, synth_normal(spec.seed, layer_tid(l, 0), H, 1.0, 0.02, threads))
        model.set_norm(l, N_POST, synth_normal(spec.seed, layer_tid(l, 8), H, 1.0, 0.02, threads))
        for s in SLOTS:
            put(l, s, *linear(spec, layer_tid(l, 1 + s), s, threads))


def with_sizes(spec: Spec, **kw) -> Spec:
    return replace(spec, **kw)
