"""Batch-1 decode benchmark of the llm.rs MI355X backend (one JSON line).

Default workload: the Llama-3-8B-shaped Q4_0 decoder with an f16 KV cache,
a 512-token random prompt, then 256 greedy decode steps (warmup + timed).
value = decode tok/s over the timed steps, weights resident in HBM.

roofline: the dominant kernel (gate|up dequant-GEMV) - algorithmic bytes per
launch over its mean duration from HIP events on the model's stream.
cpu_baseline: the CPU oracle (C++ restatement of the reference CPU backend)
on a bounded sample of the same workload, timed on this host.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from collections import defaultdict
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "llm.rs_amd"))
sys.path.insert(0, str(REPO))

HBM_PEAK_GBS = 8000.0
METRIC = "decode tok/s (bs1, 8B-shape Q4_0) + Q4_0 GEMV HBM GB/s vs peak"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_baseline(spec, w, seconds: float) -> dict:
    """Oracle decode tok/s on a bounded sample: an 8-token prefix prefilled
    (untimed), then as many decode steps as fit in about `seconds`."""
    import numpy as np

    import oracle
    oracle.set_threads(int(os.environ.get("ORACLE_THREADS", "0")))
    om = oracle.OracleModel.from_spec(spec, max_seq=64)
    om.load(w)
    from llmrs_hip import synthetic as syn
    toks = syn.prompt(spec)[:8]
    lg, _ = om.forward(toks, 0)
    t = int(np.argmax(lg))
    pos = len(toks)
    steps, t0 = 0, time.perf_counter()
    while steps < 48 and (time.perf_counter() - t0) < seconds:
        lg, _ = om.forward([t], pos)
        t = int(np.argmax(lg))
        pos += 1
        steps += 1
    dt = time.perf_counter() - t0
    return {"value": round(steps / dt, 3), "unit": "tok/s", "cores": oracle.threads(), "kind": "port",
            "sample": f"{steps} decode steps of the same model after an 8-token prefill "
                      f"(positions 8..{7 + steps}), oracle threads={oracle.threads()}"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=240)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--workload", type=int, default=2)
    ap.add_argument("--prompt", type=int, default=None, help="override the prompt length")
    ap.add_argument("--profile-steps", type=int, default=4)
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this backend runs on one GPU; multi-GPU figures are not produced "
              "(run with --gpus 1)", file=sys.stderr)
        return 2

    import numpy as np

    import llmrs_hip as lh
    from llmrs_hip import synthetic as syn

    base = syn.WORKLOADS[args.workload]
    n_prompt = args.prompt or base.prompt
    spec = syn.with_sizes(base, prompt=n_prompt, decode=args.warmup + args.steps)
    lh.init(0)
    max_seq = spec.max_seq + args.profile_steps + 1
    log(f"workload {spec.name}: prompt {n_prompt}, decode {args.warmup}+{args.steps}, max_seq {max_seq}")

    t0 = time.perf_counter()
    keep = not args.no_cpu_baseline
    model = lh.HipModel(spec.config(max_seq))
    if keep:
        w = syn.make_weights(spec)
        syn.load_model(model, w)
    else:
        w = None
        syn.stream_model(model, spec)
    log(f"weights generated and uploaded in {time.perf_counter() - t0:.1f}s "
        f"({model.weight_bytes() / 1e9:.3f} GB of linear weights)")

    prompt = syn.prompt(spec)
    t0 = time.perf_counter()
    model.begin(prompt)
    lh.sync()
    prompt_s = time.perf_counter() - t0
    log(f"prompt of {n_prompt} tokens processed in {prompt_s * 1e3:.1f} ms")

    model.decode_steps(args.warmup)
    lh.sync()
    try:
        import torch
        sync_all = torch.cuda.synchronize if torch.cuda.is_available() else lh.sync
    except Exception:  # torch is only the device-wide barrier here
        sync_all = lh.sync
    sync_all()
    lh.sync()
    t0 = time.perf_counter()
    model.decode_steps(args.steps)
    lh.sync()
    sync_all()
    dt = time.perf_counter() - t0
    toks = model.tokens(n_prompt + args.warmup + args.steps + 1)
    assert toks.min() >= 0 and toks.max() < spec.vocab
    value = args.steps / dt
    log(f"decode: {value:.1f} tok/s ({dt / args.steps * 1e3:.3f} ms/token)")

    # Per-kernel timing with HIP events on the model's stream (eager steps).
    per = defaultdict(lambda: [0.0, 0.0, 0])
    for _ in range(args.profile_steps):
        for k in model.profile_step():
            e = per[k.name]
            e[0] += k.ms
            e[1] += k.bytes
            e[2] += 1
    kernels = {}
    for name, (ms, by, n) in sorted(per.items(), key=lambda kv: -kv[1][0]):
        avg_s = ms / n / 1e3
        kernels[name] = {"launches_per_step": n // max(1, args.profile_steps),
                         "avg_us": round(avg_s * 1e6, 2),
                         "gb_s": round(by / n / avg_s / 1e9, 1) if avg_s > 0 else None,
                         "share": None}
    tot = sum(ms for ms, _, _ in per.values())
    for name, (ms, _, _) in per.items():
        kernels[name]["share"] = round(ms / tot, 4)
    dom = max((n for n in kernels if n.startswith("gemv_")), key=lambda n: per[n][0])
    ms, by, n = per[dom]
    achieved = by / n / (ms / n / 1e3) / 1e9
    wbytes = model.weight_bytes()
    roof_tok_s = HBM_PEAK_GBS * 1e9 / wbytes

    cpu = None
    if keep:
        log("timing the CPU oracle on a bounded sample ...")
        cpu = cpu_baseline(spec, w, args.cpu_seconds)
        log(f"cpu baseline: {cpu['value']} tok/s on {cpu['cores']} threads")

    line = {
        "metric": METRIC, "value": round(value, 2), "unit": "tok/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(dt / args.steps * 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8 dot4 (q4_0 x q8_0) + f32", "data": "synthetic",
        "config": {"workload": f"{spec.name} decode", "layers": spec.n_layers, "hidden": spec.hidden,
                   "heads": spec.n_heads, "kv_heads": spec.n_kv_heads, "head_dim": spec.head_dim,
                   "ffn": spec.ffn, "vocab": spec.vocab, "weights": spec.weight.name,
                   "kv_cache": spec.kv.name.lower(), "prompt": n_prompt,
                   "decode_steps": args.warmup + args.steps, "batch": 1},
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "bytes_per_launch": round(by / n), "avg_us": round(ms / n * 1e3, 2),
                     "traffic": None},
        "cpu_baseline": cpu,
        "decode_roofline_tok_s": round(roof_tok_s, 1),
        "frac_of_decode_roofline": round(value / roof_tok_s, 4),
        "weight_gb_per_token": round(wbytes / 1e9, 4),
        "prompt_ms": round(prompt_s * 1e3, 1),
        "kernels": kernels,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
