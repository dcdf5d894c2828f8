"""Batch-1 decode benchmark of the llm.rs MI355X backend (one JSON line).

Default workload: the Llama-3-8B-shaped Q4_0 decoder with an f16 KV cache,
a 512-token random prompt, then 256 greedy decode steps (warmup + timed).
value = decode tok/s over the timed steps, weights resident in HBM.

roofline: the dominant kernel (the gate|up dequant-GEMV): algorithmic bytes
per launch over its mean launch duration inside eager decode steps, timed
by the dispatches' own start/end timestamps (hipExtModuleLaunchKernel
events on the model's stream) - the figure a rocprofv3 kernel trace of the
same steps reports.  The same kernel launched back to back over every layer
(llmrs_model_time_linear) is reported beside it.  traffic: HBM bytes per
launch from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary
(profiles/hbm_traffic.json), each counter scaled by its reading for a known
256 MiB scale_f32 pass.
prefill: the 2048-token prompt of the prefill workload through the same 8B
model (batched prefill, int8 MFMA GEMMs), timed in the same run.
cpu_baseline: the CPU oracle (C++ restatement of the reference CPU backend)
decoding at the GPU's context length on a bounded sample.
exact_decode: the same model on the reference-order kernels
(llmrs_model_set_exact), whose logits and tokens are bit-identical to the
reference CPU path's.
long_context: the 70B-shaped Q4_0 model decoding from 8192 pre-filled f16
positions (its own model, timed in the same run): tok/s, the decode
attention's duration and HBM rate, the weights + K/V roofline, and the CPU
oracle on a bounded sample of the same steps when the host has the memory.

--workload 3: the 2048-token batched prefill alone (prefill tok/s; roofline
against the int8 MFMA peak).
--traffic-probe: the dispatches the rocprofv3 --pmc runs measure.
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
INT8_PEAK_TOPS = 5000.0  # MI355X dense int8 MFMA
FP16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA
METRIC = "decode tok/s (bs1, 8B-shape Q4_0) + Q4_0 GEMV HBM GB/s vs peak"
PREFILL_METRIC = "prefill tok/s (8B-shape Q4_0, one 2048-token prompt) + GEMM MFMA utilisation"


def metric_for(index: int, name: str) -> str:
    """The headline metric for the 8B decode workload; the same measurement
    named by its own workload otherwise."""
    return METRIC if index == 2 else f"decode tok/s (bs1, {name}) + GEMV HBM GB/s vs peak"


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def hbm_traffic(workload: str, kernel: str):
    """HBM bytes per launch of `kernel` on `workload` from the committed
    rocprofv3 counter summary, or None when it holds no entry."""
    path = REPO / "profiles" / "hbm_traffic.json"
    try:
        e = json.loads(path.read_text())[workload][kernel]
    except (OSError, KeyError, ValueError):
        return None
    return e["fetch_kib"] * 1024 * e["fetch_scale"] + e["write_kib"] * 1024 * e["write_scale"]


def cpu_baseline(spec, w, context: int, seconds: float) -> dict:
    """Oracle decode tok/s on a bounded sample at the GPU's context length:
    the cache below `context` is filled with N(0,1) K/V rows (a decode
    step's cost depends on the context length, not on the cached values),
    then as many decode steps as fit in about `seconds` (at most 48)."""
    import numpy as np

    import oracle
    from llmrs_hip import synthetic as syn
    oracle.set_threads(int(os.environ.get("ORACLE_THREADS", str(min(16, os.cpu_count() or 1)))))
    om = oracle.OracleModel.from_spec(spec, max_seq=context + 64)
    om.load(w)
    fill = syn.with_sizes(spec, prefilled=context)
    for layer in range(spec.n_layers):
        for g in range(spec.n_kv_heads):
            om.kv_write(layer, g, 0, *syn.prefill_kv(fill, layer, g))
    t = int(syn.prompt(spec)[-1])
    pos, steps, t0 = context, 0, time.perf_counter()
    while steps < 48 and (time.perf_counter() - t0) < seconds:
        lg, _ = om.forward([t], pos)
        t = int(np.argmax(lg))
        pos += 1
        steps += 1
    dt = time.perf_counter() - t0
    return {"value": round(steps / dt, 3), "unit": "tok/s", "cores": oracle.threads(), "kind": "port",
            "cpu": cpu_model(),
            "sample": f"{steps} decode steps of the same model at positions {context}..{context + steps - 1} "
                      f"(the GPU's timed context; cache below {context} filled with N(0,1) K/V), "
                      f"oracle threads={oracle.threads()}"}


def cpu_prefill_baseline(spec, w, seconds: float) -> dict:
    """Oracle prefill tok/s on a bounded sample: one batched forward of a
    prompt prefix sized to take about `seconds`."""
    import oracle
    oracle.set_threads(int(os.environ.get("ORACLE_THREADS", str(min(16, os.cpu_count() or 1)))))
    from llmrs_hip import synthetic as syn
    om = oracle.OracleModel.from_spec(spec, max_seq=256)
    om.load(w)
    toks = syn.prompt(spec)
    n = 8
    t0 = time.perf_counter()
    om.forward(toks[:n], 0)
    dt = time.perf_counter() - t0
    # second pass sized from the first
    n2 = int(max(8, min(256, n * seconds / max(dt, 1e-3) * 0.8)))
    t0 = time.perf_counter()
    om.forward(toks[:n2], 0)
    dt = time.perf_counter() - t0
    return {"value": round(n2 / dt, 3), "unit": "tok/s", "cores": oracle.threads(), "kind": "port",
            "cpu": cpu_model(),
            "sample": f"one batched forward of the first {n2} prompt tokens of the same model, "
                      f"oracle threads={oracle.threads()}"}


def host_mem_available() -> int:
    """Bytes of host memory available (MemAvailable), 0 when unknown."""
    try:
        for line in Path("/proc/meminfo").read_text().splitlines():
            if line.startswith("MemAvailable:"):
                return int(line.split()[1]) * 1024
    except (OSError, ValueError):
        pass
    return 0


def exact_decode(model, lh, prompt, pre: int, steps: int) -> dict:
    """The reference-order kernels on the same model: the prompt (batched),
    then `steps` timed greedy steps."""
    model.set_exact(True)
    try:
        t0 = time.perf_counter()
        model.begin(prompt, start_pos=pre)
        lh.sync()
        prompt_s = time.perf_counter() - t0
        model.decode_steps(2)
        lh.sync()
        t0 = time.perf_counter()
        model.decode_steps(steps)
        lh.sync()
        dt = time.perf_counter() - t0
    finally:
        model.set_exact(False)
    return {"tok_s": round(steps / dt, 1), "ms_per_token": round(dt / steps * 1e3, 3), "steps": steps,
            "prompt_ms": round(prompt_s * 1e3, 1),
            "note": "reference-order kernels (llmrs_model_set_exact): every f32 sum in the reference CPU "
                    "path's order, logits and greedy tokens bit-identical to it; the prompt runs as one "
                    "batched forward"}


def long_context(lh, syn, warmup: int, steps: int, cpu_seconds: float, cpu: bool) -> dict:
    """The 70B-shaped Q4_0 workload: decode from 8192 pre-filled N(0,1) f16
    positions on its own model."""
    import numpy as np
    spec = syn.with_sizes(syn.WORKLOADS[4], decode=warmup + steps)
    max_seq = spec.max_seq + 2
    pre = spec.prefilled
    t0 = time.perf_counter()
    model = lh.HipModel(spec.config(max_seq))
    # the oracle's sample needs its own host copy of the weights (Q4 codes
    # + f32 scales, the f32 embedding) and of the f16 cache
    need = spec.linear_bytes() * 20 / 18 + 4.0 * spec.vocab * spec.hidden + \
        2.0 * 2 * spec.n_layers * spec.n_kv_heads * spec.head_dim * max_seq
    avail = host_mem_available()
    run_cpu = cpu and avail > 1.5 * need
    if run_cpu:
        w = syn.make_weights(spec)
        syn.load_model(model, w)
    else:
        w = None
        syn.stream_model(model, spec)
    log(f"long context: {spec.name} uploaded in {time.perf_counter() - t0:.1f}s "
        f"({model.weight_bytes() / 1e9:.2f} GB of linear weights)")
    t0 = time.perf_counter()
    for layer in range(spec.n_layers):
        for g in range(spec.n_kv_heads):
            model.kv_write(layer, g, 0, *syn.prefill_kv(spec, layer, g))
    log(f"long context: K/V cache pre-filled ({pre} positions) in {time.perf_counter() - t0:.1f}s")
    prompt = syn.prompt(spec)
    model.begin(prompt, start_pos=pre)
    model.decode_steps(warmup)
    lh.sync()
    t0 = time.perf_counter()
    model.decode_steps(steps)
    lh.sync()
    dt = time.perf_counter() - t0
    first = pre + spec.prompt + warmup
    value = steps / dt
    attn = defaultdict(lambda: [0.0, 0.0, 0])
    for _ in range(2):
        for k in model.profile_step():
            if k.name.startswith("attn_decode"):
                e = attn[k.name]
                e[0] += k.ms
                e[1] += k.bytes
                e[2] += 1
    name, (ams, aby, an) = max(attn.items(), key=lambda kv: kv[1][0])
    a_us, a_bytes = ams / an * 1e3, aby / an
    wbytes = model.weight_bytes()
    kv_bytes = 2.0 * spec.n_layers * spec.n_kv_heads * spec.head_dim * (first + (steps - 1) / 2 + 1) * 2
    roof = HBM_PEAK_GBS * 1e9 / (wbytes + kv_bytes)
    model.close()
    log(f"long context: {value:.1f} tok/s, {name} {a_us:.2f} us per layer "
        f"({a_bytes / a_us / 1e3:.0f} GB/s)")
    out = {"workload": f"{spec.name} decode", "tok_s": round(value, 2), "ms_per_token": round(dt / steps * 1e3, 3),
           "steps": steps, "warmup": warmup, "timed_positions": [first, first + steps - 1],
           "attention": {"kernel": name, "avg_us": round(a_us, 2), "kv_bytes_per_launch": round(a_bytes),
                         "gb_s": round(a_bytes / a_us / 1e3, 1),
                         "frac_of_hbm_peak": round(a_bytes / a_us / 1e3 / HBM_PEAK_GBS, 4)},
           "weights_kv_roofline_tok_s": round(roof, 1), "frac_of_weights_kv_roofline": round(value / roof, 4),
           "weights_roofline_tok_s": round(HBM_PEAK_GBS * 1e9 / wbytes, 1),
           "frac_of_weights_roofline": round(value * wbytes / (HBM_PEAK_GBS * 1e9), 4)}
    if run_cpu:
        log("long context: timing the CPU oracle on a bounded sample ...")
        out["cpu_baseline"] = cpu_baseline(spec, w, first, cpu_seconds)
        log(f"long context cpu baseline: {out['cpu_baseline']['value']} tok/s")
    else:
        out["cpu_baseline"] = {"value": None, "unit": "tok/s",
                               "note": f"not run: the oracle's copy of the weights and cache needs about "
                                       f"{need / 2**30:.0f} GiB of host memory; {avail / 2**30:.0f} GiB available"
                                       if cpu else "not run (--no-cpu-baseline)"}
    del w
    return out


def measure_prefill(model, lh, prompt, warmup: int, steps: int, profile_steps: int, workload: str) -> dict:
    """Batched prefill of `prompt` from position 0: tok/s over `steps` whole
    prompts (each rewrites the KV cache), per-kernel rates from dispatch
    timestamps, GEMM MFMA utilisation against the int8 and fp16 peaks."""
    M = len(prompt)
    for _ in range(warmup):
        model.forward(prompt, 0, logits=False)
    lh.sync()
    t0 = time.perf_counter()
    for i in range(steps):
        model.forward(prompt, 0, logits=False)
        log(f"prefill {i + 1}/{steps}")
    lh.sync()
    dt = time.perf_counter() - t0
    value = steps * M / dt
    log(f"prefill: {value:.1f} tok/s ({dt / steps * 1e3:.2f} ms per {M}-token prompt)")
    per = defaultdict(lambda: [0.0, 0.0, 0])
    for _ in range(profile_steps):
        for k in model.profile_prefill(prompt):
            e = per[k.name]
            e[0] += k.ms
            e[1] += k.bytes
            e[2] += 1
    P = max(1, profile_steps)
    tot = sum(ms for ms, _, _ in per.values())
    kernels = {}
    for name, (ms, wk, n) in sorted(per.items(), key=lambda kv: -kv[1][0]):
        avg_s = ms / n / 1e3
        flop = name.startswith("gemm_") or name.startswith("attn_")
        kernels[name] = {"launches": n // P, "avg_us": round(avg_s * 1e6, 2), "share": round(ms / tot, 4),
                         ("tflop_s" if flop else "gb_s"): round(wk / n / avg_s / (1e12 if flop else 1e9), 1)}
    gemm = [n for n in per if n.startswith("gemm_")]
    g_ms = sum(per[n][0] for n in gemm)
    g_fl = sum(per[n][1] for n in gemm)
    dom = max(gemm, key=lambda n: per[n][0])
    ms, fl, n = per[dom]
    achieved = fl / n / (ms / n / 1e3) / 1e12
    traffic = hbm_traffic(workload, dom)
    gemm_rate = g_fl / (g_ms / 1e3) / 1e12
    return {
        "value": value, "ms": dt / steps * 1e3, "prompt": M,
        "roofline": {"bound": "mfma", "kernel": dom, "achieved": round(achieved, 1),
                     "peak": INT8_PEAK_TOPS, "unit": "TOP/s", "frac": round(achieved / INT8_PEAK_TOPS, 4),
                     "flops_per_launch": round(fl / n), "avg_us": round(ms / n * 1e3, 2),
                     "traffic": None if traffic is None else round(traffic),
                     "traffic_source": "profiles/hbm_traffic.json (rocprofv3 FETCH_SIZE + WRITE_SIZE)"},
        "gemm_top_s": round(gemm_rate, 1),
        "gemm_frac_int8_peak": round(gemm_rate / INT8_PEAK_TOPS, 4),
        "gemm_frac_fp16_peak": round(gemm_rate / FP16_PEAK_TFLOPS, 4),
        "gemm_share_of_prefill": round(g_ms / tot, 4),
        "kernels": kernels,
    }


def bench_prefill(args, lh, syn) -> int:
    """The 2048-token prefill workload alone (one JSON line)."""
    spec = syn.WORKLOADS[args.workload]
    if args.prompt:
        spec = syn.with_sizes(spec, prompt=args.prompt, decode=0)
    M = spec.prompt
    lh.init(0)
    t0 = time.perf_counter()
    keep = not args.no_cpu_baseline
    model = lh.HipModel(spec.config(M))
    if keep:
        w = syn.make_weights(spec)
        syn.load_model(model, w)
    else:
        w = None
        syn.stream_model(model, spec)
    log(f"workload {spec.name}: weights uploaded in {time.perf_counter() - t0:.1f}s")
    pf = measure_prefill(model, lh, syn.prompt(spec), args.warmup, args.steps, args.profile_steps,
                         f"{spec.name} prefill")
    cpu = None
    if keep:
        log("timing the CPU oracle prefill on a bounded sample ...")
        cpu = cpu_prefill_baseline(spec, w, args.cpu_seconds)
        log(f"cpu baseline: {cpu['value']} tok/s on {cpu['cores']} threads")
    line = {
        "metric": PREFILL_METRIC, "value": round(pf["value"], 1), "unit": "tok/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(pf["ms"], 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8 MFMA (q4_0 x q8_0, exact block sums) + f32", "data": "synthetic",
        "config": {"workload": f"{spec.name} prefill", "layers": spec.n_layers, "hidden": spec.hidden,
                   "heads": spec.n_heads, "kv_heads": spec.n_kv_heads, "head_dim": spec.head_dim,
                   "ffn": spec.ffn, "vocab": spec.vocab, "weights": spec.weight.name,
                   "kv_cache": spec.kv.name.lower(), "prompt": M, "batch": 1},
        "roofline": pf["roofline"],
        "gemm_mfma_utilisation": pf["gemm_frac_int8_peak"],
        "gemm_frac_fp16_peak": pf["gemm_frac_fp16_peak"],
        "gemm_share_of_prefill": pf["gemm_share_of_prefill"],
        "cpu_baseline": cpu,
        "kernels": pf["kernels"],
    }
    print(json.dumps(line), flush=True)
    return 0


def traffic_probe(args, lh, syn) -> int:
    """Dispatches for HBM-traffic counters: the workload's prompt as one
    batched prefill (every prefill kernel once per layer at its real M),
    four eager decode steps right after it (every decode kernel at the
    prompt's context length), two batched decode steps of 16 sequences
    (after their 8-token prefills) and a scale_f32 pass over 64 Mi floats, whose
    FETCH_SIZE / WRITE_SIZE readings calibrate the counters (each ideally
    256 MiB)."""
    import numpy as np
    base = syn.WORKLOADS[args.workload]
    spec = syn.with_sizes(base, prompt=args.prompt or base.prompt, decode=8)
    lh.init(0)
    model = lh.HipModel(spec.config(spec.prompt + 16))
    syn.stream_model(model, spec)
    model.begin(syn.prompt(spec))
    model.decode_steps(2)
    lh.sync()
    for _ in range(2):
        model.profile_step()
    lh.sync()
    # two batched decode steps of 16 sequences (8-token prompts): the skinny GEMMs
    bt = lh.HipBatch(model, 16)
    for sl in range(16):
        bt.begin(sl, syn.prompt(spec)[:8])
    bt.decode_steps(2)
    lh.sync()
    bt.close()
    n = 64 << 20
    x = lh.Tensor.from_numpy(np.ones((n // 4096, 4096), np.float32))
    lh.HipBackend().scale(x, 1.0)
    lh.sync()
    print(json.dumps({"probe": "traffic", "workload": spec.name, "prompt": spec.prompt,
                      "decode_context": [spec.prompt + 1, spec.prompt + 4], "calibration_kernel": "scale_f32",
                      "calibration_read_bytes": 4 * n, "calibration_write_bytes": 4 * n}), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="timed steps (decode 240, prefill 5)")
    ap.add_argument("--warmup", type=int, default=None, help="untimed steps (decode 16, prefill 1)")
    ap.add_argument("--workload", type=int, default=2)
    ap.add_argument("--prompt", type=int, default=None, help="override the prompt length")
    ap.add_argument("--profile-steps", type=int, default=4)
    ap.add_argument("--prefill-steps", type=int, default=3,
                    help="timed 2048-token prefills in the decode run (0 = none)")
    ap.add_argument("--batch-sizes", type=lambda v: [int(x) for x in v.split(",") if x], default=[4, 16, 64],
                    help="batched-decode sizes measured after the single-sequence run (empty: none)")
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--exact-steps", type=int, default=32,
                    help="timed steps of the reference-order kernels in the decode run (0 = none)")
    ap.add_argument("--long-context-steps", type=int, default=32,
                    help="timed steps of the 70B long-context workload in the 8B decode run (0 = none)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="for rocprofv3 --pmc runs: the workload's prompt prefill, eager decode steps, then one "
                         "256 MiB scale_f32 pass (reads and writes 256 MiB) that calibrates the counters")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this backend runs on one GPU; multi-GPU figures are not produced "
              "(run with --gpus 1)", file=sys.stderr)
        return 2

    import llmrs_hip as lh
    from llmrs_hip import synthetic as syn

    if args.traffic_probe:
        return traffic_probe(args, lh, syn)
    prefill_only = syn.WORKLOADS[args.workload].decode == 0
    if args.steps is None:
        args.steps = 5 if prefill_only else 240
    if args.warmup is None:
        args.warmup = 1 if prefill_only else 16
    if prefill_only:
        return bench_prefill(args, lh, syn)
    base = syn.WORKLOADS[args.workload]
    n_prompt = args.prompt or base.prompt
    spec = syn.with_sizes(base, prompt=n_prompt, decode=args.warmup + args.steps)
    lh.init(0)
    pre = spec.prefilled  # cache positions filled with N(0,1) K/V before the prompt
    # The 8B decode run also measures the 2048-token prefill workload (its
    # own model, so the decode model keeps the attention layout of its
    # context length).
    pf_spec = syn.WORKLOADS[3] if args.workload == 2 and args.prefill_steps > 0 else None
    max_seq = spec.max_seq + args.profile_steps + 1
    log(f"workload {spec.name}: pre-filled {pre}, prompt {n_prompt}, decode {args.warmup}+{args.steps}, "
        f"max_seq {max_seq}")

    t0 = time.perf_counter()
    # The CPU sample of a pre-filled long-context workload would need the
    # oracle's own copy of every weight and of the cache; it is not run.
    keep = not args.no_cpu_baseline and not pre
    model = lh.HipModel(spec.config(max_seq))
    if keep:
        w = syn.make_weights(spec)
        syn.load_model(model, w)
    else:
        w = None
        syn.stream_model(model, spec)
    log(f"weights generated and uploaded in {time.perf_counter() - t0:.1f}s "
        f"({model.weight_bytes() / 1e9:.3f} GB of linear weights)")

    if pre:
        t0 = time.perf_counter()
        for layer in range(spec.n_layers):
            for g in range(spec.n_kv_heads):
                model.kv_write(layer, g, 0, *syn.prefill_kv(spec, layer, g))
        log(f"K/V cache pre-filled ({pre} positions) in {time.perf_counter() - t0:.1f}s")
    prompt = syn.prompt(spec)
    t0 = time.perf_counter()
    model.begin(prompt, start_pos=pre)
    lh.sync()
    prompt_s = time.perf_counter() - t0
    log(f"prompt of {n_prompt} tokens processed in {prompt_s * 1e3:.1f} ms")

    model.decode_steps(args.warmup)
    lh.sync()
    # the benchmark contract brackets the timed steps with a device-wide
    # synchronisation through torch as well as the library's own
    try:
        import torch
        sync_all = torch.cuda.synchronize if torch.cuda.is_available() else lh.sync
    except Exception:
        sync_all = lh.sync
    sync_all()
    lh.sync()
    t0 = time.perf_counter()
    model.decode_steps(args.steps)
    lh.sync()
    sync_all()
    dt = time.perf_counter() - t0
    first = pre + n_prompt + args.warmup  # position of the first timed step
    toks = model.tokens(first + args.steps + 1)[pre:]
    assert toks.min() >= 0 and toks.max() < spec.vocab
    value = args.steps / dt
    log(f"decode: {value:.1f} tok/s ({dt / args.steps * 1e3:.3f} ms/token), positions {first}..{first + args.steps - 1}")

    # Per-kernel durations inside eager decode steps (dispatch timestamps).
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
    # The dominant kernel: the gate|up GEMV.
    dom = next(n for n in kernels if n.startswith("gemv_") and "_silu_" in n)
    ms, by, n = per[dom]
    dom_us, dom_bytes = ms / n * 1e3, by / n
    achieved = dom_bytes / (dom_us * 1e-6) / 1e9
    b2b_us, _ = model.time_linear(lh.W_GATE, reps=4)
    traffic = hbm_traffic(f"{spec.name} decode", dom)
    log(f"{dom}: {dom_us:.2f} us per launch in decode steps ({achieved:.0f} GB/s), {b2b_us:.2f} us back to "
        f"back; HBM traffic per launch {traffic if traffic is None else round(traffic / 1e6, 2)} MB")
    wbytes = model.weight_bytes()
    roof_tok_s = HBM_PEAK_GBS * 1e9 / wbytes
    # The weights + K/V variant: every layer also reads its cache rows
    # 0..pos, 2 * nkv * hd * (pos + 1) elements, at the mean timed position.
    kv_elem = 2 if spec.kv == lh.DType.F16 else 4
    kv_bytes = 2 * spec.n_layers * spec.n_kv_heads * spec.head_dim * (first + (args.steps - 1) / 2 + 1) * kv_elem
    roof_kv_tok_s = HBM_PEAK_GBS * 1e9 / (wbytes + kv_bytes)

    # Sampled decoding (the reference token loop's defaults: penalty 1.2 over
    # 64 ids, temperature 0.8, top_p 0.9; no end-of-sequence stop) from the
    # same prompt, and the sampler's own duration in an eager step.
    samp = lh.Sampling.make(seed=2026, eos=())
    model.set_sampling(samp)
    sampled_steps = min(64, args.steps)
    model.begin(prompt, start_pos=pre)
    model.decode_steps(min(4, args.warmup))
    lh.sync()
    t0 = time.perf_counter()
    model.decode_steps(sampled_steps)
    lh.sync()
    sdt = time.perf_counter() - t0
    sampler = [k for k in model.profile_step() if k.name.startswith("sample_")]
    model.set_sampling(None)
    sampled = {"tok_s": round(sampled_steps / sdt, 1), "steps": sampled_steps,
               "sampler_us": round(sum(k.ms for k in sampler) * 1e3, 2) if sampler else None,
               "sampler_launches": len(sampler),
               "temperature": 0.8, "top_p": 0.9, "repeat_penalty": 1.2, "penalty_window": 64}
    log(f"sampled decode: {sampled['tok_s']} tok/s, sampler {sampled['sampler_us']} us per token")

    exact = None
    exact_steps = min(args.exact_steps, max_seq - pre - n_prompt - 3)  # what the cache still holds
    if exact_steps > 0:
        exact = exact_decode(model, lh, prompt, pre, exact_steps)
        log(f"reference-order decode: {exact['tok_s']} tok/s ({exact['ms_per_token']} ms/token)")

    # Batched decode: B sequences with their own prompts and caches stepping
    # together (greedy), on the same weights; aggregate tok/s per batch size.
    batched = None
    if args.batch_sizes:
        batched = {"sizes": {}, "prompt": 64, "steps": 32,
                   "note": "B sequences, each its own 64-token random prompt and K/V cache; "
                           "aggregate tokens/s over 32 greedy steps (HIP-graph replay)"}
        import numpy as np
        rng = np.random.default_rng(7)
        for B in args.batch_sizes:
            bt = lh.HipBatch(model, B)
            for sl in range(B):
                bt.begin(sl, rng.integers(0, spec.vocab, 64).astype(np.int32))
            bt.decode_steps(2)
            lh.sync()
            t0 = time.perf_counter()
            bt.decode_steps(32)
            lh.sync()
            bdt = time.perf_counter() - t0
            batched["sizes"][str(B)] = {"tok_s": round(32 * B / bdt, 1), "ms_per_step": round(bdt / 32 * 1e3, 3)}
            bt.close()
            log(f"batched decode B={B}: {32 * B / bdt:.1f} tok/s ({bdt / 32 * 1e3:.3f} ms/step)")

    prefill = None
    if pf_spec:
        t0 = time.perf_counter()
        pf_model = lh.HipModel(pf_spec.config(pf_spec.prompt))
        syn.stream_model(pf_model, pf_spec)
        log(f"2048-token prefill model uploaded in {time.perf_counter() - t0:.1f}s")
        pf = measure_prefill(pf_model, lh, syn.prompt(pf_spec), 1, args.prefill_steps, 2,
                             f"{pf_spec.name} prefill")
        pf_model.close()
        prefill = {"workload": f"{pf_spec.name} prefill",
                   "tok_s": round(pf["value"], 1), "ms": round(pf["ms"], 3), "prompt": pf["prompt"],
                   "steps": args.prefill_steps, "roofline": pf["roofline"],
                   "gemm_top_s": pf["gemm_top_s"], "gemm_frac_int8_peak": pf["gemm_frac_int8_peak"],
                   "gemm_frac_fp16_peak": pf["gemm_frac_fp16_peak"],
                   "gemm_share_of_prefill": pf["gemm_share_of_prefill"]}

    cpu = None
    if keep:
        log("timing the CPU oracle on a bounded sample ...")
        cpu = cpu_baseline(spec, w, first, args.cpu_seconds)
        log(f"cpu baseline: {cpu['value']} tok/s on {cpu['cores']} threads")

    lc = None
    if args.workload == 2 and args.long_context_steps > 0:
        model.close()
        w = None
        lc = long_context(lh, syn, 4, args.long_context_steps, args.cpu_seconds, not args.no_cpu_baseline)

    line = {
        "metric": metric_for(args.workload, spec.name), "value": round(value, 2), "unit": "tok/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(dt / args.steps * 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8 dot4 (q4_0 x q8_0) + f32", "data": "synthetic",
        "config": {"workload": f"{spec.name} decode", "layers": spec.n_layers, "hidden": spec.hidden,
                   "heads": spec.n_heads, "kv_heads": spec.n_kv_heads, "head_dim": spec.head_dim,
                   "ffn": spec.ffn, "vocab": spec.vocab, "weights": spec.weight.name,
                   "kv_cache": spec.kv.name.lower(), "prefilled_positions": pre, "prompt": n_prompt,
                   "decode_steps": args.warmup + args.steps, "timed_positions": [first, first + args.steps - 1],
                   "batch": 1},
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "bytes_per_launch": round(dom_bytes), "avg_us": round(dom_us, 2),
                     "timing": "mean duration of its launches inside eager decode steps (dispatch timestamps)",
                     "back_to_back_us": round(b2b_us, 2),
                     "back_to_back_frac": round(dom_bytes / (b2b_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                     "traffic": None if traffic is None else round(traffic),
                     "traffic_source": "profiles/hbm_traffic.json (rocprofv3 FETCH_SIZE + WRITE_SIZE)"},
        "cpu_baseline": cpu,
        "decode_roofline_tok_s": round(roof_tok_s, 1),
        "frac_of_decode_roofline": round(value / roof_tok_s, 4),
        "decode_roofline_weights_kv_tok_s": round(roof_kv_tok_s, 1),
        "frac_of_weights_kv_roofline": round(value / roof_kv_tok_s, 4),
        "weight_gb_per_token": round(wbytes / 1e9, 4),
        "prompt_ms": round(prompt_s * 1e3, 1),
        "prefill": prefill,
        "long_context": lc,
        "exact_decode": exact,
        "sampled_decode": sampled,
        "batched_decode": batched,
        "kernels": kernels,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
