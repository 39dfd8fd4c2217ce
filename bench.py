"""Batch-1 greedy decode benchmark on one MI355X.

Workload: a 48-layer Gemma-3-12B-shaped model with seeded random weights (hidden 3840,
FFN 15360, 16 q / 8 kv heads of width 256, 5:1 local(window 1024):global layers, Q4_0
projections, tied Q6_K embedding/lm-head over 262144 ids); a 128-token random prompt is
prefilled, then W warm-up and K timed greedy decode steps run through
GenerationSession::generate (per token: one persistent launch for all 48 layers, one launch
for the Q6_K head + greedy argmax; ids come back through mapped host memory).
A "step" is one decoded token; `value` is tokens per second over the K timed steps.

After the timed region, a few more decode steps run with a hipEvent pair around every launch
(af_session_profile) to time the dominant kernel (the layers kernel) for the roofline object,
with its per-phase timeline from in-kernel timestamps.  The CPU baseline is the C oracle (a
port of the reference's FP64 CPU path) timed on a bounded sample on this host.

    python bench.py [--gpus 1] [--steps 240] [--warmup 16]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "batch-1 decode tok/s @12B-shape Q4_0; Q4_0 GEMV HBM GB/s vs 8 TB/s peak"
PEAK_GBS = 8000.0
PROMPT = 128
PROFILE_STEPS = 8


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def cpu_baseline(model, prompt, tokens, threads):
    """The oracle (C port of the reference's FP64 CPU chain) decoding `tokens` tokens after a
    one-token prefill: each token is 48 layers + final norm + Q6_K head + greedy."""
    import numpy as np

    import oracle
    ref = oracle.Model(model, capacity=tokens + 2, threads=threads)
    ref.step(int(prompt[0]))
    t0 = time.perf_counter()
    for _ in range(tokens):
        logits = ref.logits().astype(np.float32)
        ref.step(oracle.greedy(logits))
    dt = time.perf_counter() - t0
    ref.close()
    return tokens / dt, dt


def measured_traffic(kernel="void af::decode_step_kernel<2>(af::StepArgs)"):
    """HBM bytes per launch from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE passes
    (profiles/traffic_config4.json, calibrated against a copy of known size), or None."""
    path = os.path.join(ROOT, "profiles", "traffic_config4.json")
    try:
        with open(path) as f:
            return json.load(f)["kernels"][kernel]["hbm_bytes"]
    except (OSError, KeyError, ValueError):
        return None


def kv_read_bytes(model, tokens):
    """fp16 K and V rows one decode step reads at context `tokens` (window-limited layers)."""
    total = 0
    for L in model.layers:
        vis = min(tokens, L.window) if L.window else tokens
        total += vis * L.kv_heads * L.head_width * 2 * 2
    return total


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=240)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--cpu-tokens", type=int, default=4)
    ap.add_argument("--no-cpu", action="store_true")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py measures one GPU: the batch-1 decode path runs on a single MI355X "
              f"(--gpus {a.gpus} is not supported; see DESIGN.md for how the path would shard)", file=sys.stderr)
        sys.exit(2)
    if a.steps < 1 or a.warmup < 1:
        sys.exit("--steps and --warmup must be >= 1")

    from adaforge_amd import synth
    from adaforge_amd.backend import HipDiagnostics

    t = time.perf_counter()
    model = synth.model()
    log(f"model generated in {time.perf_counter() - t:.1f}s")
    prompt = [int(i) for i in synth.prompt_ids(PROMPT, model.vocabulary, name="config4.prompt")]
    stop = [model.vocabulary - 1]
    capacity = PROMPT + a.warmup + a.steps + PROFILE_STEPS + 2
    diag = HipDiagnostics()
    dev = diag.check()
    log(f"device {dev.device_name} {dev.arch} CUs={dev.compute_units}")
    t = time.perf_counter()
    session = diag.open_session(model, capacity)
    log(f"session open (weight upload) in {time.perf_counter() - t:.1f}s")

    first = session.generate(prompt, stop, a.warmup)
    cached = prompt + first.ids
    log(f"prefill {PROMPT} tokens: {first.stats.prefill_ms:.1f} ms; warm-up {len(first.ids)} tokens")

    produced = 0
    t0 = time.perf_counter()
    while produced < a.steps:
        r = session.generate(cached, stop, min(128, a.steps - produced))
        cached += r.ids
        produced += len(r.ids)
        if r.stopped:
            break
    elapsed = time.perf_counter() - t0
    if produced < a.steps:
        log(f"warning: generation stopped after {produced} timed tokens")
    tok_s = produced / elapsed
    ms_step = 1000.0 * elapsed / produced
    log(f"decode: {produced} tokens in {elapsed * 1000:.1f} ms -> {tok_s:.1f} tok/s ({ms_step:.3f} ms/token)")

    _, timings = session.profile(cached, PROFILE_STEPS)
    session.close()
    # dominant kernel: the persistent step kernel (all 48 layers of one token), timed with a
    # hipEvent pair around every launch on the session stream
    n, ms, b = timings["layers"]
    avg_ms = ms / n
    kv_bytes = kv_read_bytes(model, len(cached))
    step_bytes = b + kv_bytes
    achieved = step_bytes / (avg_ms * 1e6)
    hn, hms, hb = timings["head"]
    per_token_bytes = step_bytes + hb
    log(f"  layers kernel: {n} launches, avg {1000 * avg_ms:.1f} us, {step_bytes / 1e9:.3f} GB "
        f"(weights {b / 1e9:.3f} + KV {kv_bytes / 1e6:.1f} MB) -> {achieved:.0f} GB/s")
    log(f"  head kernel:   {hn} launches, avg {1000 * hms / hn:.1f} us, {hb / 1e6:.1f} MB -> "
        f"{hb / (hms / hn * 1e6):.0f} GB/s")
    for name in ("qkv", "attention", "o_proj", "gate_up", "down", "barrier"):
        pn, pms, pb = timings[name]
        if pn:
            us = 1000.0 * pms / pn
            rate = f"{pb / (us * 1e3):8.1f} GB/s" if pb else ""
            marks = "  ".join(f"{k.split('.')[1]} {1000.0 * v[1] / v[0]:.2f}" for k, v in timings.items()
                              if k.startswith(name + ".") and v[0])
            log(f"    phase {name:10s} x{pn:5d}  avg {us:7.2f} us  {pb / 1e6:8.3f} MB  {rate}  [{marks}]")
    log(f"algorithmic bytes per token {per_token_bytes / 1e9:.3f} GB -> roofline {PEAK_GBS * 1e9 / per_token_bytes:.0f} "
        f"tok/s at 8 TB/s; measured {tok_s:.1f} tok/s = {tok_s * per_token_bytes / (PEAK_GBS * 1e9):.3f} of it")

    cpu = None
    if not a.no_cpu:
        threads = max(1, min(16, os.cpu_count() or 1))
        cv, cdt = cpu_baseline(model, prompt, a.cpu_tokens, threads)
        cpu = {"value": round(cv, 4), "unit": "tok/s", "cores": threads, "kind": "port",
               "sample": f"C oracle (FP64-accumulation port of the reference CPU path), full 48-layer model: "
                         f"{a.cpu_tokens} greedy decode tokens (layers + Q6_K head + argmax) after a 1-token "
                         f"prefill, {cdt:.1f} s on {threads} threads"}
        log(f"cpu baseline: {cv:.3f} tok/s on {threads} threads ({cdt:.1f} s)")

    line = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": produced,
        "warmup": a.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded random weights and prompt ids)",
        "config": {
            "workload": "config4: 48-layer Gemma-3-12B-shaped decode loop, Q4_0 projections + tied Q6_K "
                        "embedding/lm-head (vocab 262144), 128-token prompt prefill then greedy decode steps "
                        "(one persistent launch for the 48 layers + one head launch per token), fp16 KV cache",
            "hidden": 3840, "intermediate": 15360, "layers": 48, "q_heads": 16, "kv_heads": 8, "head_width": 256,
            "prompt_tokens": PROMPT, "decode_tokens": a.warmup + produced, "batch": 1,
            "algorithmic_bytes_per_token": round(per_token_bytes),
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "decode_step_kernel: all 48 layers of one token in one cooperative launch (Q4_0 "
                      "GEMVs on int8 MFMA, fused norms, GQA attention over fp16 KV)",
            "achieved": round(achieved, 1),
            "peak": PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_GBS, 4),
            "traffic": measured_traffic(),
            "traffic_source": "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE per launch, calibrated on a 256 MiB copy "
                              "(profiles/decode_step_kernel_config4.md)",
            "avg_us": round(1000.0 * avg_ms, 2),
            "bytes_per_launch": round(step_bytes),
            "launches": n,
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
