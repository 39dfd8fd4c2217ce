"""Batch-1 greedy decode benchmark on one MI355X, with the standalone
operators of configs 0-3 measured beside it.

Workload (the `value`): a 48-layer Gemma-3-12B-shaped model with seeded random weights (hidden
3840, FFN 15360, 16 q / 8 kv heads of width 256, 5:1 local(window 1024):global layers, Q4_0
projections, tied Q6_K embedding/lm-head over 262144 ids); a 128-token random prompt is
prefilled, then W warm-up and K timed greedy decode steps run through
GenerationSession::generate (per token: one persistent launch for all 48 layers, one launch for
the Q6_K head + greedy argmax, replayed as one hipGraph; ids come back through mapped host
memory).  A "step" is one decoded token; `value` is tokens per second over the K timed steps.

After the timed region, PROFILE_STEPS more decode steps run with a hipEvent pair around every
launch on the session stream (af_session_profile): the first half launch the step kernel plainly
(the roofline's average launch), the second half with its in-kernel phase timeline.

Configs 0-3 (`configs` in the JSON line): each operator launched through the C ABI, cycling
through copies of its weights (or KV cache) that together exceed 1 GiB, so the 256 MB Infinity
Cache cannot serve them; one pass over the copies is captured as a hipGraph and replayed between
a hipEvent pair, so the per-launch time includes the gaps between graph nodes (a few-microsecond
kernel reads slower here than in the rocprofv3 kernel trace under profiles/).

CPU baseline: the C oracle (a port of the reference's FP64 CPU path), on this host: config 4 on
all of the box's CPU share (16 threads at most) and on one core, configs 0-3 in both modes.

Beside the headline (`prefill`, `long_context`, `speculative` and `gemma4` in the JSON line): a
512-id prompt prefilled on the config-4 model through the batched layers (32 positions per weight
pass) and one step-kernel launch per position; config-4 decode after a 7620-id prompt; greedy
speculative decoding with prompt-lookup drafts on a copying
workload (config-4 shapes, local layers only, a prompt that repeats the model's own continuation),
against plain decoding of the same prompt; and a full-size Gemma-4-shaped model (the reference's own
model family: 512-wide global layers with one KV head and K as V), prefilled and decoded on the
per-operation kernels.

    python bench.py [--gpus 1] [--steps 240] [--warmup 16] [--no-cpu] [--no-configs] [--no-extras]
"""
import argparse
import ctypes
import json
import os
import platform
import statistics
import subprocess
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "batch-1 decode tok/s @12B-shape Q4_0; Q4_0 GEMV HBM GB/s vs 8 TB/s peak"
PEAK_GBS = 8000.0
PROMPT = 128
PROFILE_STEPS = 16
ROTATE_BYTES = 1 << 30   # weight / KV copies cycled per configuration
CPU_SHARE = 16           # host threads a one-GPU box grants
HIDDEN, INTER, VOCAB = 3840, 15360, 262144


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def cpu_model():
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                return line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    return platform.processor() or "unknown"


def host_threads():
    return max(1, min(CPU_SHARE, os.cpu_count() or 1))


# ---- GPU legs of configs 0-3 ---------------------------------------------------------------------

def timed_launches(launch, n_copies, passes, stream):
    """Per-launch milliseconds of `launch(i)` over the weight copies i < n_copies: the n_copies
    launches are captured in one hipGraph, replayed `passes` times between a hipEvent pair on
    `stream`, and the elapsed time is split evenly over the launches (so it includes the gaps
    between graph nodes, not the host's dispatch).  One warm pass runs first (it also allocates
    any scratch the entry points grow on first use, which a capture must not do)."""
    from adaforge_amd import hip
    for i in range(n_copies):
        launch(i)
    stream.synchronize()
    g = hip.Graph(stream, lambda: [launch(i) for i in range(n_copies)])
    g.launch(stream)
    stream.synchronize()
    out = []
    for _ in range(passes):
        a, b = hip.Event(), hip.Event()
        a.record(stream)
        g.launch(stream)
        b.record(stream)
        stream.synchronize()
        out.append(a.elapsed_ms(b) / n_copies)
    return out


def summary(ms, nbytes, copies, extra=None):
    mean, med = statistics.fmean(ms), statistics.median(ms)
    d = {"passes": len(ms), "copies": copies, "mean_us": round(1000 * mean, 2), "median_us": round(1000 * med, 2),
         "algorithmic_bytes": int(nbytes), "gbs": round(nbytes / (med * 1e6), 1),
         "frac": round(nbytes / (med * 1e6) / PEAK_GBS, 4)}
    if extra:
        d.update(extra)
    return d


def gpu_config0():
    """Q4_0 GEMV 4096x3840 (af_q4_gemv), algorithmic bytes W + x + y."""
    from adaforge_amd import _native as N, hip, synth
    rows, cols = 4096, 3840
    w = synth.q4("config0.W", cols, rows)
    nbytes = w.size + 4 * (cols + rows)
    copies = -(-ROTATE_BYTES // w.size)
    hs = []
    for _ in range(copies):
        h = N.P()
        N.check(N.lib().af_q4_upload(w.ctypes.data_as(N.u8p), w.size, cols, rows, ctypes.byref(h)))
        hs.append(h)
    x, y, s = hip.Buffer.from_numpy(synth.normal("config0.x", cols)), hip.Buffer(rows), hip.Stream()
    try:
        ms = timed_launches(lambda i: N.check(N.lib().af_q4_gemv(hs[i], x.ptr, y.ptr, s.handle)), copies, 5, s)
    finally:
        for h in hs:
            N.lib().af_q4_free(h)
    return summary(ms, nbytes, copies, {"kernel": "q4_gemv_kernel", "shape": [rows, cols]})


def gpu_config1():
    """FFN block 3840 -> 15360 -> 3840 (af_ffn_run: RMSNorm + gate/up + GELU, down + residual)."""
    from adaforge_amd import _native as N, hip, synth
    H, I = HIDDEN, INTER
    pre = synth.normal("config1.norm", H, 1.0, 0.1)
    gate, up, down = synth.q4("config1.gate", H, I), synth.q4("config1.up", H, I), synth.q4("config1.down", I, H)
    weights = gate.size + up.size + down.size
    nbytes = weights + 4 * (3 * H + 2 * I)  # + x, norm weights, y, and the activation written and read
    copies = -(-ROTATE_BYTES // weights)
    mk = lambda a, c, r: N.MatrixDesc(a.ctypes.data_as(N.u8p), a.size, c, r)
    desc = N.FfnDesc(N.RmsNormDesc(pre.ctypes.data_as(N.f32p), H, 1e-6), mk(gate, H, I), mk(up, H, I),
                     mk(down, I, H), N.RmsNormDesc(None, 0, 0.0), 1.0)
    hs = []
    for _ in range(copies):
        h = N.P()
        N.check(N.lib().af_ffn_create(ctypes.byref(desc), ctypes.byref(h)))
        hs.append(h)
    x, y, s = hip.Buffer.from_numpy(synth.normal("config1.x", H)), hip.Buffer(H), hip.Stream()
    try:
        ms = timed_launches(lambda i: N.check(N.lib().af_ffn_run(hs[i], x.ptr, y.ptr, s.handle)), copies, 10, s)
    finally:
        for h in hs:
            N.lib().af_ffn_free(h)
    return summary(ms, nbytes, copies, {"kernel": "q4_gemv_kernel x2 (gate/up + GELU, down + residual)",
                                        "weights_bytes": weights})


def gpu_config2():
    """Q6_K head 262144x3840 + greedy argmax (af_q6_gemv_argmax): weights + x + logits."""
    from adaforge_amd import _native as N, hip, synth
    w = synth.q6("config2.head", HIDDEN, VOCAB)
    nbytes = w.size + 4 * (HIDDEN + VOCAB)
    copies = max(2, -(-ROTATE_BYTES // w.size))
    hs = []
    for _ in range(copies):
        h = N.P()
        N.check(N.lib().af_q6_upload(w.ctypes.data_as(N.u8p), w.size, HIDDEN, VOCAB, ctypes.byref(h)))
        hs.append(h)
    x, lg, res, s = (hip.Buffer.from_numpy(synth.normal("config2.x", HIDDEN)), hip.Buffer(VOCAB),
                     hip.Buffer(2, np.uint32), hip.Stream())
    try:
        ms = timed_launches(lambda i: N.check(N.lib().af_q6_gemv_argmax(hs[i], x.ptr, lg.ptr, res.ptr, s.handle)),
                            copies, 20, s)
    finally:
        for h in hs:
            N.lib().af_q6_free(h)
    return summary(ms, nbytes, copies, {"kernel": "q6_head_kernel", "shape": [VOCAB, HIDDEN]})


def gpu_config3(ctx, kind):
    """GQA decode attention (af_attention_decode) at position ctx - 1 over an fp16 KV cache of N(0,1)
    values; algorithmic bytes = the visible K and V rows read."""
    from adaforge_amd import _native as N, hip, synth
    QH, KVH, D = 16, 8, 256
    window = 1024 if kind == "local" else 0
    ring = ctx
    visible = min(ctx, window) if window else ctx
    nbytes = visible * KVH * D * 2 * 2
    cache_bytes = KVH * ring * D * 2
    copies = max(2, min(256, -(-ROTATE_BYTES // (2 * cache_bytes))))
    tag = f"bench.config3.{kind}.{ctx}"
    kv = synth.normal(tag + ".kv", KVH * ring * D).astype(np.float16)
    first = hip.Buffer.from_numpy(kv.view(np.uint16))
    caches = []
    for _ in range(copies):
        kb, vb = hip.Buffer(KVH * ring * D, np.uint16), hip.Buffer(KVH * ring * D, np.uint16)
        hip.ok(hip.rt().hipMemcpy(kb.ptr, first.ptr, cache_bytes, hip.D2D))
        hip.ok(hip.rt().hipMemcpy(vb.ptr, first.ptr, cache_bytes, hip.D2D))
        caches.append((kb, vb))
    q = hip.Buffer.from_numpy(synth.normal(tag + ".q", QH * D))
    k = hip.Buffer.from_numpy(synth.normal(tag + ".k", KVH * D))
    v = hip.Buffer.from_numpy(synth.normal(tag + ".v", KVH * D))
    qn = hip.Buffer.from_numpy(synth.normal("config3.qnorm", D, 1.0, 0.1))
    kn = hip.Buffer.from_numpy(synth.normal("config3.knorm", D, 1.0, 0.1))
    out, s = hip.Buffer(QH * D), hip.Stream()
    factors = np.ones(D // 2, np.float32)
    base = 1e4 if kind == "local" else 1e6
    args = []
    for kb, vb in caches:
        args.append(N.AttentionArgs(q.ptr, k.ptr, v.ptr, qn.ptr, kn.ptr, 1e-6, 1e-6, 1e-6, 0,
                                    N.RopeDesc(D, base, factors.ctypes.data_as(N.f32p), 131072),
                                    N.AttentionConfigDesc(QH, KVH, D, window, 1.0 / 16.0), kb.ptr, vb.ptr, ring,
                                    ctx - 1, out.ptr))
    ms = timed_launches(lambda i: N.check(N.lib().af_attention_decode(ctypes.byref(args[i]), s.handle)), copies,
                        max(3, 512 // copies), s)
    del caches
    return summary(ms, nbytes, copies, {"kernel": "attention_kernel", "ctx": ctx, "window": window or None})


def gpu_configs():
    out = {}
    for name, fn in (("config0_q4_gemv", gpu_config0), ("config1_ffn", gpu_config1), ("config2_q6_head", gpu_config2)):
        t = time.perf_counter()
        out[name] = fn()
        log(f"  {name}: median {out[name]['median_us']} us -> {out[name]['gbs']} GB/s "
            f"({100 * out[name]['frac']:.1f} % of 8 TB/s) over {out[name]['copies']} copies "
            f"[{time.perf_counter() - t:.1f}s]")
    for ctx in (512, 4096, 32768):
        for kind in ("global", "local"):
            name = f"config3_attention_{kind}_{ctx}"
            out[name] = gpu_config3(ctx, kind)
            log(f"  {name}: median {out[name]['median_us']} us -> {out[name]['gbs']} GB/s")
    return out


# ---- CPU legs (the oracle: test infrastructure, timed here as the reference CPU path) --------------

def median_time(fn, runs):
    ts = []
    for _ in range(runs):
        t = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t)
    return statistics.median(ts)


def cpu_configs(threads):
    """Configs 0-3 on the oracle, one core and `threads` cores (median of 5 runs each)."""
    import oracle
    from adaforge_amd import synth
    out = {}
    w0, x0 = synth.q4("config0.W", 3840, 4096), synth.normal("config0.x", 3840)
    pre = synth.normal("config1.norm", HIDDEN, 1.0, 0.1)
    g, u, d = synth.q4("config1.gate", HIDDEN, INTER), synth.q4("config1.up", HIDDEN, INTER), synth.q4(
        "config1.down", INTER, HIDDEN)
    x1 = synth.normal("config1.x", HIDDEN)
    w2, x2 = synth.q6("config2.head", HIDDEN, VOCAB), synth.normal("config2.x", HIDDEN)
    jobs = {
        "config0_q4_gemv": lambda t: oracle.q4_matvec(w0, 3840, 4096, x0, threads=t),
        "config1_ffn": lambda t: oracle.ffn(pre, 1e-6, g, u, d, HIDDEN, INTER, None, 1e-6, 1.0, x1, threads=t),
        "config2_q6_head": lambda t: oracle.greedy(oracle.q6_matvec(w2, HIDDEN, VOCAB, x2, threads=t).astype(np.float32)),
    }
    for ctx in (512, 4096, 32768):
        for kind in ("global", "local"):
            rng = np.random.default_rng(ctx)
            q = rng.standard_normal(16 * 256).astype(np.float32)
            kv = rng.standard_normal(ctx * 8 * 256).astype(np.float16).astype(np.float32)
            window = 1024 if kind == "local" else None
            jobs[f"config3_attention_{kind}_{ctx}"] = (
                lambda t, q=q, kv=kv, window=window, ctx=ctx:
                oracle.attention(16, 8, 256, window, 1.0 / 16.0, q, kv, kv, ctx, ctx - 1, threads=t))
    for name, fn in jobs.items():
        one = median_time(lambda: fn(1), 5)
        many = median_time(lambda: fn(threads), 5)
        out[name] = {"one_core_ms": round(1000 * one, 3), "all_core_ms": round(1000 * many, 3), "cores": threads}
        log(f"  cpu {name}: 1 core {1000 * one:.2f} ms, {threads} cores {1000 * many:.2f} ms")
    return out


def cpu_decode(model, prompt, tokens, threads):
    """The oracle decoding `tokens` greedy tokens (48 layers + final norm + Q6_K head + greedy each)
    after a one-token prefill; returns tokens/s."""
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


# ---- the headline: config 4 -------------------------------------------------------------------------

TRAFFIC_JSON = os.path.join(ROOT, "profiles", "traffic_config4.json")
# the sources whose code the counted kernels run (a counter figure describes only the build it came from)
TRAFFIC_SOURCES = ["adaforge_amd/csrc/step.hip", "adaforge_amd/csrc/kernels.hip", "adaforge_amd/csrc/device.h",
                   "adaforge_amd/csrc/af_internal.h"]


def source_hashes():
    import hashlib
    out = {}
    for rel in TRAFFIC_SOURCES:
        with open(os.path.join(ROOT, rel), "rb") as f:
            out[rel] = hashlib.sha256(f.read()).hexdigest()[:16]
    return out


def measured_traffic(kernel="void af::decode_step_kernel<2, true>(af::StepArgs)"):
    """HBM bytes per launch from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE passes
    (profiles/traffic_config4.json, calibrated against a copy of known size), or None when the file
    is missing or was measured on other kernel sources than these (their hashes are stored in it)."""
    try:
        with open(TRAFFIC_JSON) as f:
            t = json.load(f)
        if t.get("sources") != source_hashes():
            return None
        return t["kernels"][kernel]["hbm_bytes"]
    except (OSError, KeyError, ValueError):
        return None


def write_traffic(fetch_csv, write_csv, cal_fetch_csv, cal_write_csv, copy_bytes=1 << 28):
    """profiles/traffic_config4.json from rocprofv3 --pmc runs (one counter per run): per kernel the mean
    FETCH_SIZE and WRITE_SIZE per dispatch (KiB), each scaled by what the same counter reads for one
    device-to-device copy of copy_bytes (the largest copy dispatch of the calibration runs), and the
    hashes of the kernel sources measured."""
    import csv

    def per_kernel(path):
        acc = {}
        with open(path) as f:
            for row in csv.DictReader(f):
                acc.setdefault(row["Kernel_Name"], []).append(float(row["Counter_Value"]))
        return acc

    cal_f = max(max(v) for k, v in per_kernel(cal_fetch_csv).items() if "copy" in k.lower())
    cal_w = max(max(v) for k, v in per_kernel(cal_write_csv).items() if "copy" in k.lower())
    ff, wf = copy_bytes / 1024.0 / cal_f, copy_bytes / 1024.0 / cal_w
    fetch, write = per_kernel(fetch_csv), per_kernel(write_csv)
    kernels = {}
    for name in ("void af::decode_step_kernel<2, true>(af::StepArgs)", "void af::q6_head_kernel<2>(af::HeadArgs)"):
        if name in fetch and name in write:
            fk, wk = statistics.mean(fetch[name]), statistics.mean(write[name])
            kernels[name] = {"dispatches": len(fetch[name]), "fetch_kib": round(fk, 1), "write_kib": round(wk, 1),
                             "hbm_bytes": int(round((fk * ff + wk * wf) * 1024))}
    out = {"calibration": {"copy_bytes": copy_bytes, "fetch_kib": round(cal_f, 1), "write_kib": round(cal_w, 1),
                           "fetch_factor": round(ff, 4), "write_factor": round(wf, 4)},
           "sources": source_hashes(), "kernels": kernels}
    with open(TRAFFIC_JSON, "w") as f:
        json.dump(out, f, indent=1)
    print(json.dumps(out, indent=1))


def kv_read_bytes(model, tokens):
    """fp16 K and V rows one decode step reads at context `tokens` (window-limited layers)."""
    total = 0
    for L in model.layers:
        vis = min(tokens, L.window) if L.window else tokens
        total += vis * L.kv_heads * L.head_width * 2 * 2
    return total


def open_env(model, capacity, **env):
    """A session opened with the given AF_* switches set (restored afterwards)."""
    from adaforge_amd.backend import HipDiagnostics
    saved = {k: os.environ.get(k) for k in env}
    os.environ.update({k: str(v) for k, v in env.items()})
    try:
        return HipDiagnostics().open_session(model, capacity)
    finally:
        for k, v in saved.items():
            if v is None:
                del os.environ[k]
            else:
                os.environ[k] = v


def prefill_leg(model, stop, tokens=512):
    """Prefill of a `tokens`-id prompt on the config-4 model: batched (32 positions per weight pass,
    the default) against one step-kernel launch per position (AF_PREFILL_BATCH=0); the first generated
    id must agree."""
    from adaforge_amd import synth
    prompt = [int(i) for i in synth.prompt_ids(tokens, model.vocabulary, name="config4.prefill")]
    out = {"prompt_tokens": tokens}
    first = {}
    for name, batch in (("batched", 32), ("stepwise", 0)):
        with open_env(model, tokens + 8, AF_PREFILL_BATCH=batch) as s:
            s.generate(prompt[:40], stop, 1)  # allocations and graph warm-up
            s.reset()
            r = s.generate(prompt, stop, 1)
        ms = r.stats.prefill_ms
        first[name] = r.ids
        out[name] = {"ms": round(ms, 2), "tok_s": round((tokens - 1) / ms * 1000.0, 1)}
        log(f"prefill {tokens} tokens ({name}): {ms:.1f} ms -> {out[name]['tok_s']} tok/s")
    out["same_first_id"] = first["batched"] == first["stepwise"]
    return out


def speculative_leg(lead_tokens=160, new_tokens=128):
    """Greedy speculative decoding (AF_SPECULATIVE=1) on a copying workload: the config-4 shapes
    with every layer local (window 4, so each position depends on at most the 145 before it), and a
    prompt lead + G + lead where G is the model's own greedy continuation of lead, so that the
    continuation repeats G and prompt lookup drafts it.  Decode tok/s with and without speculation;
    the ids must agree."""
    from adaforge_amd import synth
    model = synth.model(name="config4-local", window=4, global_every=1000)
    stop = [model.vocabulary - 1]
    lead = [int(i) for i in synth.prompt_ids(lead_tokens, model.vocabulary, name="spec.lead")]
    cap = 2 * lead_tokens + 2 * new_tokens + 8
    with open_env(model, cap) as s:
        g = s.generate(lead, stop, new_tokens).ids
    prompt = lead + g + lead
    out = {"workload": f"48 local layers (window 4) of the config-4 shapes, prompt = {lead_tokens} ids + the "
                       f"model's {new_tokens}-id greedy continuation of them + the {lead_tokens} ids again, "
                       f"{new_tokens} new ids"}
    ids = {}
    for name, spec in (("plain", 0), ("speculative", 1)):
        with open_env(model, cap, AF_SPECULATIVE=spec) as s:
            r = s.generate(prompt, stop, new_tokens)
            st = s.speculation()
        tok_s = r.stats.decode_tokens / r.stats.decode_ms * 1000.0
        ids[name] = r.ids
        out[name] = {"decode_tok_s": round(tok_s, 1)}
        if spec:
            out[name].update({"passes": st[0], "drafted": st[1], "accepted": st[2]})
        log(f"copying workload ({name}): {tok_s:.1f} tok/s {out[name]}")
    out["same_ids"] = ids["plain"] == ids["speculative"]
    out["speedup"] = round(out["speculative"]["decode_tok_s"] / out["plain"]["decode_tok_s"], 2)
    return out


def long_context_leg(model, stop, tokens=7620, new_tokens=64):
    """Decode on the config-4 model at a long context: a `tokens`-id prompt prefilled through the
    batched layers, then greedy decode (the global layers attend over every position, the local
    ones over their 1024-token window); prefill tok/s and decode tok/s."""
    from adaforge_amd import synth
    prompt = [int(i) for i in synth.prompt_ids(tokens, model.vocabulary, name="config4.long")]
    with open_env(model, tokens + new_tokens + 32) as s:
        r = s.generate(prompt, stop, 8)
        prefill_ms = r.stats.prefill_ms
        cached = prompt + r.ids
        t0 = time.perf_counter()
        r = s.generate(cached, stop, new_tokens)
        dt = time.perf_counter() - t0
    out = {"prompt_tokens": tokens, "prefill_ms": round(prefill_ms, 1),
           "prefill_tok_s": round((tokens - 1) / prefill_ms * 1000.0, 1),
           "context": len(cached), "decode_tokens": len(r.ids), "decode_tok_s": round(len(r.ids) / dt, 1)}
    log(f"long context: prefill {tokens} ids in {prefill_ms:.0f} ms, decode {len(r.ids)} tokens at context "
        f"{len(cached)} -> {out['decode_tok_s']} tok/s")
    return out


def gemma4_leg(new_tokens=256):
    """The reference's own model family at full size: a 48-layer Gemma-4-shaped model with seeded
    random weights (local layers as config 4; every sixth layer global with 16 query heads on one KV
    head of width 512, K reused as V, proportional RoPE; attention scale 1, V-norm, softcap 30).  Its
    512-wide global layers are outside the persistent step kernel's limits: the step kernel takes the
    five-layer runs of local layers between them (one launch per run) and the per-operation kernels
    the global layers, launched directly (no graph: the same rate).  Batched prefill of 128 ids, then greedy decode
    in 128-token turns; decode tok/s over the turns."""
    from adaforge_amd import synth
    model = synth.gemma4_model(name="gemma4-bench", layers=48, hidden=HIDDEN, intermediate=INTER,
                               local_q=(16, 8, 256), global_q=(16, 1, 512), vocabulary=VOCAB, window=1024)
    stop = [model.vocabulary - 1]
    prompt = [int(i) for i in synth.prompt_ids(PROMPT, model.vocabulary, name="gemma4-bench.prompt")]
    with open_env(model, PROMPT + new_tokens + 32) as s:
        r = s.generate(prompt, stop, 16)
        prefill_ms = r.stats.prefill_ms
        cached = prompt + r.ids
        produced, t0 = 0, time.perf_counter()
        while produced < new_tokens:
            r = s.generate(cached, stop, min(128, new_tokens - produced))
            cached += r.ids
            produced += len(r.ids)
            if r.stopped:
                break
        dt = time.perf_counter() - t0
    out = {"workload": "48-layer Gemma-4-shaped model (local layers 16 q / 8 kv x 256, window 1024; every "
                       "sixth layer global: 16 q / 1 kv x 512, K as V, proportional RoPE; scale 1, V-norm, "
                       "softcap 30), Q4_0 projections, tied Q6_K table (vocab 262144); the step kernel "
                       "over each run of local layers, the per-operation kernels on the global layers, "
                       "launched directly (no graph)",
           "prompt_tokens": PROMPT, "prefill_ms": round(prefill_ms, 2),
           "prefill_tok_s": round((PROMPT - 1) / prefill_ms * 1000.0, 1),
           "decode_tokens": produced, "decode_tok_s": round(produced / dt, 1)}
    log(f"gemma4-shaped model: prefill {PROMPT} in {prefill_ms:.1f} ms, decode {produced} tokens -> "
        f"{out['decode_tok_s']} tok/s")
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=240)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--cpu-tokens", type=int, default=4)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-configs", action="store_true", help="skip the configs 0-3 operator legs")
    ap.add_argument("--configs-only", action="store_true", help="only the configs 0-3 GPU legs (profiling)")
    ap.add_argument("--no-extras", action="store_true", help="skip the prefill and speculative-decoding legs")
    ap.add_argument("--traffic", nargs=4, metavar=("FETCH_CSV", "WRITE_CSV", "CAL_FETCH_CSV", "CAL_WRITE_CSV"),
                    help="write profiles/traffic_config4.json from rocprofv3 --pmc counter CSVs and exit")
    ap.add_argument("--legs", default="prefill,long,speculative,gemma4",
                    help="the extra legs to run (comma-separated subset of prefill, long, speculative, gemma4)")
    a = ap.parse_args()
    if a.traffic:
        write_traffic(*a.traffic)
        return
    if a.gpus != 1:
        print(f"bench.py measures one GPU: the batch-1 decode path runs on a single MI355X "
              f"(--gpus {a.gpus} is not supported: one process, one GPU)", file=sys.stderr)
        sys.exit(2)
    if a.steps < 1 or a.warmup < 1:
        sys.exit("--steps and --warmup must be >= 1")
    legs = set() if a.no_extras else {x for x in a.legs.split(",") if x}
    if legs - {"prefill", "long", "speculative", "gemma4"}:
        sys.exit(f"--legs: unknown leg(s) {sorted(legs - {'prefill', 'long', 'speculative', 'gemma4'})}")

    from adaforge_amd import synth
    from adaforge_amd.backend import HipDiagnostics

    diag = HipDiagnostics()
    dev = diag.check()
    log(f"device {dev.device_name} {dev.arch} CUs={dev.compute_units}")
    if a.configs_only:
        print(json.dumps(gpu_configs()), flush=True)
        return

    t = time.perf_counter()
    model = synth.model()
    log(f"model generated in {time.perf_counter() - t:.1f}s")
    prompt = [int(i) for i in synth.prompt_ids(PROMPT, model.vocabulary, name="config4.prompt")]
    stop = [model.vocabulary - 1]
    capacity = PROMPT + a.warmup + a.steps + PROFILE_STEPS + 2
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
    # dominant kernel: the persistent step kernel (all 48 layers of one token), plain launches timed
    # with a hipEvent pair around each on the session stream
    n, ms, b = timings["layers"]
    avg_ms = ms / n
    kv_bytes = kv_read_bytes(model, len(cached))
    step_bytes = b + kv_bytes
    achieved = step_bytes / (avg_ms * 1e6)
    tn, tms, _ = timings["layers_timeline"]
    hn, hms, hb = timings["head"]
    per_token_bytes = step_bytes + hb
    log(f"  layers kernel: {n} plain launches, avg {1000 * avg_ms:.1f} us, {step_bytes / 1e9:.3f} GB "
        f"(weights {b / 1e9:.3f} + KV {kv_bytes / 1e6:.1f} MB) -> {achieved:.0f} GB/s; "
        f"{tn} launches with the timeline avg {1000 * tms / max(tn, 1):.1f} us")
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

    configs = None
    if not a.no_configs:
        configs = gpu_configs()

    prefill = spec = gemma4 = longctx = None
    if "prefill" in legs:
        prefill = prefill_leg(model, stop)
    if "long" in legs:
        longctx = long_context_leg(model, stop)
    if "speculative" in legs:
        spec = speculative_leg()
    if "gemma4" in legs:
        gemma4 = gemma4_leg()

    cpu = None
    if not a.no_cpu:
        threads = host_threads()
        model_name, nproc = cpu_model(), os.cpu_count()
        cv, cdt = cpu_decode(model, prompt, a.cpu_tokens, threads)
        log(f"cpu baseline: {cv:.3f} tok/s on {threads} threads ({cdt:.1f} s)")
        c1, c1dt = cpu_decode(model, prompt, 1, 1)
        log(f"cpu baseline, one core: {c1:.4f} tok/s ({c1dt:.1f} s)")
        cpu = {"value": round(cv, 4), "unit": "tok/s", "cores": threads, "kind": "port",
               "sample": f"C oracle (FP64-accumulation port of the reference CPU path), full 48-layer model: "
                         f"{a.cpu_tokens} greedy decode tokens (layers + Q6_K head + argmax) after a 1-token "
                         f"prefill, {cdt:.1f} s on {threads} threads (rows split across threads, per-row order "
                         f"unchanged)",
               "one_core": {"value": round(c1, 5), "unit": "tok/s", "cores": 1,
                            "sample": f"1 greedy decode token after a 1-token prefill, {c1dt:.1f} s on one thread"},
               "nproc": nproc, "cpu_model": model_name}
        if configs is not None:
            cpu["configs"] = cpu_configs(threads)

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
                        "(one persistent launch for the 48 layers + one head launch per token, replayed as a "
                        "hipGraph), fp16 KV cache",
            "hidden": 3840, "intermediate": 15360, "layers": 48, "q_heads": 16, "kv_heads": 8, "head_width": 256,
            "prompt_tokens": PROMPT, "decode_tokens": a.warmup + produced, "batch": 1,
            "algorithmic_bytes_per_token": round(per_token_bytes),
            "tok_s_roofline_frac": round(tok_s * per_token_bytes / (PEAK_GBS * 1e9), 4),
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "decode_step_kernel: all 48 layers of one token in one persistent launch of one "
                      "workgroup per CU (Q4_0 GEMVs on int8 MFMA, fused norms, GQA attention over fp16 KV)",
            "achieved": round(achieved, 1),
            "peak": PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_GBS, 4),
            "traffic": measured_traffic(),
            "traffic_source": "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE per launch, calibrated on a 256 MiB copy "
                              "(profiles/decode_step_kernel_config4.md); null when the committed figures were "
                              "measured on other kernel sources than this build's",
            "avg_us": round(1000.0 * avg_ms, 2),
            "bytes_per_launch": round(step_bytes),
            "launches": n,
            "timeline_avg_us": round(1000.0 * tms / max(tn, 1), 2),
        },
        "configs": configs,
        "prefill": prefill,
        "long_context": longctx,
        "speculative": spec,
        "gemma4": gemma4,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
