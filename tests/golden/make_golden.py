"""Writes the golden fixtures under tests/golden/ from the C oracle (CPU, this repository's
restatement of AdaForge's FP64 oracles).  Inputs come from the seeded generators in
adaforge_amd/synth.py, so any host regenerates identical inputs.

    python tests/golden/make_golden.py            # configs 0-3 (seconds)
    python tests/golden/make_golden.py --config4  # + the 48-layer decode (~15 min on 8 cores)
"""
import argparse
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle  # noqa: E402
from adaforge_amd import synth  # noqa: E402
from tests import workloads  # noqa: E402


def dump(name, obj):
    path = os.path.join(HERE, name)
    with open(path, "w") as f:
        json.dump(obj, f, indent=1)
        f.write("\n")
    print("wrote", path)


def f64list(a):
    return [float(v) for v in a]


def config0():
    w, xs = workloads.config0()
    out = {"shape": [workloads.C0_ROWS, workloads.C0_COLS], "inputs": ["zero", "ramp", "normal"], "rows": {}}
    for name, x in zip(out["inputs"], xs):
        y = oracle.q4_matvec(w, workloads.C0_COLS, workloads.C0_ROWS, x)
        out["rows"][name] = {"first64": f64list(y[:64]), "last64": f64list(y[-64:]),
                             "sum": float(y.sum()), "sumabs": float(np.abs(y).sum())}
    dump("config0_q4_gemv.json", out)


def config1():
    f = workloads.config1()
    y = oracle.ffn(f["pre"], 1e-6, f["gate"], f["up"], f["down"], f["hidden"], f["inter"], None, 1e-6, 1.0, f["x"])
    dump("config1_ffn.json", {"hidden": f["hidden"], "intermediate": f["inter"], "first64": f64list(y[:64]),
                              "last64": f64list(y[-64:]), "sum": float(y.sum()), "sumabs": float(np.abs(y).sum())})


def config2():
    w, x = workloads.config2()
    y = oracle.q6_matvec(w, workloads.C2_COLS, workloads.C2_ROWS, x)
    y32 = y.astype(np.float32)
    top = np.argsort(-y32, kind="stable")[:8]
    dump("config2_q6_head.json", {"shape": [workloads.C2_ROWS, workloads.C2_COLS], "argmax": oracle.greedy(y32),
                                  "top8_ids": [int(i) for i in top], "top8_logits": f64list(y[top]),
                                  "margin": float(y32[top[0]] - y32[top[1]]), "sum": float(y.sum())})


def config3():
    out = {}
    for ctx in workloads.C3_CONTEXTS:
        for kind in ("global", "local"):
            case = workloads.config3(ctx, kind)
            y = workloads.config3_reference(case)
            out[f"{kind}-{ctx}"] = {"first64": f64list(y[:64]), "sum": float(y.sum()),
                                    "sumabs": float(np.abs(y).sum())}
    dump("config3_attention.json", out)


def config4(threads, top=8):
    """The oracle's greedy run (or_model_generate's order: each step's logits, f32 greedy, then the
    id is consumed) with each step's top `top` ids by f32 logit and their f64 logits."""
    model = synth.model()
    prompt = synth.prompt_ids(workloads.C4_PROMPT, model.vocabulary, name="config4.prompt")
    ref = oracle.Model(model, capacity=workloads.C4_PROMPT + workloads.C4_DECODE + 1, threads=threads)
    t = time.time()
    for tok in prompt:
        ref.step(int(tok))
    ids, margins, top_ids, top_logits = [], [], [], []
    for _ in range(workloads.C4_DECODE):
        logits = ref.logits()
        l32 = logits.astype(np.float32)
        tok = oracle.greedy(l32)
        order = np.argsort(-l32, kind="stable")[:top]
        second = np.max(np.delete(l32, tok))
        ids.append(int(tok))
        margins.append(float(l32[tok] - second))
        top_ids.append([int(i) for i in order])
        top_logits.append(f64list(logits[order]))
        ref.step(tok)
    ref.close()
    dump("config4_decode.json", {"prompt": [int(i) for i in prompt], "tokens": ids, "stopped": False,
                                 "margins": margins, "top_ids": top_ids, "top_logits": top_logits,
                                 "distinct": len(set(ids)), "oracle_seconds": time.time() - t,
                                 "threads": threads})


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--config4", action="store_true")
    ap.add_argument("--only4", action="store_true")
    ap.add_argument("--threads", type=int, default=os.cpu_count() or 1)
    a = ap.parse_args()
    if not a.only4:
        config0()
        config1()
        config2()
        config3()
    if a.config4 or a.only4:
        config4(a.threads)
