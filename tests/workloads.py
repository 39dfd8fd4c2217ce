"""The BASELINE configurations as seeded inputs (shared by tests, fixtures and the bench's
parity legs).  Shapes and distributions follow BASELINE.json's `configs`."""
import numpy as np

import oracle
from adaforge_amd import synth

# config 0: single Q4_0 GEMV
C0_ROWS, C0_COLS = 4096, 3840
# config 1: FFN block
C1_HIDDEN, C1_INTER = 3840, 15360
# config 2: Q6_K lm-head
C2_ROWS, C2_COLS = 262144, 3840
# config 3: GQA decode attention
C3_Q_HEADS, C3_KV_HEADS, C3_WIDTH = 16, 8, 256
C3_CONTEXTS = (512, 4096, 32768)
C3_WINDOW = 1024
# config 4: 48-layer decode loop
C4_PROMPT, C4_DECODE = 128, 256


def config0():
    w = synth.q4("config0.W", C0_COLS, C0_ROWS)
    xs = [np.zeros(C0_COLS, np.float32), synth.ramp(C0_COLS), synth.normal("config0.x", C0_COLS)]
    return w, xs


def config1():
    H, I = C1_HIDDEN, C1_INTER
    return {"hidden": H, "inter": I, "pre": synth.normal("config1.norm", H, 1.0, 0.1),
            "gate": synth.q4("config1.gate", H, I), "up": synth.q4("config1.up", H, I),
            "down": synth.q4("config1.down", I, H), "x": synth.normal("config1.x", H)}


def config2():
    return synth.q6("config2.head", C2_COLS, C2_ROWS), synth.normal("config2.x", C2_COLS)


def config3(ctx, kind, v_norm=False):
    """One decode step at position ctx - 1 with ctx - 1 cached tokens of N(0,1) fp16 K/V.

    Returns a dict with raw q/k/v for the new token, q/k norm weights, RoPE base, the window,
    the fp16 cache contents for positions 0..ctx-2 ([ctx-1][kv_heads][width] float32 values)."""
    W, KVH, QH = C3_WIDTH, C3_KV_HEADS, C3_Q_HEADS
    tag = f"config3.{kind}.{ctx}"
    hist = ctx - 1
    keys = synth.normal(tag + ".K", hist * KVH * W).astype(np.float16).astype(np.float32)
    values = synth.normal(tag + ".V", hist * KVH * W).astype(np.float16).astype(np.float32)
    return {"ctx": ctx, "kind": kind, "window": C3_WINDOW if kind == "local" else None,
            "base": 1e4 if kind == "local" else 1e6, "scale": 1.0 / 16.0, "v_norm": v_norm,
            "q": synth.normal(tag + ".q", QH * W), "k": synth.normal(tag + ".k", KVH * W),
            "v": synth.normal(tag + ".v", KVH * W), "q_norm": synth.normal("config3.qnorm", W, 1.0, 0.1),
            "k_norm": synth.normal("config3.knorm", W, 1.0, 0.1), "keys": keys, "values": values, "eps": 1e-6}


def config3_new_kv(case):
    """The oracle's new K and V for the case (normed, rotated, fp16-rounded), stack.rs:683-690."""
    W = C3_WIDTH
    pos = case["ctx"] - 1
    f = np.ones(W // 2, np.float32)
    k = oracle.rmsnorm(case["k_norm"], case["eps"], case["k"]).astype(np.float32)
    k = oracle.rope(W, case["base"], f, 131072, k, pos).astype(np.float32)
    v = case["v"]
    if case["v_norm"]:
        v = oracle.rmsnorm(np.ones(W, np.float32), case["eps"], v).astype(np.float32)
    return k.astype(np.float16).astype(np.float32), np.asarray(v, np.float32).astype(np.float16).astype(np.float32)


def config3_reference(case):
    """Oracle attention output (float64 [q_heads * width]) for a config-3 case."""
    W = C3_WIDTH
    pos = case["ctx"] - 1
    f = np.ones(W // 2, np.float32)
    q = oracle.rmsnorm(case["q_norm"], case["eps"], case["q"]).astype(np.float32)
    q = oracle.rope(W, case["base"], f, 131072, q, pos).astype(np.float32)
    k, v = config3_new_kv(case)
    keys = np.concatenate([case["keys"], k])
    values = np.concatenate([case["values"], v])
    return oracle.attention(C3_Q_HEADS, C3_KV_HEADS, W, case["window"], case["scale"], q, keys, values, pos + 1, pos)
