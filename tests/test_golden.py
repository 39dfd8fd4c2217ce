"""The committed golden fixtures (tests/golden/*.json, written by tests/golden/make_golden.py
from the C oracle) against the oracle as it builds now: a change to the oracle or to the seeded
generators that moves any BASELINE configuration shows up here, on the CPU."""
import json
import os

import numpy as np
import pytest

import oracle
from tests import workloads as W

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    with open(os.path.join(HERE, name)) as f:
        return json.load(f)


def close(a, b):
    np.testing.assert_allclose(np.asarray(a, np.float64), np.asarray(b, np.float64), rtol=1e-12, atol=1e-15)


def test_config0_fixture():
    g = load("config0_q4_gemv.json")
    w, xs = W.config0()
    for name, x in zip(g["inputs"], xs):
        y = oracle.q4_matvec(w, W.C0_COLS, W.C0_ROWS, x)
        r = g["rows"][name]
        close(y[:64], r["first64"])
        close(y[-64:], r["last64"])
        close(y.sum(), r["sum"])


def test_config1_fixture():
    g = load("config1_ffn.json")
    f = W.config1()
    y = oracle.ffn(f["pre"], 1e-6, f["gate"], f["up"], f["down"], f["hidden"], f["inter"], None, 1e-6, 1.0, f["x"])
    close(y[:64], g["first64"])
    close(y[-64:], g["last64"])


def test_config2_fixture():
    g = load("config2_q6_head.json")
    w, x = W.config2()
    y = oracle.q6_matvec(w, W.C2_COLS, W.C2_ROWS, x)
    assert oracle.greedy(y.astype(np.float32)) == g["argmax"]
    close(y[g["top8_ids"]], g["top8_logits"])


@pytest.mark.parametrize("ctx", W.C3_CONTEXTS[:2])
def test_config3_fixture(ctx):
    g = load("config3_attention.json")
    for kind in ("global", "local"):
        y = W.config3_reference(W.config3(ctx, kind))
        close(y[:64], g[f"{kind}-{ctx}"]["first64"])


def test_config4_fixture_is_consistent():
    """The 48-layer fixture is too slow to regenerate in the CPU suite (about half an hour);
    check its shape and the prompt it was made from."""
    path = os.path.join(HERE, "config4_decode.json")
    if not os.path.exists(path):
        pytest.skip("config4 fixture not generated")
    g = load("config4_decode.json")
    from adaforge_amd import synth
    prompt = synth.prompt_ids(W.C4_PROMPT, 262144, name="config4.prompt")
    assert g["prompt"] == [int(i) for i in prompt]
    assert len(g["tokens"]) == W.C4_DECODE and len(g["margins"]) == W.C4_DECODE
    assert all(0 <= t < 262144 for t in g["tokens"]) and not g["stopped"]
    # a varied greedy path (a model that repeats one id checks nothing about positions and caches)
    assert len(set(g["tokens"])) >= 32 and g["distinct"] == len(set(g["tokens"]))
    # per-step top-8: the chosen id first, f32 logits descending, margins from the same values
    for k, (tok, ids, lg, m) in enumerate(zip(g["tokens"], g["top_ids"], g["top_logits"], g["margins"])):
        l32 = np.asarray(lg, np.float64).astype(np.float32)
        assert ids[0] == tok and len(set(ids)) == len(ids) == 8, k
        assert np.all(np.diff(l32) <= 0), k
        assert abs(float(l32[0] - l32[1]) - m) <= 1e-6 * max(1.0, abs(float(l32[0]))), k
