"""Batched prefill on the GPU against the CPU oracle: the batched Q4_0 GEMV (af_q4_gemm: up to 32
vectors per weight pass, crates/cuda-backend/src/batch.rs:113-148, MAX_BATCH at batch.rs:10), every
vector within the matvec tolerance |gpu - ref| <= 1e-4 + 1e-4 |ref| (crates/cuda-backend/src/
matvec.rs:175-193); and whole prompts through the batched layers (stack.rs:1063-1099 consume_batch),
teacher-forced per layer and by greedy ids."""
import ctypes
import os

import numpy as np
import pytest

import oracle
from adaforge_amd import _native as N, hip, synth
from adaforge_amd.backend import HipDiagnostics

pytestmark = pytest.mark.gpu


def gemm(w, columns, rows, xs):
    h = N.P()
    N.check(N.lib().af_q4_upload(w.ctypes.data_as(N.u8p), w.size, columns, rows, ctypes.byref(h)))
    try:
        xb, yb = hip.Buffer.from_numpy(np.ascontiguousarray(xs, np.float32)), hip.Buffer(len(xs) * rows)
        N.check(N.lib().af_q4_gemm(h, xb.ptr, len(xs), yb.ptr, None))
        hip.synchronize()
        return yb.numpy().reshape(len(xs), rows)
    finally:
        N.lib().af_q4_free(h)


@pytest.mark.parametrize("tokens", [1, 3, 4, 5, 17, 32])
def test_batched_gemv_matches_oracle_per_vector(tokens):
    cols, rows = 3840, 4096
    w = synth.q4("config0.W", cols, rows)
    rng = np.random.default_rng(tokens)
    xs = rng.standard_normal((tokens, cols)).astype(np.float32)
    xs[0] *= np.float32(0.0) if tokens > 1 else np.float32(1.0)
    y = gemm(w, cols, rows, xs)
    for t in range(tokens):
        oracle.compare(oracle.q4_matvec(w, cols, rows, xs[t]), y[t])
    if tokens > 1:
        assert np.all(y[0] == 0.0)


@pytest.mark.parametrize("columns,rows,tokens", [(32, 5, 7), (96, 77, 32), (640, 77, 9), (15360, 3843, 6),
                                                 (2560, 10240 + 16, 32)])
def test_batched_gemv_ragged_shapes(columns, rows, tokens):
    w = synth.q4(f"bg{columns}x{rows}", columns, rows, signed=True)
    rng = np.random.default_rng(columns + rows)
    xs = (rng.standard_normal((tokens, columns)) * np.exp2(rng.integers(-20, 8, (tokens, columns)))).astype(np.float32)
    y = gemm(w, columns, rows, xs)
    for t in range(tokens):
        oracle.compare(oracle.q4_matvec(w, columns, rows, xs[t]), y[t])


def test_batched_gemv_rejects_empty_and_oversized_batches():
    cols, rows = 64, 16
    w = synth.q4("bgrej", cols, rows)
    h = N.P()
    N.check(N.lib().af_q4_upload(w.ctypes.data_as(N.u8p), w.size, cols, rows, ctypes.byref(h)))
    try:
        xb, yb = hip.Buffer(33 * cols), hip.Buffer(33 * rows)
        for tokens in (0, 33):
            with pytest.raises(N.AfError):
                N.check(N.lib().af_q4_gemm(h, xb.ptr, tokens, yb.ptr, None))
    finally:
        N.lib().af_q4_free(h)


# ---- batched prefill: every prompt position through the layers 32 at a time -------------------------

THREADS = max(1, min(16, os.cpu_count() or 1))


def open_with_env(model, capacity, **env):
    """A session opened with the given AF_* environment switches set (restored afterwards)."""
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


def batch_model(q_heads, kv_heads, window, name):
    """Three layers (local, local, global), hidden 1024, FFN 2048, head width 256."""
    return synth.model(name=name, layers=3, hidden=1024, intermediate=2048, q_heads=q_heads, kv_heads=kv_heads,
                       head_width=256, vocabulary=2048, window=window, global_every=3)


@pytest.mark.parametrize("q_heads,kv_heads,window,n,batch", [
    (16, 8, 16, 80, 32),    # BASELINE head geometry; the window-16 ring (48 slots) wraps inside a batch
    (16, 4, 64, 150, 32),   # four query heads per KV head; attention chunks past 32 positions
    (8, 8, 24, 45, 7),      # one query head per KV head, ragged batches of 7
])
def test_batched_trace_teacher_forced(q_heads, kv_heads, window, n, batch):
    """Every layer output and appended K/V of a batched prefill (AF_TRACE_BATCH: af_session_trace
    through the batched layers) against the oracle, teacher-forced on the GPU's own layer inputs."""
    model = batch_model(q_heads, kv_heads, window, name=f"batch{q_heads}x{kv_heads}")
    ids = [int(i) for i in synth.prompt_ids(n, model.vocabulary, name=f"batch{n}.ids")]
    kv_rows = kv_heads * 256
    with open_with_env(model, n + 8, AF_TRACE_BATCH=batch) as s:
        outputs, kv, logits, hidden = s.trace(ids, kv_rows=kv_rows)
    marks = {0, 1, batch - 1, batch, batch + 1, window - 1, window, window + 1, 2 * batch - 1, 2 * batch, 63, 64,
             n - 2, n - 1}
    positions = sorted(p for p in marks if 0 <= p < n)
    ratio, ulps, differ = oracle.check_layer_stack(model, ids, outputs, kv, threads=THREADS, positions=positions)
    print(f"batched trace {q_heads}x{kv_heads} n={n} batch={batch}: layer ratio {ratio:.3f}, K/V ratio {ulps:.3f}, "
          f"{differ} fp16 values differ", flush=True)
    # the logits after the last id, from the batch's last hidden state
    nrm = oracle.rmsnorm(model.final_norm, model.final_eps, hidden).astype(np.float32)
    oracle.compare(oracle.q6_matvec(model.table, model.hidden, model.vocabulary, nrm, threads=THREADS), logits)


def test_batched_trace_gemma4_width_512_shared_v():
    """Gemma 4 geometry through the batched layers: global layer of one width-512 KV head for 16 query
    heads with K's weights reused as V, proportional RoPE factors, unit-weight V RMSNorm."""
    model = synth.gemma4_model(name="gemma4-batch", layers=6, hidden=1024, intermediate=2048, local_q=(16, 8, 256),
                               global_q=(16, 1, 512), vocabulary=2048, window=16)
    n = 70
    ids = [int(i) for i in synth.prompt_ids(n, model.vocabulary, name="gemma4-batch.ids")]
    kv_rows = max(L.kv_heads * L.head_width for L in model.layers)
    with open_with_env(model, n + 8, AF_TRACE_BATCH=32) as s:
        outputs, kv, _, _ = s.trace(ids, kv_rows=kv_rows, logits=False, hidden=False)
    positions = [0, 1, 15, 16, 31, 32, 33, 47, 48, 63, 64, 69]
    ratio, ulps, differ = oracle.check_layer_stack(model, ids, outputs, kv, threads=THREADS, positions=positions)
    print(f"gemma4 batched: layer ratio {ratio:.3f}, K/V ratio {ulps:.3f}, {differ} fp16 values differ", flush=True)


@pytest.mark.parametrize("width", [256, 512])
def test_batched_trace_long_chunks_teacher_forced(width):
    """The batched attention's chunks that span several key blocks (more than 2,048 keys at width 256,
    1,024 at width 512: batch_attention_kernel's multi-block branch, which every prompt longer than
    that takes in a batched prefill), traced 32 positions at a time through a global layer and checked
    teacher-forced past those lengths."""
    if width == 256:
        model = synth.model(name="batch-long", layers=2, hidden=1024, intermediate=2048, q_heads=16, kv_heads=8,
                            head_width=256, vocabulary=2048, window=0, global_every=1)
        n, positions = 2200, [0, 1023, 1024, 2047, 2048, 2049, 2079, 2080, 2199]
    else:
        model = synth.gemma4_model(name="batch-long512", layers=2, hidden=1024, intermediate=2048,
                                   local_q=(16, 8, 256), global_q=(16, 1, 512), vocabulary=2048, window=16,
                                   global_every=2)
        n, positions = 1100, [0, 511, 512, 1023, 1024, 1025, 1055, 1056, 1099]
    ids = [int(i) for i in synth.prompt_ids(n, model.vocabulary, name=f"batch-long{width}.ids")]
    kv_rows = max(L.kv_heads * L.head_width for L in model.layers)
    with open_with_env(model, n + 8, AF_TRACE_BATCH=32) as s:
        outputs, kv, _, _ = s.trace(ids, kv_rows=kv_rows, logits=False, hidden=False)
    ratio, ulps, differ = oracle.check_layer_stack(model, ids, outputs, kv, threads=THREADS, positions=positions)
    print(f"batched long trace width {width} n={n}: layer ratio {ratio:.3f}, K/V ratio {ulps:.3f}, "
          f"{differ} fp16 values differ", flush=True)
    assert np.isfinite(outputs).all()


def test_batched_prefill_generation_matches_oracle_and_resumes():
    """Generation with the default batched prefill: greedy ids equal the oracle's for a 75-token prompt
    (three batches, the local ring wrapping), then a follow-up turn on the cached prefix (its pending
    tokens prefilled in a batch) continues exactly as the oracle does."""
    model = batch_model(16, 8, 16, name="batch-gen")
    prompt = [int(i) for i in synth.prompt_ids(75, model.vocabulary, name="batch-gen.prompt")]
    stop = [model.vocabulary - 1]
    with open_with_env(model, 160) as s:
        first = s.generate(prompt, stop, 8)
        turn2 = prompt + first.ids + [int(i) for i in synth.prompt_ids(40, model.vocabulary, name="batch-gen.more")]
        second = s.generate(turn2, stop, 8)
    want = []
    for p in (prompt, turn2):  # the oracle runs each conversation from an empty cache
        ref = oracle.Model(model, capacity=160, threads=THREADS)
        want.append(ref.generate(p, stop, 8)[0])
        ref.close()
    assert first.ids == want[0], (first.ids, want[0])
    assert second.ids == want[1], (second.ids, want[1])


def test_batched_and_stepwise_prefill_caches_agree():
    """A batched prefill and the step kernel's token-by-token prefill agree: their fp32 sums run in
    different orders (so, unlike the reference's consume_batch, not bit for bit; each is checked against
    the oracle above), and after 40 untethered positions through 3 layers the appended K/V, the layer
    outputs and the final logits still agree to 1e-3 of their scale, with the same greedy id."""
    model = batch_model(16, 8, 16, name="batch-vs-step")
    ids = [int(i) for i in synth.prompt_ids(40, model.vocabulary, name="batch-vs-step.ids")]
    kv_rows = 8 * 256
    with open_with_env(model, 48, AF_TRACE_BATCH=32) as s:
        out_b, kv_b, lg_b, _ = s.trace(ids, kv_rows=kv_rows)
    with open_with_env(model, 48) as s:
        out_s, kv_s, lg_s, _ = s.trace(ids, kv_rows=kv_rows)
    assert np.abs(kv_b - kv_s).max() <= 1e-3 * np.abs(kv_s).max()  # (fp16 values as float32)
    assert not np.array_equal(out_b, out_s)  # two different paths ran
    assert np.abs(out_b - out_s).max() <= 1e-3 * np.abs(out_s).max()
    assert np.abs(lg_b - lg_s).max() <= 1e-3 * np.abs(lg_s).max()
    assert int(np.argmax(lg_b)) == int(np.argmax(lg_s))
