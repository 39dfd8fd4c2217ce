"""Long traces of the decode step at BASELINE attention geometry, checked against the CPU oracle
teacher-forced (crates/cuda-backend/src/stack.rs:707-817 contract; attention semantics
crates/domain/src/attention.rs:52-111, GPU checks crates/cuda-backend/src/attention.rs:482-543).

The persistent step kernel splits each KV head's visible range into chunks of at least 32 tokens
(at most one per workgroup), stages chunks of up to 64 cached rows in LDS (32 for four query heads
per KV head) and merges the chunk partials in the last chunk's workgroup.  These traces reach:
  * one chunk (positions < 32), two chunks (32..63) and many chunks with a cross-workgroup merge;
  * chunks too long to stage, read straight from the cache (global layers past 2048 tokens);
  * the sliding-window ring wrapping (local layers past their window);
and check every layer output at positions around each of those boundaries within
1e-4 + 1e-4 |ref|, with the oracle running each layer on the GPU's own layer input and fp16 K/V
history.  The per-operation kernels (AF_STEP_KERNEL=0, the fall-back path) are checked the same way."""
import os

import numpy as np
import pytest

import oracle
from adaforge_amd import synth
from adaforge_amd.backend import HipDiagnostics

pytestmark = pytest.mark.gpu
THREADS = max(1, min(16, os.cpu_count() or 1))


def long_model(q_heads, kv_heads, window, name):
    """Two layers (0 local with `window`, 1 global), hidden 1024, FFN 2048, head width 256."""
    return synth.model(name=name, layers=2, hidden=1024, intermediate=2048, q_heads=q_heads, kv_heads=kv_heads,
                       head_width=256, vocabulary=2048, window=window, global_every=2)


def boundary_positions(n, window):
    """Positions around the chunking, staging and ring boundaries below n."""
    marks = {0, 1, 31, 32, 33, 63, 64, 65, 127, 128, 255, 256, 511, 512, window - 1, window, window + 1,
             2 * window, 2047, 2048, 2049, 2080, n - 1}
    return sorted(p for p in marks if 0 <= p < n)


def trace_and_check(model, n, env=None, name="long", step=None):
    """step: whether the persistent step kernel is expected to run (default: without env)."""
    ids = [int(i) for i in synth.prompt_ids(n, model.vocabulary, name=name + ".ids")]
    kv_rows = model.layers[0].kv_heads * model.layers[0].head_width
    saved = {}
    for k, v in (env or {}).items():
        saved[k] = os.environ.get(k)
        os.environ[k] = v
    try:
        s = HipDiagnostics().open_session(model, n + 8)
    finally:
        for k, v in saved.items():
            if v is None:
                del os.environ[k]
            else:
                os.environ[k] = v
    with s:
        outputs, kv, _, _ = s.trace(ids, kv_rows=kv_rows, logits=False, hidden=False)
        # which path ran: the persistent step kernel reports "layers" launches, the per-operation
        # kernels their own kinds
        _, timings = s.profile(ids, 2)  # the first id comes from the traced state, the second from a step
        assert (timings["layers"][0] > 0) == (env is None if step is None else step), timings["layers"]
    positions = boundary_positions(n, model.layers[0].window)
    print(f"{name}: n={n}, checking positions {positions}", flush=True)
    ratio, ulps, differ = oracle.check_layer_stack(model, ids, outputs, kv, threads=THREADS, positions=positions)
    print(f"{name}: layer max ratio {ratio:.3f}, K/V ratio {ulps:.3f}, {differ} fp16 values differ", flush=True)
    assert np.isfinite(outputs).all()
    return ratio


@pytest.mark.parametrize("q_heads,kv_heads,window,n", [
    (16, 8, 1024, 2200),   # BASELINE geometry: multi-chunk merges, unstaged chunks past 2048, ring wrap
    (16, 4, 256, 700),     # four query heads per KV head (32-row staging), ring wrap at 256
    (8, 8, 128, 400),      # one query head per KV head (odd chunk-partial width), ring wrap at 128
])
def test_step_kernel_long_trace_teacher_forced(q_heads, kv_heads, window, n):
    model = long_model(q_heads, kv_heads, window, name=f"long{q_heads}x{kv_heads}")
    trace_and_check(model, n, name=f"step-{q_heads}x{kv_heads}")


def test_step_kernel_memory_side_exchange_teacher_forced():
    """The BASELINE geometry on the step kernel without its XCD-local exchange (AF_STEP_XCD_LOCAL=0,
    read at session open: the kernel that runs when a launch's workgroups do not reach the XCDs in
    turn), so the qkv rows, the chunk partials and the merge tickets go through the memory side;
    multi-chunk merges and the ring's wrap at 256, teacher-forced."""
    model = long_model(16, 8, 256, name="longmem")
    trace_and_check(model, 600, env={"AF_STEP_XCD_LOCAL": "0"}, name="step-mem", step=True)


def test_step_kernel_trace_past_8192_positions_teacher_forced():
    """The BASELINE attention geometry traced through the step kernel over 8,300 positions: the global
    layer's 32 unstaged chunks of up to 260 tokens (and their merges) at contexts past 8,192, and the
    local layer's ring after eight wraps, checked teacher-forced at positions there (the bench decodes
    at contexts up to 7,628; the kernel accepts capacities up to 32,768)."""
    model = long_model(16, 8, 1024, name="long8k")
    n = 8300
    ids = [int(i) for i in synth.prompt_ids(n, model.vocabulary, name="long8k.ids")]
    kv_rows = model.layers[0].kv_heads * model.layers[0].head_width
    with HipDiagnostics().open_session(model, n + 8) as s:
        outputs, kv, _, _ = s.trace(ids, kv_rows=kv_rows, logits=False, hidden=False)
        _, timings = s.profile(ids, 2)
        assert timings["layers"][0] > 0, timings["layers"]  # the step kernel ran
    positions = [0, 4095, 4096, 8191, 8192, 8193, 8223, 8224, 8299]
    ratio, ulps, differ = oracle.check_layer_stack(model, ids, outputs, kv, threads=THREADS, positions=positions)
    print(f"step-8k: layer max ratio {ratio:.3f}, K/V ratio {ulps:.3f}, {differ} fp16 values differ", flush=True)
    assert np.isfinite(outputs).all()


def test_per_operation_kernels_long_trace_teacher_forced():
    """The per-operation kernels (the fall-back path; split attention over up to 64 chunks of at
    least 32 tokens merged by the last block) on the BASELINE geometry past the window's wrap."""
    model = long_model(16, 8, 1024, name="long-perop")
    trace_and_check(model, 1100, env={"AF_STEP_KERNEL": "0"}, name="perop-16x8")
