"""GenerationSession on the GPU through the C ABI (af_session_*): the reference's session tests
(crates/cuda-backend/src/stack.rs:1887-2060) on the same fixtures, and multi-layer models
checked against the CPU oracle teacher-forced per layer (stack.rs:707-817 contract) with
greedy ids identical to the oracle's."""
import os

import numpy as np
import pytest

import oracle
from adaforge_amd import synth
from adaforge_amd._native import AfError
from adaforge_amd.backend import HipDiagnostics
from adaforge_amd.synth import SynthLayer, SynthModel

pytestmark = pytest.mark.gpu


def ref_matrix(columns, rows, seed):
    """The Q4_0 test matrix of stack.rs:1772-1782: every block has d = 0x2000 (2^-7) and byte j
    of block i holds (i + j + seed) % 16 low, (i + 15 - j + seed) % 16 high."""
    n = columns // 32 * rows
    i = np.arange(n)[:, None]
    j = np.arange(16)[None, :]
    out = np.empty((n, 18), np.uint8)
    out[:, 0], out[:, 1] = 0x00, 0x20
    out[:, 2:] = ((i + j + seed) % 16) | (((i + 15 - j + seed) % 16) << 4)
    return out.ravel()


def packed_table():
    """The 5-row Q6_K table of stack.rs:2008-2017."""
    rows = []
    for row in range(5):
        b = np.zeros(210, np.uint8)
        b[:192] = (np.arange(192) * 17 + row * 29) % 256
        b[192:208] = 3
        b[208], b[209] = 0x00, 0x28
        rows.append(b)
    return np.concatenate(rows)


def fixture_model(table, rope_context, window):
    """Two identical 256-wide layers, stack.rs:1890-1910 / 1982-2002."""
    ones = np.ones(256, np.float32)

    def layer():
        return SynthLayer(input_norm=ones, q=ref_matrix(256, 512, 0), k=ref_matrix(256, 256, 1),
                          v=ref_matrix(256, 256, 2), q_norm=ones, k_norm=ones, rope_base=1e4,
                          rope_factors=np.ones(128, np.float32), rope_context=rope_context, q_heads=2, kv_heads=1,
                          head_width=256, window=window, scale=1.0, o=ref_matrix(512, 256, 3), post_attn_norm=ones,
                          ffn_norm=ones, gate=ref_matrix(256, 512, 4), up=ref_matrix(256, 512, 5),
                          down=ref_matrix(512, 256, 6), post_ffn_norm=ones)

    return SynthModel(hidden=256, intermediate=512, vocabulary=5, table=table, final_norm=ones, final_eps=1e-6,
                      layers=[layer(), layer()])


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


def open_direct(model, capacity):
    """A session whose steps run as direct launches instead of graph replays."""
    return open_with_env(model, capacity, AF_DISABLE_GRAPHS=1)


def ran_step_kernel(session, cached):
    """True if the session's decode steps run on the persistent step kernel (it reports "layers"
    launches; the per-operation kernels report their own kinds).  Consumes two more ids."""
    _, t = session.profile(cached, 2)
    return t["layers"][0] > 0


def head_reference(model, hidden):
    n = oracle.rmsnorm(model.final_norm, model.final_eps, hidden).astype(np.float32)
    return oracle.q6_matvec(model.table, model.hidden, model.vocabulary, n)


def test_session_prefix_reset_stop_and_budget_stack_rs_1887():
    model = fixture_model(np.zeros(210 * 5, np.uint8), 8, None)
    with HipDiagnostics().open_session(model, 8) as s:
        emitted = []
        first = s.generate_stream([1, 2], [4], 2, emitted.append)
        assert emitted == first.ids
        st = first.stats
        assert (st.prompt_tokens, st.cached_tokens, st.decode_tokens) == (2, 0, 1)
        assert st.prefill_ms >= 0.0 and st.decode_ms >= 0.0
        assert st.total_ms >= st.first_token_ms + st.decode_ms
        assert first.ids == [0, 0] and not first.stopped
        with pytest.raises(AfError):
            s.generate([1, 3], [4], 1)  # not an extension of the cached [1, 2, 0, 0]
        second = s.generate([1, 2, 0, 0, 3], [4], 1)
        assert second.ids == [0]
        assert (second.stats.prompt_tokens, second.stats.cached_tokens) == (1, 4)
        with pytest.raises(AfError):
            s.generate([1, 2, 0, 0, 3, 0], [4], 3)  # 6 + 3 > capacity 8
        s.reset()
        stopped = s.generate([3], [0], 2)
        assert stopped.stopped and stopped.ids == []
        assert stopped.stats.first_token_ms is None
        assert stopped.stats.decode_tokens == 0 and stopped.stats.decode_ms == 0.0
        with pytest.raises(AfError):
            s.generate([2], [4], 1)  # the cache holds [3]
        again = s.generate([3, 1], [4], 1)
        assert again.stats.cached_tokens == 1 and again.stats.prompt_tokens == 1


@pytest.mark.parametrize("step_kernel", ["1", "0"])
def test_graph_matches_direct_for_changing_tokens_positions_and_reset_stack_rs_1980(step_kernel):
    """Graph replays and direct launches leave bit-identical caches: after generating from each
    sequence, a trace of one more token (which reads every cached K/V row of the sliding
    window) returns identical layer outputs, appended K/V and logits on both sessions.  Both the
    persistent step kernel (with the head, one graph per token) and the per-operation kernels."""
    model = fixture_model(packed_table(), 8, 2)
    graph = open_with_env(model, 8, AF_STEP_KERNEL=step_kernel)
    direct = open_with_env(model, 8, AF_STEP_KERNEL=step_kernel, AF_DISABLE_GRAPHS=1)
    try:
        for seq in ([0, 3, 1, 2], [4, 2, 0, 1]):
            a = graph.generate(seq[:3], [4], 2)
            b = direct.generate(seq[:3], [4], 2)
            assert (a.ids, a.stopped) == (b.ids, b.stopped)
            ta = graph.trace([seq[3]], kv_rows=256)
            tb = direct.trace([seq[3]], kv_rows=256)
            for x, y in zip(ta, tb):
                assert np.array_equal(x, y)
            graph.reset()
            direct.reset()
    finally:
        graph.close()
        direct.close()


def test_fixture_model_tokens_and_logits_match_oracle():
    model = fixture_model(packed_table(), 16, 2)
    prompt = [0, 3, 1, 2, 4]
    ref = oracle.Model(model, capacity=16)
    want, want_stopped, _ = ref.generate(prompt, [4], 8)
    ref.close()
    with HipDiagnostics().open_session(model, 16) as s:
        got = s.generate(prompt, [4], 8)
        assert (got.ids, got.stopped) == (want, want_stopped)
        s.reset()
        outputs, kv, logits, hidden = s.trace(prompt, kv_rows=256)
    oracle.check_layer_stack(model, prompt, outputs, kv)
    oracle.compare(head_reference(model, hidden), logits)


@pytest.mark.parametrize("v_norm,layer_scale,q_heads,kv_heads,shared_v,step_kernel", [
    (False, 1.0, 2, 1, False, "1"),
    (True, 0.5, 2, 1, False, "1"),
    (False, 1.0, 2, 2, False, "1"),   # one query head per KV head
    (False, 1.0, 4, 1, False, "1"),   # four query heads per KV head
    (True, 1.0, 2, 1, True, "1"),     # V shares K's weights (stack.rs:172), V-norm on
    (False, 1.0, 4, 2, True, "0"),    # the per-operation kernels in their graph
])
def test_multi_layer_model_teacher_forced_and_greedy_ids(v_norm, layer_scale, q_heads, kv_heads, shared_v,
                                                         step_kernel):
    """Four layers (local window 3, global every second layer) past the window's wrap; with a
    layer scale the post-FFN norm and residual run outside the down projection.  Greedy ids equal
    the oracle's, and every layer of a trace is within tolerance teacher-forced."""
    model = synth.tiny_model(layers=4, vocabulary=2048, window=3, name=f"session{q_heads}{kv_heads}", v_norm=v_norm,
                             q_heads=q_heads, kv_heads=kv_heads)
    for L in model.layers:
        L.layer_scale = layer_scale
        if shared_v:
            L.v = None
    prompt = [int(i) for i in synth.prompt_ids(9, model.vocabulary, name="session.prompt")]
    stop = [model.vocabulary - 1]
    ref = oracle.Model(model, capacity=40)
    want, _, margins = ref.generate(prompt, stop, 8)
    ref.close()
    kv_rows = model.layers[0].kv_heads * model.layers[0].head_width
    with open_with_env(model, 40, AF_STEP_KERNEL=step_kernel) as s:
        got = s.generate(prompt, stop, 8)
        s.reset()
        ids = prompt + want[:4]
        outputs, kv, logits, hidden = s.trace(ids, kv_rows=kv_rows)
        assert ran_step_kernel(s, ids) == (step_kernel == "1")
    assert got.ids == want, (got.ids, want, margins)
    oracle.check_layer_stack(model, ids, outputs, kv)
    oracle.compare(head_reference(model, hidden), logits)


@pytest.mark.parametrize("segmented", [False, True])
def test_step_kernel_time_out_falls_back_to_per_operation_kernels(segmented):
    """A step-kernel launch whose grid barrier times out (forced from the host: the barrier opening
    layer 1's down projection waits for one arrival more than the grid makes) does not poison the
    session: the failed step and the rest of the generation run again on the per-operation
    kernels, and ids, layer outputs and logits match the oracle.  Covers a failure during prefill
    (the first launch is a prefill step) and the session's later calls.  segmented: a Gemma-4-shaped
    model whose global layers 2 and 5 run on the per-operation kernels between step-kernel runs
    [0, 2), [3, 5), [6, 7); the first run times out, and the later launches of the step return at
    once."""
    if segmented:
        model = synth.gemma4_model(name="fallback-g4", layers=7, hidden=1024, intermediate=2048, local_q=(4, 2, 256),
                                   global_q=(4, 1, 512), vocabulary=2048, window=3, global_every=3)
    else:
        model = synth.tiny_model(layers=4, vocabulary=2048, window=3, name="fallback")
    prompt = [int(i) for i in synth.prompt_ids(7, model.vocabulary, name="fallback.prompt")]
    stop = [model.vocabulary - 1]
    ref = oracle.Model(model, capacity=40)
    want, _, margins = ref.generate(prompt, stop, 10)
    ref.close()
    kv_rows = max(L.kv_heads * L.head_width for L in model.layers)
    with open_with_env(model, 40, AF_STEP_FAIL_PHASE=9) as s:
        got = s.generate(prompt, stop, 10)
        assert got.ids == want, (got.ids, want, margins)
        s.reset()
        outputs, kv, logits, hidden = s.trace(prompt, kv_rows=kv_rows)
        assert not ran_step_kernel(s, prompt)
    oracle.check_layer_stack(model, prompt, outputs, kv)
    oracle.compare(head_reference(model, hidden), logits)
    # the same failure met first by a trace, then by a decode step
    with open_with_env(model, 40, AF_STEP_FAIL_PHASE=9) as s:
        outputs2, kv2, _, _ = s.trace(prompt[:3], kv_rows=kv_rows)
        oracle.check_layer_stack(model, prompt[:3], outputs2, kv2)
        got = s.generate(prompt, stop, 10)
        assert got.ids == want, (got.ids, want)
    with open_with_env(model, 40, AF_STEP_FAIL_PHASE=9) as s:
        got = s.generate(prompt[:1], stop, 10)  # no prefill step: the first decode step fails
        ref = oracle.Model(model, capacity=40)
        want1, _, _ = ref.generate(prompt[:1], stop, 10)
        ref.close()
        assert got.ids == want1, (got.ids, want1)
    # prefill one step per position: the first prefill step fails, its position is not advanced
    # (the step ends in the position's advance, not in the head), and the prefill runs again there
    with open_with_env(model, 40, AF_STEP_FAIL_PHASE=9, AF_PREFILL_BATCH=0) as s:
        got = s.generate(prompt, stop, 10)
        assert got.ids == want, (got.ids, want)


def test_continuation_and_streaming_equal_one_generation():
    model = synth.tiny_model(layers=2, vocabulary=1024, window=4, name="continue")
    prompt = [int(i) for i in synth.prompt_ids(5, model.vocabulary, name="continue.prompt")]
    stop = [model.vocabulary - 1]
    with HipDiagnostics().open_session(model, 40) as s:
        whole = s.generate(prompt, stop, 12)
        s.reset()
        first = s.generate(prompt, stop, 5)
        seen = []
        rest = s.generate_stream(prompt + first.ids, stop, 7, seen.append)
        assert seen == rest.ids
        assert rest.stats.cached_tokens == len(prompt) + 5
        assert first.ids + rest.ids == whole.ids
        # prompt + max_new may reach the capacity exactly, not pass it
        s.reset()
        assert len(s.generate(prompt, stop, 35).ids) == 35
        s.reset()
        with pytest.raises(AfError):
            s.generate(prompt, stop, 36)


def test_stop_ids_end_generation_and_session_continues():
    """The fixture model repeats its last input id (its tied embedding dominates every residual
    branch): stop on that id ends the call with no ids, any other stop id lets all max_new through.
    A stop in the middle of a varied sequence is covered by the 48-layer decode test."""
    model = fixture_model(packed_table(), 32, 2)
    prompt = [1, 4, 2]
    with HipDiagnostics().open_session(model, 32) as s:
        free = s.generate(prompt, [3, 0], 10)
        assert free.ids == [2] * 10 and not free.stopped
        s.reset()
        hit = s.generate(prompt, [0, 2], 10)
        assert hit.stopped and hit.ids == []
        more = s.generate(prompt + [0], [3], 2)
        assert more.ids == [0, 0] and not more.stopped
        assert (more.stats.cached_tokens, more.stats.prompt_tokens) == (3, 1)
