"""Greedy speculative decoding with prompt-lookup drafts (AF_SPECULATIVE=1; the reference's
ADAFORGE_SPECULATIVE path, crates/cuda-backend/src/stack.rs:1252-1338, drafts stack.rs:1491-1511,
verification passes of at most MAX_VERIFY = 16 tokens, batch.rs:13) on the GPU: the ids equal the CPU
oracle's plain greedy decoding, drafts are proposed and accepted, stop ids inside an accepted draft
end the generation, and a later turn continues from the rolled-back caches."""
import os

import numpy as np
import pytest

import oracle
from adaforge_amd import synth
from adaforge_amd.backend import HipDiagnostics

pytestmark = pytest.mark.gpu
THREADS = max(1, min(16, os.cpu_count() or 1))


def open_with_env(model, capacity, **env):
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


def spec_model(window=16, global_every=3):
    """Three layers at the BASELINE head geometry, hidden 1024 (default: local window 16, local, global)."""
    return synth.model(name="spec", layers=3, hidden=1024, intermediate=2048, q_heads=16, kv_heads=8,
                       head_width=256, vocabulary=2048, window=window, global_every=global_every)


def echo_prompt(model, n_head=12, pattern=24, repeats=3):
    """A prompt ending in a repeated pattern, so that prompt lookup finds 3-gram matches."""
    head = [int(i) for i in synth.prompt_ids(n_head, model.vocabulary, name="spec.head")]
    pat = [int(i) for i in synth.prompt_ids(pattern, model.vocabulary, name="spec.pattern")]
    return head + pat * repeats


def copying_setup(n_lead=20, n_cont=40):
    """A model whose layers are all local with window 4 (each position sees at most the 10 positions
    before it through the 3 layers; RoPE scores depend on position differences only), and a prompt
    lead + G[:n_cont] + lead[-10:], where G is the model's own greedy continuation of `lead`: at the
    prompt's end the model is in the state that produced G, and prompt lookup drafts G from the copy
    of it in the prompt."""
    model = spec_model(window=4, global_every=4)
    lead = [int(i) for i in synth.prompt_ids(n_lead, model.vocabulary, name="spec.lead")]
    with open_with_env(model, 64) as s:
        g = s.generate(lead, [model.vocabulary - 1], n_cont).ids
    return model, lead + g + lead[-10:], g


def oracle_greedy(model, prompt, stop, n, capacity):
    ref = oracle.Model(model, capacity=capacity, threads=THREADS)
    ids, stopped, _ = ref.generate(prompt, stop, n)
    ref.close()
    return ids, stopped


def test_draft_lookup_matches_reference_rule_on_the_host_side():
    """The draft rule, restated: tokens after the most recent earlier occurrence of the last 3 tokens."""
    h = [1, 2, 3, 4, 5, 1, 2, 3, 9, 1, 2, 3]
    # most recent earlier occurrence of (1, 2, 3) starts at 5 -> followed by 9, 1, 2, 3
    starts = [i for i in range(len(h) - 3) if h[i:i + 3] == h[-3:]]
    assert starts[-1] == 5 and h[starts[-1] + 3:starts[-1] + 3 + 4] == [9, 1, 2, 3]


def test_speculative_generation_equals_oracle_greedy_and_accepts_drafts():
    model, prompt, g = copying_setup()
    stop = [model.vocabulary - 1]
    n = 48
    with open_with_env(model, 192, AF_SPECULATIVE=1) as s:
        got = s.generate(prompt, stop, n)
        passes, drafted, accepted = s.speculation()
    print(f"speculative: {len(got.ids)} ids, {passes} verification passes, {drafted} drafted, {accepted} accepted; "
          f"continuation repeats G for {next((i for i, (a, b) in enumerate(zip(got.ids, g)) if a != b), len(g))} ids",
          flush=True)
    want, _ = oracle_greedy(model, prompt, stop, n, 192)
    assert got.ids == want, (got.ids, want)
    assert passes > 0 and accepted > 0


def test_speculative_on_a_repeated_pattern_equals_oracle():
    model = spec_model()
    prompt = echo_prompt(model)
    stop = [model.vocabulary - 1]
    with open_with_env(model, 256, AF_SPECULATIVE=1) as s:
        got = s.generate(prompt, stop, 96)
    want, _ = oracle_greedy(model, prompt, stop, 96, 256)
    assert got.ids == want


def test_speculative_and_plain_sessions_agree_over_turns():
    """Two turns: the second prompt extends the first conversation (its last id pending in the plain
    session, consumed in the speculative one); both sessions give the oracle's ids."""
    model = spec_model()
    prompt = echo_prompt(model, repeats=2)
    stop = [model.vocabulary - 1]
    out = {}
    for spec in (0, 1):
        with open_with_env(model, 320, AF_SPECULATIVE=spec) as s:
            a = s.generate(prompt, stop, 40)
            turn2 = prompt + a.ids + prompt[5:29]
            b = s.generate(turn2, stop, 40)
            out[spec] = (a.ids, b.ids, turn2)
    assert out[0][0] == out[1][0]
    assert out[0][2] == out[1][2] and out[0][1] == out[1][1]
    want, _ = oracle_greedy(model, out[1][2], stop, 40, 320)
    assert out[1][1] == want


def test_speculative_stop_inside_an_accepted_draft():
    """A stop id that the greedy continuation reaches inside an accepted draft ends the generation
    before it, with the oracle's ids, and the next turn continues from the rolled-back caches."""
    model, prompt, g = copying_setup()
    stop0 = [model.vocabulary - 1]
    free, _ = oracle_greedy(model, prompt, stop0, 40, 192)
    # a stop id first reached several tokens into the continuation (inside a draft when drafts match)
    k = next((i for i in range(6, len(free)) if free[i] not in free[:i]), len(free) - 1)
    stop = [free[k]]
    with open_with_env(model, 192, AF_SPECULATIVE=1) as s:
        got = s.generate(prompt, stop, 40)
        assert got.ids == free[:k] and got.stopped
        more = s.generate(prompt + got.ids + [free[k]], stop0, 12)
    want, _ = oracle_greedy(model, prompt + free[:k + 1], stop0, 12, 192)
    assert more.ids == want
