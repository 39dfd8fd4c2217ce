"""Gemma 4 semantics on the GPU (the reference's own model family; README.md:135-150,
crates/application/src/stack.rs:26-107, 195-198): global layers of width-512 heads with one KV head
for 16 query heads and V computed with K's weights, proportional RoPE factors (1e30 on 192 of 256
pairs), attention scale 1.0, unit-weight V RMSNorm, and the final logit softcap.  Checked against the
CPU oracle: every layer output teacher-forced (stack.rs:707-817 contract), greedy ids, the
standalone attention operator at width 512, and the capped logits (logits.rs:70-201)."""
import ctypes
import os

import numpy as np
import pytest

import oracle
from adaforge_amd import _native as N, hip, synth
from adaforge_amd.backend import HipDiagnostics, softcap

pytestmark = pytest.mark.gpu
THREADS = max(1, min(16, os.cpu_count() or 1))


def model_16q(layers=6, global_every=6):
    """Local layers of 16 query / 8 KV heads of 256 (window 16) and every `global_every`-th layer global
    (16 query heads, one KV head of 512, K weights reused as V, Gemma 4's RoPE factors), at hidden
    1024: by default five local layers and a global one."""
    return synth.gemma4_model(name="gemma4-test", layers=layers, hidden=1024, intermediate=2048, local_q=(16, 8, 256),
                              global_q=(16, 1, 512), vocabulary=2048, window=16, global_every=global_every)


# The step kernel takes the local layers in runs between the global ones, which the per-operation
# kernels take: runs [0, 5) then layer 5; or runs [0, 2), [3, 5), [6, 7) around layers 2 and 5 (runs
# that start after a per-operation layer and one that ends the model).
@pytest.mark.parametrize("layers,global_every", [(6, 6), (7, 3)])
def test_gemma4_layers_teacher_forced_and_greedy_ids(layers, global_every):
    model = model_16q(layers, global_every)
    glob = [i for i in range(layers) if i % global_every == global_every - 1]
    runs = sum(1 for i in range(layers) if i not in glob and (i == 0 or i - 1 in glob))
    g = model.layers[glob[0]]
    assert g.v is None and g.head_width == 512 and g.kv_heads == 1 and (g.rope_factors == 1e30).sum() == 192
    n = 80  # past the local window (16) and several 32-token attention chunks
    ids = [int(i) for i in synth.prompt_ids(n, model.vocabulary, name="gemma4-test.ids")]
    kv_rows = max(L.kv_heads * L.head_width for L in model.layers)
    with HipDiagnostics().open_session(model, n + 16) as s:
        outputs, kv, logits, hidden = s.trace(ids, kv_rows=kv_rows)
        positions = [0, 1, 15, 16, 17, 31, 32, 33, 63, 64, 79]
        ratio, ulps, differ = oracle.check_layer_stack(model, ids, outputs, kv, threads=THREADS, positions=positions)
        print(f"gemma4: layer max ratio {ratio:.3f}, K/V ratio {ulps:.3f}, {differ} fp16 values differ", flush=True)
        # the logits after the last id, raw and capped
        nrm = oracle.rmsnorm(model.final_norm, model.final_eps, hidden).astype(np.float32)
        raw = oracle.q6_matvec(model.table, model.hidden, model.vocabulary, nrm, threads=THREADS)
        oracle.compare(raw, logits)
        capped_ref = np.array([oracle.softcap(float(v), model.cap) for v in raw.astype(np.float32)], np.float64)
        oracle.compare(capped_ref, softcap(logits, model.cap))
        # greedy continuation equals the oracle's (raw logits, smallest id on ties)
        s.reset()
        prompt = ids[:12]
        got = s.generate(prompt, [model.vocabulary - 1], 6)
        # each decode step: one step-kernel launch per run, the per-operation kernels per global layer
        s.reset()
        _, t = s.profile(prompt, 2)
        assert t["layers"][0] == 2 * runs and t["qkv"][0] == 2 * len(glob), t
    ref = oracle.Model(model, capacity=32, threads=THREADS)
    want, _, _ = ref.generate(prompt, [model.vocabulary - 1], 6)
    ref.close()
    assert got.ids == want, (got.ids, want)


def attention_512(ctx, window, group, v_shared, v_norm, seed):
    """af_attention_decode at width 512 against the oracle; returns the max tolerance ratio."""
    D, KVH = 512, 1 if group == 16 else 2
    QH = KVH * group
    pos = ctx - 1
    rng = np.random.default_rng(seed)
    ring = min(ctx, window) if window else ctx
    hist_k = rng.standard_normal((pos, KVH, D)).astype(np.float16).astype(np.float32)
    hist_v = hist_k if v_shared else rng.standard_normal((pos, KVH, D)).astype(np.float16).astype(np.float32)
    kc = np.zeros((KVH, ring, D), np.float16)
    vc = np.zeros((KVH, ring, D), np.float16)
    for t in range(max(0, pos - ring), pos):
        kc[:, t % ring] = hist_k[t]
        vc[:, t % ring] = hist_v[t]
    q = rng.standard_normal(QH * D).astype(np.float32)
    k = rng.standard_normal(KVH * D).astype(np.float32)
    v = k if v_shared else rng.standard_normal(KVH * D).astype(np.float32)
    qn = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    kn = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    factors = synth.gemma4_rope_factors(D)
    base, eps, scale = 1e6, 1e-6, 1.0
    qb, kb_, qnb, knb = (hip.Buffer.from_numpy(a) for a in (q, k, qn, kn))
    vb_ = kb_ if v_shared else hip.Buffer.from_numpy(v)
    kcb, vcb = hip.Buffer.from_numpy(kc.view(np.uint16)), hip.Buffer.from_numpy(vc.view(np.uint16))
    out = hip.Buffer(QH * D)
    args = N.AttentionArgs(qb.ptr, kb_.ptr, vb_.ptr, qnb.ptr, knb.ptr, eps, eps, eps, 1 if v_norm else 0,
                           N.RopeDesc(D, base, factors.ctypes.data_as(N.f32p), 131072),
                           N.AttentionConfigDesc(QH, KVH, D, window or 0, scale), kcb.ptr, vcb.ptr, ring, pos, out.ptr)
    N.check(N.lib().af_attention_decode(ctypes.byref(args), None))
    hip.synchronize()
    got = out.numpy()
    # oracle: normed + rotated q and new k (fp16), v (unit-normed when v_norm) fp16
    qr = oracle.rmsnorm(qn, eps, q).astype(np.float32)
    qr = oracle.rope(D, base, factors, 131072, qr, pos).astype(np.float32)
    kr = oracle.rmsnorm(kn, eps, k).astype(np.float32)
    kr = oracle.rope(D, base, factors, 131072, kr, pos).astype(np.float32).astype(np.float16).astype(np.float32)
    vr = oracle.rmsnorm(np.ones(D, np.float32), eps, v).astype(np.float32) if v_norm else v
    vr = np.asarray(vr, np.float32).astype(np.float16).astype(np.float32)
    keys = np.concatenate([hist_k.reshape(-1), kr])
    values = np.concatenate([hist_v.reshape(-1), vr])
    ref = oracle.attention(QH, KVH, D, window, scale, qr, keys, values, pos + 1, pos, threads=THREADS)
    _, r = oracle.compare(ref, got)
    kc2 = kcb.numpy().view(np.float16).reshape(KVH, ring, D)[:, pos % ring].astype(np.float32).ravel()
    assert np.abs(kc2 - kr).max() <= 2e-3 * max(1.0, np.abs(kr).max()), "appended K"
    return r


@pytest.mark.parametrize("ctx,window,group,v_shared,v_norm", [
    (1, None, 16, True, True),
    (100, None, 16, True, True),     # several chunks, one KV head, 8 query groups of 2
    (4096, None, 16, True, True),
    (700, 512, 16, True, False),     # window at width 512
    (300, None, 2, False, False),    # two KV heads, separate V
    (65, None, 1, False, True),
])
def test_attention_decode_width_512(ctx, window, group, v_shared, v_norm):
    r = attention_512(ctx, window, group, v_shared, v_norm, seed=ctx + group)
    print(f"width 512 ctx {ctx} group {group}: ratio {r:.3f}", flush=True)


def test_softcap_matches_reference_and_rejects_invalid_cap():
    rng = np.random.default_rng(7)
    x = np.concatenate([rng.standard_normal(4096) * 40, [0.0, -0.0, 1e-30, 300.0, -300.0, 29.99]]).astype(np.float32)
    got = softcap(x, 30.0)
    want = np.array([oracle.softcap(float(v), 30.0) for v in x], np.float64)
    oracle.compare(want, got)
    assert np.all(np.abs(got) <= 30.0)
    with pytest.raises(N.AfError):
        softcap(x, 0.0)


def test_session_from_gguf_file_equals_session_from_memory(tmp_path):
    """The same Gemma 4 model stored as a GGUF file (tests/gguf_writer.py) and opened with
    af_gguf_session_open (the reference's layer assembly from file metadata) decodes exactly like the
    session built from the weights in memory (identical greedy ids and raw logits), and is checked
    against the CPU oracle on its own: every layer output teacher-forced, the logits of its final
    hidden state, and its greedy ids equal to the oracle's."""
    from adaforge_amd.gguf import GgufInspector
    from tests import gguf_writer

    model = model_16q()
    path = tmp_path / "gemma4.gguf"
    path.write_bytes(gguf_writer.gemma4_gguf(model))
    prompt = [int(i) for i in synth.prompt_ids(20, model.vocabulary, name="gemma4-gguf.prompt")]
    stop = [model.vocabulary - 1]
    kv_rows = max(L.kv_heads * L.head_width for L in model.layers)
    with HipDiagnostics().open_session(model, 64) as mem:
        want = mem.generate(prompt, stop, 8)
        mem.reset()
        _, _, want_logits, _ = mem.trace(prompt, layer_outputs=False)
    with GgufInspector().open_session(str(path), 64) as s:
        got = s.generate(prompt, stop, 8)
        s.reset()
        outputs, kv, got_logits, hidden = s.trace(prompt, kv_rows=kv_rows)
    assert got.ids == want.ids
    assert np.array_equal(got_logits, want_logits)
    ratio, ulps, differ = oracle.check_layer_stack(model, prompt, outputs, kv, threads=THREADS)
    print(f"gguf session: layer max ratio {ratio:.3f}, K/V ratio {ulps:.3f}, {differ} fp16 values differ", flush=True)
    nrm = oracle.rmsnorm(model.final_norm, model.final_eps, hidden).astype(np.float32)
    oracle.compare(oracle.q6_matvec(model.table, model.hidden, model.vocabulary, nrm, threads=THREADS), got_logits)
    ref = oracle.Model(model, capacity=64, threads=THREADS)
    ref_ids, _, _ = ref.generate(prompt, stop, 8)
    ref.close()
    assert got.ids == ref_ids, (got.ids, ref_ids)
