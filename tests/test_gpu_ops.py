"""Device-pointer operators through the C ABI against the CPU oracle: BASELINE configs 1-3 and
the reference's GPU edge cases (crates/cuda-backend/src/ffn.rs:637-679, logits.rs:665-773,
greedy.rs:189-243, attention.rs:482-543).  Tolerance 1e-4 + 1e-4 |ref| on every element."""
import ctypes

import numpy as np
import pytest

import oracle
from adaforge_amd import _native as N
from adaforge_amd import hip, synth
from tests import workloads as W

pytestmark = pytest.mark.gpu
L = N.lib


def u8p(a):
    return a.ctypes.data_as(N.u8p)


def norm_desc(w, eps):
    w = np.ascontiguousarray(w, np.float32)
    return N.RmsNormDesc(w.ctypes.data_as(N.f32p), w.size, eps), w


def mat_desc(d, cols, rows):
    d = np.ascontiguousarray(d, np.uint8)
    return N.MatrixDesc(u8p(d), d.size, cols, rows), d


def run_ffn(pre, gate, up, down, hidden, inter, x, post=None, scale=1.0):
    keep = []
    pd, a = norm_desc(pre, 1e-6); keep.append(a)
    gd, a = mat_desc(gate, hidden, inter); keep.append(a)
    ud, a = mat_desc(up, hidden, inter); keep.append(a)
    dd, a = mat_desc(down, inter, hidden); keep.append(a)
    if post is None:
        qd = N.RmsNormDesc(None, 0, 1e-6)
    else:
        qd, a = norm_desc(post, 1e-6)
        keep.append(a)
    desc = N.FfnDesc(pd, gd, ud, dd, qd, scale)
    h = N.P()
    N.check(L().af_ffn_create(ctypes.byref(desc), ctypes.byref(h)))
    try:
        xb, yb = hip.Buffer.from_numpy(np.asarray(x, np.float32)), hip.Buffer(hidden)
        N.check(L().af_ffn_run(h, xb.ptr, yb.ptr, None))
        hip.synchronize()
        return yb.numpy()
    finally:
        L().af_ffn_free(h)


def test_config1_ffn_block():
    f = W.config1()
    y = run_ffn(f["pre"], f["gate"], f["up"], f["down"], f["hidden"], f["inter"], f["x"])
    ref = oracle.ffn(f["pre"], 1e-6, f["gate"], f["up"], f["down"], f["hidden"], f["inter"], None, 1e-6, 1.0, f["x"])
    oracle.compare(ref, y)


def test_ffn_with_post_norm_and_layer_scale_ffn_rs_60():
    H, I = 1024, 2048
    pre, post = synth.normal("fp.pre", H, 1.0, 0.1), synth.normal("fp.post", H, 1.0, 0.1)
    g, u, d = synth.q4("fp.g", H, I), synth.q4("fp.u", H, I), synth.q4("fp.d", I, H)
    x = synth.normal("fp.x", H)
    y = run_ffn(pre, g, u, d, H, I, x, post=post, scale=0.75)
    oracle.compare(oracle.ffn(pre, 1e-6, g, u, d, H, I, post, 1e-6, 0.75, x), y)


def test_ffn_zero_branch_preserves_residual_and_scale_ffn_rs_165():
    z = np.zeros(576, np.uint8)
    y = run_ffn(np.ones(32), z, z, z, 32, 32, np.full(32, 2.0, np.float32), post=np.ones(32), scale=0.5)
    assert np.array_equal(y, np.ones(32, np.float32))


def q6_head(data, cols, rows, x):
    h = N.P()
    N.check(L().af_q6_upload(u8p(np.ascontiguousarray(data)), data.size, cols, rows, ctypes.byref(h)))
    try:
        xb, lb, rb = hip.Buffer.from_numpy(np.asarray(x, np.float32)), hip.Buffer(rows), hip.Buffer(2, np.uint32)
        N.check(L().af_q6_gemv_argmax(h, xb.ptr, lb.ptr, rb.ptr, None))
        hip.synchronize()
        return lb.numpy(), rb.numpy()
    finally:
        L().af_q6_free(h)


def test_config2_q6_head_and_argmax():
    w, x = W.config2()
    logits, (idx, bad) = q6_head(w, W.C2_COLS, W.C2_ROWS, x)
    ref = oracle.q6_matvec(w, W.C2_COLS, W.C2_ROWS, x)
    oracle.compare(ref, logits)
    r32 = ref.astype(np.float32)
    want = oracle.greedy(r32)
    assert bad == 0 and idx == want == oracle.greedy(logits)
    top2 = np.sort(r32)[-2:]
    assert top2[1] - top2[0] > 1e-3  # the id is well separated from the runner-up


@pytest.mark.parametrize("rows", [1, 5, 17, 1023])
def test_q6_signed_subscales_subnormal_d_partial_rows_logits_rs_665(rows):
    cols = 512
    data = synth.q6(f"q6e{rows}", cols, rows).reshape(rows, cols // 256, 210).copy()
    data[0::3, :, 208], data[0::3, :, 209] = 0x01, 0x00      # subnormal d (2^-24)
    data[1::3, :, 192:208] = np.uint8(0x80)                     # sub-scale -128
    data = data.ravel()
    x = synth.normal(f"q6ex{rows}", cols)
    logits, (idx, bad) = q6_head(data, cols, rows, x)
    oracle.compare(oracle.q6_matvec(data, cols, rows, x), logits)
    assert bad == 0 and idx == oracle.greedy(logits)


def constant_head(values):
    """A 256-column Q6_K matrix whose logit r for x = e_0 equals values[r] (d = 1, sc = 1)."""
    rows = len(values)
    b = np.zeros((rows, 210), np.uint8)
    b[:, 192:208] = 1
    b[:, 208], b[:, 209] = 0x00, 0x3C                           # d = 1.0
    for r, v in enumerate(values):
        code = int(v) + 32                                      # element 0: ql[0] low nibble, qh[0] bits 0-1
        b[r, 0] = code & 15
        b[r, 128] = code >> 4
    return b.ravel()


@pytest.mark.parametrize("size", [1, 5, 255, 256, 257, 1025, 262144])
def test_greedy_ties_boundaries_and_nonfinite_greedy_rs_189(size):
    vals = np.full(size, -3.0, np.float32)
    vals[-1] = 1.0
    vals[0] = 1.0
    x = np.zeros(256, np.float32)
    x[0] = 1.0
    _, (idx, bad) = q6_head(constant_head(vals), 256, size, x)
    assert bad == 0 and idx == oracle.greedy(vals) == 0
    vals[0] = -7.0
    _, (idx, bad) = q6_head(constant_head(vals), 256, size, x)
    assert bad == 0 and idx == oracle.greedy(vals) == size - 1
    for inf in (np.inf, np.nan):
        xi = x.copy()
        xi[0] = inf
        _, (idx, bad) = q6_head(constant_head(vals), 256, size, xi)
        assert bad == 1


def attention_case(case, group=2, extra=None):
    """Runs af_attention_decode on a config-3 style case; returns (out, appended k, appended v)."""
    QH, KVH, Wd = case.get("q_heads", W.C3_Q_HEADS), case.get("kv_heads", W.C3_KV_HEADS), W.C3_WIDTH
    pos = case["ctx"] - 1
    window = case["window"]
    ring = min(case["ctx"], window) if window else case["ctx"]
    kc = np.zeros((KVH, ring, Wd), np.float16)
    vc = np.zeros((KVH, ring, Wd), np.float16)
    hist_k = case["keys"].reshape(pos, KVH, Wd)
    hist_v = case["values"].reshape(pos, KVH, Wd)
    lo = max(0, pos + 1 - window) if window else 0
    for t in range(lo, pos):
        kc[:, t % ring] = hist_k[t]
        vc[:, t % ring] = hist_v[t]
    bufs = {k: hip.Buffer.from_numpy(np.asarray(case[k], np.float32)) for k in ("q", "k", "v", "q_norm", "k_norm")}
    kb, vb = hip.Buffer.from_numpy(kc.view(np.uint16)), hip.Buffer.from_numpy(vc.view(np.uint16))
    out = hip.Buffer(QH * Wd)
    f = np.ones(Wd // 2, np.float32)
    args = N.AttentionArgs(bufs["q"].ptr, bufs["k"].ptr, bufs["v"].ptr, bufs["q_norm"].ptr, bufs["k_norm"].ptr,
                           case["eps"], case["eps"], case["eps"], int(case["v_norm"]),
                           N.RopeDesc(Wd, case["base"], f.ctypes.data_as(N.f32p), 131072),
                           N.AttentionConfigDesc(QH, KVH, Wd, window or 0, case["scale"]),
                           kb.ptr, vb.ptr, ring, pos, out.ptr)
    N.check(L().af_attention_decode(ctypes.byref(args), None))
    hip.synchronize()
    kc2 = kb.numpy().view(np.float16).reshape(KVH, ring, Wd)
    vc2 = vb.numpy().view(np.float16).reshape(KVH, ring, Wd)
    return out.numpy(), kc2[:, pos % ring].astype(np.float32).ravel(), vc2[:, pos % ring].astype(np.float32).ravel()


@pytest.mark.parametrize("ctx", W.C3_CONTEXTS)
@pytest.mark.parametrize("kind", ["global", "local"])
def test_config3_gqa_attention(ctx, kind):
    case = W.config3(ctx, kind)
    out, k, v = attention_case(case)
    oracle.compare(W.config3_reference(case), out)
    kr, vr = W.config3_new_kv(case)
    assert oracle.f16_ulps(k, kr).max() <= 1 and oracle.f16_ulps(v, vr).max() == 0


@pytest.mark.parametrize("ctx", W.C3_CONTEXTS[:2])
def test_config3_attention_memory_side_merge_matches_xcd_local(ctx, monkeypatch):
    """The chunk partials and merge ticket through the memory side (AF_ATTN_XCD_LOCAL=0, read at
    every call) give the oracle's result too, bit for bit the XCD-local merge's output: both merge
    the same partials in the same order, only their cache policies differ."""
    case = W.config3(ctx, "global")
    xl, k1, v1 = attention_case(case)
    monkeypatch.setenv("AF_ATTN_XCD_LOCAL", "0")
    mem, k2, v2 = attention_case(case)
    oracle.compare(W.config3_reference(case), mem)
    assert np.array_equal(xl.view(np.uint32), mem.view(np.uint32))
    assert np.array_equal(k1, k2) and np.array_equal(v1, v2)


def small_case(ctx, window=None, q_heads=4, kv_heads=2, qscale=1.0, v_norm=False, tag="sc"):
    Wd = W.C3_WIDTH
    hist = ctx - 1
    t = f"{tag}.{ctx}.{window}.{q_heads}.{kv_heads}"
    return {"ctx": ctx, "window": window, "base": 1e4, "scale": 1.0 / 16.0, "v_norm": v_norm, "eps": 1e-6,
            "q_heads": q_heads, "kv_heads": kv_heads,
            "q": synth.normal(t + ".q", q_heads * Wd) * np.float32(qscale), "k": synth.normal(t + ".k", kv_heads * Wd),
            "v": synth.normal(t + ".v", kv_heads * Wd), "q_norm": synth.normal(t + ".qn", Wd, 1.0, 0.1) * np.float32(qscale),
            "k_norm": synth.normal(t + ".kn", Wd, 1.0, 0.1),
            "keys": synth.normal(t + ".K", hist * kv_heads * Wd).astype(np.float16).astype(np.float32),
            "values": synth.normal(t + ".V", hist * kv_heads * Wd).astype(np.float16).astype(np.float32)}


def small_reference(case):
    Wd = W.C3_WIDTH
    pos = case["ctx"] - 1
    f = np.ones(Wd // 2, np.float32)
    q = oracle.rope(Wd, case["base"], f, 131072, oracle.rmsnorm(case["q_norm"], 1e-6, case["q"]).astype(np.float32),
                    pos).astype(np.float32)
    k = oracle.rope(Wd, case["base"], f, 131072, oracle.rmsnorm(case["k_norm"], 1e-6, case["k"]).astype(np.float32),
                    pos).astype(np.float32)
    v = case["v"]
    if case["v_norm"]:
        v = oracle.rmsnorm(np.ones(Wd, np.float32), 1e-6, v).astype(np.float32)
    keys = np.concatenate([case["keys"], k.astype(np.float16).astype(np.float32)])
    values = np.concatenate([case["values"], np.asarray(v, np.float32).astype(np.float16).astype(np.float32)])
    return oracle.attention(case["q_heads"], case["kv_heads"], Wd, case["window"], case["scale"], q, keys, values,
                            pos + 1, pos)


@pytest.mark.parametrize("ctx,window,qh,kvh", [(1, None, 2, 1), (2, 1, 2, 1), (33, None, 4, 4), (65, 64, 8, 2),
                                              (100, 7, 4, 1), (3000, 2500, 4, 2)])
def test_attention_masking_window_and_gqa_mapping_attention_rs_482(ctx, window, qh, kvh):
    case = small_case(ctx, window, qh, kvh)
    out, _, _ = attention_case(case)
    oracle.compare(small_reference(case), out)


@pytest.mark.parametrize("ctx,window,qh,kvh", [(31, None, 16, 8), (32, None, 16, 8), (33, None, 16, 8),
                                              (64, None, 16, 8), (65, None, 16, 8), (481, None, 16, 8),
                                              (497, None, 16, 8), (511, None, 16, 8), (512, None, 16, 8),
                                              (513, None, 16, 8), (700, 500, 16, 8), (97, None, 8, 8),
                                              (512, None, 8, 8), (97, None, 8, 2), (512, None, 8, 2)])
def test_attention_chunk_and_short_form_boundaries(ctx, window, qh, kvh):
    """Visible-position counts around the chunk length (32 positions) and the short form's limit
    (at most 512 positions in at most 16 chunks, kernels.hip:launch_attention_dg: 512 takes it, 513
    the long form), a window whose 500 visible positions take the short form after the ring has
    wrapped, and 1, 2 and 4 query heads per KV head (attention.rs:52-111)."""
    case = small_case(ctx, window, qh, kvh, tag="sf")
    out, _, _ = attention_case(case)
    oracle.compare(small_reference(case), out)


def test_attention_large_scores_and_value_norm():
    case = small_case(300, None, 4, 2, qscale=8.0, v_norm=True, tag="big")
    out, _, _ = attention_case(case)
    oracle.compare(small_reference(case), out)


@pytest.mark.parametrize("width", [3840, 256, 100])
def test_rmsnorm_check_port_eight_patterns_rms_norm_rs_22(width):
    """GpuDiagnostics::check_rms_norm (crates/cuda-backend/src/rms_norm.rs:9-149): the reference's
    eight input vectors (zeros, ones, 1e-8, alternating signs, ramp, xorshift, one spike,
    +-8e9 steps) normalised on the GPU with weights 1 + N(0, 0.1) and eps 1e-6, every element
    within 2e-5 + 2e-5 |ref| of the FP64 oracle (rms_norm.rs:131-149)."""
    from adaforge_amd.backend import HipDiagnostics, RmsNorm
    w = synth.normal(f"rmscheck.{width}", width, 1.0, 0.1)
    report = HipDiagnostics(domain=oracle).check_rms_norm(RmsNorm(w, 1e-6))
    assert (report.width, report.vectors) == (width, 8)
    assert report.max_tolerance_ratio <= 1.0 and report.median_kernel_ms > 0.0
    print(f"rmsnorm-check width {width}: max ratio {report.max_tolerance_ratio:.3g}, "
          f"median {1000 * report.median_kernel_ms:.1f} us")


def test_rmsnorm_device_entry_point_multiple_vectors():
    """af_rmsnorm on device pointers: several contiguous vectors in one launch, each normalised
    on its own (crates/domain/src/rms_norm.rs:24-41)."""
    width, vectors = 3840, 5
    w = synth.normal("rmsdev.w", width, 1.0, 0.1)
    x = synth.normal("rmsdev.x", width * vectors, 0.0, 3.0)
    xb, wb, yb = hip.Buffer.from_numpy(x), hip.Buffer.from_numpy(w), hip.Buffer(width * vectors)
    N.check(L().af_rmsnorm(xb.ptr, wb.ptr, yb.ptr, width, vectors, ctypes.c_float(1e-6), None))
    hip.synchronize()
    oracle.compare(oracle.rmsnorm(w, 1e-6, x), yb.numpy(), 2e-5, 2e-5)
