"""TEST INFRASTRUCTURE ONLY: ctypes bindings to the C oracle (oracle/liboracle.so).

The oracle is a CPU restatement of AdaForge's FP64-accumulation domain oracles
(crates/domain/src/*.rs) and of the backend's CPU layer chain
(crates/cuda-backend/src/stack.rs:662-700).  Only tests/, the smoke check and
bench.py's cpu_baseline leg import this module, always as the checker.  Every
wrapper raises OracleError where the reference returns Err(...).
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")


class OracleError(ValueError):
    pass


def _load():
    if not os.path.exists(_LIB_PATH):
        raise OracleError(f"{_LIB_PATH} is missing: run `make -C oracle`")
    lib = ctypes.CDLL(_LIB_PATH)
    P = ctypes.c_void_p
    u32, i32, f32, f64, sz = ctypes.c_uint32, ctypes.c_int, ctypes.c_float, ctypes.c_double, ctypes.c_size_t
    sig = {
        "or_half_to_f32": (f32, [ctypes.c_uint16]),
        "or_f32_to_half": (ctypes.c_uint16, [f32]),
        "or_f16_round": (f32, [f32]),
        "or_q4_validate": (i32, [P, sz, u32, u32]),
        "or_q4_matvec": (i32, [P, u32, u32, P, P, i32]),
        "or_q6_validate": (i32, [P, sz, u32, u32]),
        "or_q6_matvec": (i32, [P, u32, u32, P, P, i32]),
        "or_softcap": (i32, [f32, f32, P]),
        "or_rmsnorm_validate": (i32, [P, u32, f32]),
        "or_rmsnorm": (i32, [P, u32, f32, P, sz, P]),
        "or_rope_validate": (i32, [u32, f64, P, u32]),
        "or_rope": (i32, [u32, f64, P, u32, P, sz, u32, P]),
        "or_attention_validate": (i32, [u32, u32, u32, u32, f32]),
        "or_visible_range": (i32, [u32, u32, u32, P, P]),
        "or_attention": (i32, [u32, u32, u32, u32, f32, P, P, P, u32, u32, P]),
        "or_attention_mt": (i32, [u32, u32, u32, u32, f32, P, P, P, u32, u32, P, i32]),
        "or_attention_output": (i32, [P, u32, u32, P, f32, P, P, P, i32]),
        "or_gelu_tanh": (f64, [f64]),
        "or_ffn": (i32, [P, f32, P, P, P, u32, u32, P, f32, f32, P, P, i32]),
        "or_embedding": (i32, [P, u32, u32, P, sz, i32, P]),
        "or_greedy": (i32, [P, sz, P]),
        "or_compare": (i32, [P, P, sz, f64, f64, P, P, P]),
        "or_layer_forward": (i32, [P, u32, u32, P, P, P, u32, i32, P, P, P, i32]),
        "or_model_new": (P, [u32, u32, u32, P, P, u32, P, f32, u32, i32]),
        "or_model_free": (None, [P]),
        "or_model_reset": (None, [P]),
        "or_model_step": (i32, [P, u32, P, P]),
        "or_model_logits": (i32, [P, P]),
        "or_model_generate": (i32, [P, P, sz, P, sz, u32, P, P, P, P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


_lib = _load()
THREADS = max(1, min(16, os.cpu_count() or 1))


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _u8(a):
    return np.ascontiguousarray(np.frombuffer(a, dtype=np.uint8) if isinstance(a, (bytes, bytearray)) else a,
                                dtype=np.uint8)


def _check(rc, what):
    if rc != 0:
        raise OracleError(what)


def half_to_f32(bits):
    return _lib.or_half_to_f32(int(bits))


def f32_to_half(value):
    return _lib.or_f32_to_half(float(value))


def f16_round(a):
    """Round-to-nearest-even through binary16 (the fp16 KV boundary), elementwise."""
    a = _f32(a)
    return np.array([_lib.or_f16_round(float(v)) for v in a.ravel()], dtype=np.float32).reshape(a.shape)


def q4_validate(data, columns, rows):
    data = _u8(data)
    return _lib.or_q4_validate(_p(data), data.size, columns, rows) == 0


def q4_matvec(data, columns, rows, x, threads=None):
    """crates/domain/src/q4.rs:41-66 -> float64[rows]."""
    data, x = _u8(data), _f32(x)
    if x.size != columns or data.size != columns // 32 * rows * 18:
        raise OracleError("invalid input vector")
    y = np.empty(rows, dtype=np.float64)
    _check(_lib.or_q4_matvec(_p(data), columns, rows, _p(x), _p(y), threads or THREADS), "q4 matvec rejected")
    return y


def q6_validate(data, columns, rows):
    data = _u8(data)
    return _lib.or_q6_validate(_p(data), data.size, columns, rows) == 0


def q6_matvec(data, columns, rows, x, threads=None):
    """crates/domain/src/q6.rs:36-65 -> float64[rows]."""
    data, x = _u8(data), _f32(x)
    if x.size != columns or data.size != columns // 256 * rows * 210:
        raise OracleError("invalid Q6_K input")
    y = np.empty(rows, dtype=np.float64)
    _check(_lib.or_q6_matvec(_p(data), columns, rows, _p(x), _p(y), threads or THREADS), "q6 matvec rejected")
    return y


def softcap(value, cap):
    out = ctypes.c_float()
    _check(_lib.or_softcap(float(value), float(cap), ctypes.byref(out)), "softcap rejected")
    return out.value


def rmsnorm(weights, eps, x):
    """crates/domain/src/rms_norm.rs:24-41 -> float64 (one or more contiguous vectors)."""
    w, x = _f32(weights), _f32(x)
    y = np.empty(x.size, dtype=np.float64)
    _check(_lib.or_rmsnorm(_p(w), w.size, float(eps), _p(x), x.size, _p(y)), "rmsnorm rejected")
    return y


def rope(width, base, factors, context, x, position):
    """crates/domain/src/rope.rs:52-77 -> float64."""
    f, x = _f32(factors), _f32(x)
    if f.size != width // 2:
        raise OracleError("factors length")
    y = np.empty(x.size, dtype=np.float64)
    _check(_lib.or_rope(width, float(base), _p(f), context, _p(x), x.size, position, _p(y)), "rope rejected")
    return y


def attention_validate(q_heads, kv_heads, width, window, scale):
    return _lib.or_attention_validate(q_heads, kv_heads, width, window or 0, float(scale)) == 0


def visible_range(window, tokens, position):
    s, e = ctypes.c_uint32(), ctypes.c_uint32()
    _check(_lib.or_visible_range(window or 0, tokens, position, ctypes.byref(s), ctypes.byref(e)), "position")
    return s.value, e.value


def attention(q_heads, kv_heads, width, window, scale, q, keys, values, tokens, position, threads=1):
    """crates/domain/src/attention.rs:66-111 -> float64[q_heads*width]; window None/0 = global.
    With threads > 1 the query heads run on separate threads (bit-identical output)."""
    q, k, v = _f32(q), _f32(keys), _f32(values)
    if q.size != q_heads * width or k.size != tokens * kv_heads * width or v.size != k.size:
        raise OracleError("attention layout")
    out = np.empty(q.size, dtype=np.float64)
    _check(_lib.or_attention_mt(q_heads, kv_heads, width, window or 0, float(scale), _p(q), _p(k), _p(v), tokens,
                                position, _p(out), int(threads)), "attention rejected")
    return out


def attention_output(o_bytes, columns, rows, norm_w, eps, attn, residual, threads=None):
    """crates/domain/src/attention_output.rs:21-37 -> float64[rows]."""
    o, w, a, r = _u8(o_bytes), _f32(norm_w), _f32(attn), _f32(residual)
    if r.size != rows or w.size != rows or a.size != columns:
        raise OracleError("output branch shapes")
    out = np.empty(rows, dtype=np.float64)
    _check(_lib.or_attention_output(_p(o), columns, rows, _p(w), float(eps), _p(a), _p(r), _p(out),
                                    threads or THREADS), "output branch rejected")
    return out


def gelu_tanh(x):
    return _lib.or_gelu_tanh(float(x))


def ffn(pre_w, pre_eps, gate, up, down, hidden, intermediate, post_w, post_eps, layer_scale, x, threads=None):
    """crates/domain/src/ffn.rs:60-94; post_w None = no post-FFN norm (tail f32(down) + x)."""
    pw, x = _f32(pre_w), _f32(x)
    g, u, d = _u8(gate), _u8(up), _u8(down)
    qw = _f32(post_w) if post_w is not None else None
    if x.size != hidden:
        raise OracleError("ffn input size")
    out = np.empty(hidden, dtype=np.float64)
    _check(_lib.or_ffn(_p(pw), float(pre_eps), _p(g), _p(u), _p(d), hidden, intermediate, _p(qw), float(post_eps),
                       float(layer_scale), _p(x), _p(out), threads or THREADS), "ffn rejected")
    return out


def embedding(table, width, vocabulary, ids, scaled=True):
    """crates/domain/src/embedding.rs:53-78 over rows `ids` of a Q6_K table -> float32[len(ids)*width]."""
    t = _u8(table)
    ids = np.ascontiguousarray(ids, dtype=np.uint32)
    out = np.empty(ids.size * width, dtype=np.float32)
    _check(_lib.or_embedding(_p(t), width, vocabulary, _p(ids), ids.size, 1 if scaled else 0, _p(out)),
           "embedding rejected")
    return out


def greedy(logits):
    """crates/domain/src/sampling.rs:2-16."""
    l = _f32(logits)
    out = ctypes.c_uint32()
    _check(_lib.or_greedy(_p(l), l.size, ctypes.byref(out)), "logits empty or non-finite")
    return out.value


def compare(reference, actual, atol=1e-4, rtol=1e-4):
    """crates/cuda-backend/src/matvec.rs:175-193 -> (max_error, max_ratio); raises on failure."""
    r = np.ascontiguousarray(reference, dtype=np.float64)
    a = _f32(actual)
    if r.size != a.size:
        raise OracleError("sizes differ")
    me, mr, bad = ctypes.c_double(), ctypes.c_double(), ctypes.c_size_t()
    rc = _lib.or_compare(_p(r), _p(a), r.size, atol, rtol, ctypes.byref(me), ctypes.byref(mr), ctypes.byref(bad))
    if rc != 0:
        i = bad.value
        raise OracleError(f"mismatch at {i}: reference {r[i]!r}, actual {a[i]!r}, ratio {mr.value:.3g}")
    return me.value, mr.value


class Layer(ctypes.Structure):
    _fields_ = [
        ("input_norm", ctypes.c_void_p), ("input_eps", ctypes.c_float),
        ("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p),
        ("q_norm", ctypes.c_void_p), ("q_eps", ctypes.c_float),
        ("k_norm", ctypes.c_void_p), ("k_eps", ctypes.c_float),
        ("rope_base", ctypes.c_double), ("rope_factors", ctypes.c_void_p), ("rope_context", ctypes.c_uint32),
        ("q_heads", ctypes.c_uint32), ("kv_heads", ctypes.c_uint32), ("head_width", ctypes.c_uint32),
        ("window", ctypes.c_uint32), ("scale", ctypes.c_float),
        ("o", ctypes.c_void_p), ("post_attn_norm", ctypes.c_void_p), ("post_attn_eps", ctypes.c_float),
        ("ffn_norm", ctypes.c_void_p), ("ffn_eps", ctypes.c_float),
        ("gate", ctypes.c_void_p), ("up", ctypes.c_void_p), ("down", ctypes.c_void_p),
        ("post_ffn_norm", ctypes.c_void_p), ("post_ffn_eps", ctypes.c_float), ("layer_scale", ctypes.c_float),
        ("v_norm", ctypes.c_int), ("kv_fp16", ctypes.c_int),
    ]


def layer_table(model):
    """or_layer descriptors for a synthetic model (adaforge_amd.synth.SynthModel)."""
    n = len(model.layers)
    table = (Layer * n)()
    for i, L in enumerate(model.layers):
        t = table[i]
        t.input_norm, t.input_eps = _p(L.input_norm), L.eps
        t.q, t.k = _p(L.q), _p(L.k)
        t.v = _p(L.k) if L.v is None else _p(L.v)
        t.q_norm, t.q_eps = _p(L.q_norm), L.eps
        t.k_norm, t.k_eps = _p(L.k_norm), L.eps
        t.rope_base, t.rope_factors, t.rope_context = L.rope_base, _p(L.rope_factors), L.rope_context
        t.q_heads, t.kv_heads, t.head_width = L.q_heads, L.kv_heads, L.head_width
        t.window, t.scale = L.window or 0, L.scale
        t.o, t.post_attn_norm, t.post_attn_eps = _p(L.o), _p(L.post_attn_norm), L.eps
        t.ffn_norm, t.ffn_eps = _p(L.ffn_norm), L.eps
        t.gate, t.up, t.down = _p(L.gate), _p(L.up), _p(L.down)
        t.post_ffn_norm, t.post_ffn_eps, t.layer_scale = _p(L.post_ffn_norm), L.eps, L.layer_scale
        t.v_norm, t.kv_fp16 = int(L.v_norm), 1
    return table


def layer_forward(model, table, index, x, keys, values, position, given_kv=False, threads=None):
    """One layer (stack.rs:670-700) on input x with the K/V history `keys`/`values`
    ([position + 1][kv_rows] float32, modified in place unless given_kv).  Returns
    (output float32[hidden], the layer's own new k, new v)."""
    L = model.layers[index]
    kn = L.kv_heads * L.head_width
    x = _f32(x)
    assert keys.dtype == np.float32 and keys.flags.c_contiguous and keys.size >= (position + 1) * kn
    y = np.empty(model.hidden, np.float32)
    kn_, vn_ = np.empty(kn, np.float32), np.empty(kn, np.float32)
    _check(_lib.or_layer_forward(ctypes.byref(table[index]), model.hidden, model.intermediate, _p(x), _p(keys),
                                 _p(values), position, 1 if given_kv else 0, _p(kn_), _p(vn_), _p(y),
                                 threads or THREADS), "layer rejected")
    return y, kn_, vn_


def f16_ulps(a, b):
    """Distance in fp16 units in the last place between two arrays of fp16-representable floats."""
    ia = np.asarray(a, np.float32).astype(np.float16).view(np.int16).astype(np.int32)
    ib = np.asarray(b, np.float32).astype(np.float16).view(np.int16).astype(np.int32)
    ia = np.where(ia < 0, -32768 - ia, ia)
    ib = np.where(ib < 0, -32768 - ib, ib)
    return np.abs(ia - ib)


class Model:
    """Whole-model CPU chain (stack.rs:670-700) over a synthetic model description.

    `model` is an adaforge_amd.synth.SynthModel (host arrays); the oracle holds
    pointers into them, so the SynthModel must outlive this object."""

    def __init__(self, model, capacity, threads=None):
        self._keep = model
        n = len(model.layers)
        table = layer_table(model)
        self._table = table
        self.hidden, self.vocabulary = model.hidden, model.vocabulary
        self.layers = n
        self._h = _lib.or_model_new(model.hidden, model.intermediate, n, ctypes.cast(table, ctypes.c_void_p),
                                    _p(model.table), model.vocabulary, _p(model.final_norm), model.final_eps,
                                    capacity, threads or THREADS)
        if not self._h:
            raise OracleError("model allocation failed")

    def close(self):
        if self._h:
            _lib.or_model_free(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def reset(self):
        _lib.or_model_reset(self._h)

    def step(self, token, per_layer=False):
        h = np.empty(self.hidden, dtype=np.float32)
        pl = np.empty(self.layers * self.hidden, dtype=np.float32) if per_layer else None
        _check(_lib.or_model_step(self._h, int(token), _p(h), _p(pl)), "model step rejected")
        return (h, pl.reshape(self.layers, self.hidden)) if per_layer else h

    def logits(self):
        out = np.empty(self.vocabulary, dtype=np.float64)
        _check(_lib.or_model_logits(self._h, _p(out)), "logits rejected")
        return out

    def generate(self, prompt, stop, max_new):
        prompt = np.ascontiguousarray(prompt, dtype=np.uint32)
        stop = np.ascontiguousarray(stop, dtype=np.uint32)
        ids = np.zeros(max_new, dtype=np.uint32)
        margins = np.zeros(max_new, dtype=np.float32)
        n, stopped = ctypes.c_size_t(), ctypes.c_int()
        _check(_lib.or_model_generate(self._h, _p(prompt), prompt.size, _p(stop), stop.size, max_new, _p(ids),
                                      ctypes.byref(n), ctypes.byref(stopped), _p(margins)), "generation rejected")
        k = n.value
        return ids[:k].tolist(), bool(stopped.value), margins[:k + int(stopped.value)]


def check_layer_stack(model, ids, outputs, kv, atol=1e-4, rtol=1e-4, kv_slack=1e-5, threads=None, positions=None):
    """Teacher-forced check of a GPU trace (crates/cuda-backend/src/stack.rs:707-817 contract).

    For each token t (positions 0..n-1 from an empty cache) and layer l the oracle runs layer l
    on the GPU's own layer input (the embedding for l = 0, else the GPU's output of layer l - 1)
    with the GPU's own fp16 K/V history, including the K/V the GPU appended at t, and the GPU's
    layer output must lie within atol + rtol |ref| on every element.

    The appended K/V themselves are checked against the oracle's own values for the same input
    before the fp16 boundary: each GPU fp16 value must be within one fp16 ulp of the oracle's
    value plus kv_slack times the largest magnitude in that head (the two sides agree to about
    1e-7 of the head's scale before rounding, which near zero spans several fp16 ulps).

    outputs: [n][layers][hidden]; kv: [n][layers][2][kv_rows] float32 (fp16 values).
    positions: the token positions to check (default: all); the K/V history of every position
    still comes from the GPU's trace.
    Returns (max layer tolerance ratio, max K/V ratio (<= 1 passes), number of K/V values whose
    fp16 rounding differs from the oracle's)."""
    H, V = model.hidden, model.vocabulary
    n = len(ids)
    table = layer_table(model)
    ids = np.ascontiguousarray(ids, dtype=np.uint32)
    # EmbeddingBatch takes at most 256 ids per call (crates/domain/src/embedding.rs)
    emb = np.concatenate([embedding(model.table, H, V, ids[i:i + 256], scaled=True)
                          for i in range(0, n, 256)]).reshape(n, H)
    hist = []
    for L in model.layers:
        kn = L.kv_heads * L.head_width
        hist.append((np.zeros(n * kn, np.float32), np.zeros(n * kn, np.float32), kn, L.head_width))
    worst, kv_worst, differ = 0.0, 0.0, 0
    check = set(range(n)) if positions is None else set(int(p) for p in positions)
    for t in range(n):
        for l in range(len(model.layers)):
            keys, values, kn, hw = hist[l]
            keys[t * kn:(t + 1) * kn] = kv[t, l, 0, :kn]
            values[t * kn:(t + 1) * kn] = kv[t, l, 1, :kn]
            if t not in check:
                continue
            x = emb[t] if l == 0 else outputs[t, l - 1]
            y, k_own, v_own = layer_forward(model, table, l, x, keys, values, t, given_kv=True, threads=threads)
            try:
                _, r = compare(y.astype(np.float64), outputs[t, l], atol, rtol)
            except OracleError as e:
                raise OracleError(f"token {t}, layer {l}: {e}") from None
            worst = max(worst, r)
            for gpu, own in ((kv[t, l, 0, :kn], k_own), (kv[t, l, 1, :kn], v_own)):
                own16 = own.astype(np.float16)
                spacing = np.abs(np.spacing(own16)).astype(np.float64)
                head_max = np.repeat(np.abs(own).reshape(-1, hw).max(axis=1), hw).astype(np.float64)
                bound = spacing + kv_slack * head_max
                ratio = np.abs(gpu.astype(np.float64) - own.astype(np.float64)) / bound
                kv_worst = max(kv_worst, float(ratio.max()))
                differ += int((gpu != own16.astype(np.float32)).sum())
    if kv_worst > 1.0:
        raise OracleError(f"appended K/V outside one fp16 ulp (+{kv_slack} x head max): ratio {kv_worst:.3g}")
    return worst, kv_worst, differ
