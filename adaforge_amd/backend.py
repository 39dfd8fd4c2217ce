"""Host-side mirror of AdaForge's GPU ports over the HIP C ABI.

`HipDiagnostics` implements the hot-path subset of the `GpuDiagnostics` port
(crates/application/src/lib.rs:28-187) and `HipGenerationSession` the
`GenerationSession` port (lib.rs:1092-1126), with the reference's names,
argument meanings and error behaviour (errors raise AfError, the
DiagnosticError of lib.rs:17-25).  A Rust FFI crate on the reference's side
binds the same entry points, declared in include/af.h.

The reference backend compares GPU results against the domain crate's CPU
references inside check_matvec/check_rms_norm.  Here those references are
injected (`domain=`), so this package never links a CPU compute path.
"""
import ctypes
import statistics
from dataclasses import dataclass, field
from typing import Callable, List, Optional, Sequence

import numpy as np

from . import _native as N
from ._native import AfError, check


# ---- reports (crates/application/src/lib.rs:7-15, 264-293, 1067-1081) --------------------------

@dataclass
class GpuCheckReport:
    device_name: str
    arch: str
    compute_units: int
    free_memory_bytes: int
    total_memory_bytes: int


@dataclass
class MatvecReport:
    rows: int
    columns: int
    checked_vectors: int
    max_absolute_error: float
    max_tolerance_ratio: float
    median_kernel_ms: float
    repetitions: int


@dataclass
class RmsNormReport:
    width: int
    vectors: int
    epsilon: float
    max_absolute_error: float
    max_tolerance_ratio: float
    median_kernel_ms: float


@dataclass
class GenerationStats:
    prompt_tokens: int
    cached_tokens: int
    prefill_ms: float
    first_token_ms: Optional[float]
    decode_tokens: int
    decode_ms: float
    total_ms: float


@dataclass
class GenerationTokens:
    ids: List[int]
    stopped: bool
    stats: Optional[GenerationStats]


# ---- domain-shaped inputs ---------------------------------------------------------------------

@dataclass
class Q4Matrix:
    columns: int
    rows: int
    data: np.ndarray


@dataclass
class RmsNorm:
    weights: np.ndarray
    epsilon: float


def _u8(a):
    return np.ascontiguousarray(a, dtype=np.uint8)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


class _Keep:
    """Keeps host arrays referenced by ctypes descriptors alive."""

    def __init__(self):
        self.items = []

    def __call__(self, a):
        self.items.append(a)
        return a


def _norm(keep, w, eps):
    w = keep(_f32(w))
    return N.RmsNormDesc(w.ctypes.data_as(N.f32p), w.size, eps)


def _mat(keep, data, columns, rows):
    d = keep(_u8(data))
    return N.MatrixDesc(d.ctypes.data_as(N.u8p), d.size, columns, rows)


def layer_descs(model):
    """af_layer_weights[] + af_output_head for a decode model (adaforge_amd.synth.SynthModel)."""
    keep = _Keep()
    H, I = model.hidden, model.intermediate
    arr = (N.LayerDesc * len(model.layers))()
    for i, L in enumerate(model.layers):
        d = arr[i]
        hw = L.head_width
        d.input_norm = _norm(keep, L.input_norm, L.eps)
        d.matrices[0] = _mat(keep, L.q, H, L.q_heads * hw)
        d.matrices[1] = _mat(keep, L.k, H, L.kv_heads * hw)
        d.matrices[2] = d.matrices[1] if L.v is None else _mat(keep, L.v, H, L.kv_heads * hw)
        d.head_norms[0] = _norm(keep, L.q_norm, L.eps)
        d.head_norms[1] = _norm(keep, L.k_norm, L.eps)
        f = keep(_f32(L.rope_factors))
        d.rope = N.RopeDesc(hw, L.rope_base, f.ctypes.data_as(N.f32p), L.rope_context)
        d.attention = N.AttentionConfigDesc(L.q_heads, L.kv_heads, hw, L.window or 0, L.scale)
        d.output = _mat(keep, L.o, L.q_heads * hw, H)
        d.output_norm = _norm(keep, L.post_attn_norm, L.eps)
        d.ffn = N.FfnDesc(_norm(keep, L.ffn_norm, L.eps), _mat(keep, L.gate, H, I), _mat(keep, L.up, H, I),
                          _mat(keep, L.down, I, H), _norm(keep, L.post_ffn_norm, L.eps), L.layer_scale)
        d.flags = N.AF_LAYER_V_NORM if L.v_norm else 0
    head = N.HeadDesc(_norm(keep, model.final_norm, model.final_eps), _mat(keep, model.table, H, model.vocabulary),
                      model.cap)
    return arr, head, keep


def _stats(s):
    return GenerationStats(int(s.prompt_tokens), int(s.cached_tokens), s.prefill_ms,
                           s.first_token_ms if s.has_first_token else None, int(s.decode_tokens), s.decode_ms,
                           s.total_ms)


def _ids(a):
    a = np.ascontiguousarray(a, dtype=np.uint32)
    return a, a.ctypes.data_as(N.u32p)


class HipGenerationSession:
    """GenerationSession (crates/application/src/lib.rs:1092-1126) over af_session_*."""

    def __init__(self, handle, keep, vocabulary, hidden, layers):
        self._h = handle
        self._keep = keep
        self.vocabulary, self.hidden, self.layers = vocabulary, hidden, layers

    def generate_stream(self, prompt: Sequence[int], stop: Sequence[int], max_new: int,
                        on_token: Optional[Callable[[int], None]] = None) -> GenerationTokens:
        pa, pp = _ids(prompt)
        sa, sp = _ids(stop)
        out = np.zeros(max(int(max_new), 1), dtype=np.uint32)
        n, stopped, st = N.sz(), N.i32(), N.GenerationStats()
        cb = N.TOKEN_FN(lambda _u, i: on_token(int(i))) if on_token else N.TOKEN_FN()
        check(N.lib().af_session_generate(self._h, pp, pa.size, sp, sa.size, int(max_new), cb, None,
                                          out.ctypes.data_as(N.u32p), ctypes.byref(n), ctypes.byref(stopped),
                                          ctypes.byref(st)))
        return GenerationTokens(out[:n.value].tolist(), bool(stopped.value), _stats(st))

    def generate(self, prompt, stop, max_new) -> GenerationTokens:
        return self.generate_stream(prompt, stop, max_new, None)

    def reset(self):
        check(N.lib().af_session_reset(self._h))

    def speculation(self):
        """(verification passes, draft tokens, accepted draft tokens) since open."""
        p, d, a = N.u64(), N.u64(), N.u64()
        check(N.lib().af_session_speculation(self._h, ctypes.byref(p), ctypes.byref(d), ctypes.byref(a)))
        return int(p.value), int(d.value), int(a.value)

    def profile(self, prompt, max_new):
        """Decode with per-kernel event timing (ADAFORGE_TIMING_DECODE, stack.rs:1245-1251):
        returns (ids, {kind: (launches, total_ms, bytes_per_launch)})."""
        pa, pp = _ids(prompt)
        out = np.zeros(max(int(max_new), 1), np.uint32)
        n = N.sz()
        t = (N.KernelTiming * 256)()
        nt = N.sz()
        check(N.lib().af_session_profile(self._h, pp, pa.size, int(max_new), out.ctypes.data_as(N.u32p),
                                         ctypes.byref(n), t, 256, ctypes.byref(nt)))
        return out[:n.value].tolist(), {t[i].name.decode(): (t[i].launches, t[i].total_ms, t[i].bytes_per_launch)
                                        for i in range(nt.value)}

    def trace(self, ids, kv_rows=None, layer_outputs=True, logits=True, hidden=True):
        """GPU half of check_layer_stack / check_logits (stack.rs:707-817).

        Returns (layer outputs [n][layers][hidden], appended K/V [n][layers][2][kv_rows] as
        float32 (None unless kv_rows is given), raw logits after the last id, final hidden)."""
        ia, ip = _ids(ids)
        lo = np.empty((ia.size, self.layers, self.hidden), np.float32) if layer_outputs else None
        kv = np.empty((ia.size, self.layers, 2, kv_rows), np.uint16) if kv_rows else None
        lg = np.empty(self.vocabulary, np.float32) if logits else None
        hd = np.empty(self.hidden, np.float32) if hidden else None
        p = lambda a: a.ctypes.data_as(N.f32p) if a is not None else None
        check(N.lib().af_session_trace(self._h, ip, ia.size, p(lo), kv.ctypes.data_as(N.u16p) if kv is not None
                                       else None, p(lg), p(hd)))
        kvf = kv.view(np.float16).astype(np.float32) if kv is not None else None
        return lo, kvf, lg, hd

    def close(self):
        if self._h:
            N.lib().af_session_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class HipDiagnostics:
    """GpuDiagnostics (crates/application/src/lib.rs:28-187), hot-path subset, on gfx950."""

    def __init__(self, domain=None):
        self.domain = domain

    def check(self) -> GpuCheckReport:
        info = N.DeviceInfo()
        check(N.lib().af_device_query(ctypes.byref(info)))
        return GpuCheckReport(info.name.decode(), info.arch.decode(), info.compute_units, info.free_memory_bytes,
                              info.total_memory_bytes)

    def matvec_run(self, matrix: Q4Matrix, inputs: np.ndarray, repetitions: int = 10):
        """GPU half of check_matvec: outputs [n][rows] and the median kernel time."""
        inputs = _f32(inputs).reshape(-1, matrix.columns)
        data = _u8(matrix.data)
        out = np.empty((inputs.shape[0], matrix.rows), np.float32)
        med = N.f32()
        check(N.lib().af_matvec_run(data.ctypes.data_as(N.u8p), data.size, matrix.columns, matrix.rows,
                                    inputs.ctypes.data_as(N.f32p), inputs.shape[0], repetitions,
                                    out.ctypes.data_as(N.f32p), ctypes.byref(med)))
        return out, med.value

    def check_matvec(self, matrix: Q4Matrix) -> MatvecReport:
        """crates/cuda-backend/src/matvec.rs:9-122: zero, ramp and xorshift inputs; tolerance 1e-4 + 1e-4|ref|."""
        from . import synth
        n = matrix.columns
        inputs = np.stack([np.zeros(n, np.float32), synth.ramp(n), synth.xorshift_vector(n)])
        out, med = self.matvec_run(matrix, inputs, 10)
        err = ratio = 0.0
        for x, y in zip(inputs, out):
            ref = self.domain.q4_matvec(matrix.data, matrix.columns, matrix.rows, x)
            e, r = self.domain.compare(ref, y, 1e-4, 1e-4)
            err, ratio = max(err, e), max(ratio, r)
        return MatvecReport(matrix.rows, matrix.columns, 3, err, ratio, med, 10)

    def rmsnorm_run(self, norm: RmsNorm, inputs: np.ndarray, repetitions: int = 10):
        w = _f32(norm.weights)
        inputs = _f32(inputs).reshape(-1, w.size)
        out = np.empty_like(inputs)
        med = N.f32()
        check(N.lib().af_rmsnorm_run(w.ctypes.data_as(N.f32p), w.size, norm.epsilon, inputs.ctypes.data_as(N.f32p),
                                     inputs.shape[0], repetitions, out.ctypes.data_as(N.f32p), ctypes.byref(med)))
        return out, med.value

    def check_rms_norm(self, norm: RmsNorm) -> RmsNormReport:
        """crates/cuda-backend/src/rms_norm.rs:9-149: eight input patterns, tolerance 2e-5 + 2e-5|ref|."""
        inputs = rmsnorm_patterns(len(norm.weights))
        out, med = self.rmsnorm_run(norm, inputs, 10)
        ref = self.domain.rmsnorm(norm.weights, norm.epsilon, inputs.ravel())
        e, r = self.domain.compare(ref, out.ravel(), 2e-5, 2e-5)
        return RmsNormReport(len(norm.weights), inputs.shape[0], norm.epsilon, e, r, med)

    def open_session(self, model, capacity: int) -> HipGenerationSession:
        arr, head, keep = layer_descs(model)
        h = N.P()
        check(N.lib().af_session_open(arr, len(model.layers), ctypes.byref(head), int(capacity), ctypes.byref(h)))
        return HipGenerationSession(h.value, keep, model.vocabulary, model.hidden, len(model.layers))

    def generate(self, model, prompt, stop, max_new) -> GenerationTokens:
        arr, head, keep = layer_descs(model)
        pa, pp = _ids(prompt)
        sa, sp = _ids(stop)
        out = np.zeros(max(int(max_new), 1), np.uint32)
        n, stopped, st = N.sz(), N.i32(), N.GenerationStats()
        check(N.lib().af_generate(arr, len(model.layers), ctypes.byref(head), pp, pa.size, sp, sa.size, int(max_new),
                                  out.ctypes.data_as(N.u32p), ctypes.byref(n), ctypes.byref(stopped),
                                  ctypes.byref(st)))
        return GenerationTokens(out[:n.value].tolist(), bool(stopped.value), _stats(st))


def softcap(logits, cap):
    """Final logit softcapping on the GPU (af_softcap; crates/domain/src/q6.rs:66-71): the capped
    logits of the reference's logits report (crates/cuda-backend/src/logits.rs:70-201)."""
    from . import hip
    x = np.ascontiguousarray(logits, dtype=np.float32)
    xb, yb = hip.Buffer.from_numpy(x), hip.Buffer(x.shape, np.float32)
    check(N.lib().af_softcap(xb.ptr, yb.ptr, x.size, float(cap), None))
    hip.synchronize()
    return yb.numpy()


def rmsnorm_patterns(width):
    """The eight vectors of crates/cuda-backend/src/rms_norm.rs:22-52 (xorshift32 from 0x4090)."""
    out = np.empty((8, width), np.float32)
    i = np.arange(width)
    out[0] = 0.0
    out[1] = 1.0
    out[2] = 1e-8
    out[3] = np.where(i % 2 == 0, 1.0, -1.0)
    out[4] = (i % 97).astype(np.float32) / np.float32(48.0) - np.float32(1.0)
    s = 0x4090
    for k in range(width):
        s ^= (s << 13) & 0xFFFFFFFF
        s ^= s >> 17
        s ^= (s << 5) & 0xFFFFFFFF
        out[5, k] = np.float32(s & 65535) / np.float32(32768.0) - np.float32(1.0)
    out[6] = 0.0
    out[6, 0] = 10.0
    out[7] = ((i % 17).astype(np.float32) - np.float32(8.0)) * np.float32(1e9)
    return out
