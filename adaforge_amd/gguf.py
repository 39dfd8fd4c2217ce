"""GgufInspector: the ModelInspector port (crates/application/src/lib.rs) over GGUF v3 files, as
crates/model-formats/src/gguf.rs:10-540 implements it, on the C ABI's reader (af_gguf_*).

inspect() returns the header (ModelInfo: version, size, data offset, metadata, tensors); the
read_* methods return the domain inputs the GPU ports take (Q4_0 / Q6_K matrices, RMSNorm
weights with the file's epsilon, F32 vectors, embedding rows); open_session() opens a generation
session straight from a Gemma 4 file (af_gguf_session_open: the reference's layer assembly,
crates/application/src/stack.rs:26-107).  Errors raise AfError (DiagnosticError)."""
import ctypes
from dataclasses import dataclass, field
from typing import Dict, List, Sequence

import numpy as np

from . import _native as N
from ._native import AfError, check
from .backend import HipGenerationSession, Q4Matrix, RmsNorm

TYPE_NAMES = {N.GGUF_F32: "F32", N.GGUF_F16: "F16", N.GGUF_Q4_0: "Q4_0", N.GGUF_Q8_0: "Q8_0",
              N.GGUF_Q6_K: "Q6K", N.GGUF_BF16: "BF16"}


@dataclass
class TensorInfo:
    """crates/domain/src/lib.rs TensorInfo: dimensions contiguous-first, absolute file offset."""
    name: str
    dimensions: List[int]
    weight_type: str
    file_offset: int
    byte_length: int


@dataclass
class ArraySummary:
    """MetadataValue::ArraySummary: an array too long to keep (more than 4096 elements)."""
    element_type: int
    length: int


@dataclass
class ModelInfo:
    format_version: int
    file_bytes: int
    data_offset: int
    metadata: Dict[str, object] = field(default_factory=dict)
    tensors: List[TensorInfo] = field(default_factory=list)


@dataclass
class Q6Matrix:
    columns: int
    rows: int
    data: np.ndarray


class GgufFile:
    """An open, indexed GGUF file (af_gguf); closed on close() or garbage collection."""

    def __init__(self, path):
        h = N.P()
        check(N.lib().af_gguf_open(str(path).encode(), ctypes.byref(h)))
        self._h = h.value

    def _value(self, v):
        if v.kind == N.GGUF_UNSIGNED:
            return int(v.u)
        if v.kind == N.GGUF_SIGNED:
            return int(v.i)
        if v.kind == N.GGUF_FLOAT:
            return float(v.f)
        if v.kind == N.GGUF_BOOL:
            return bool(v.u)
        if v.kind == N.GGUF_TEXT:
            return ctypes.string_at(v.text, v.length).decode("utf-8") if v.length else ""
        if v.kind == N.GGUF_ARRAY_SUMMARY:
            return ArraySummary(int(v.element_type), int(v.length))
        return None  # arrays: read element by element

    def meta(self, key):
        v = N.GgufValue()
        check(N.lib().af_gguf_meta(self._h, key.encode(), N.AF_GGUF_WHOLE, ctypes.byref(v)))
        if v.kind != N.GGUF_ARRAY:
            return self._value(v)
        out = []
        for i in range(v.length):
            e = N.GgufValue()
            check(N.lib().af_gguf_meta(self._h, key.encode(), i, ctypes.byref(e)))
            out.append(self._value(e))
        return out

    def info(self) -> ModelInfo:
        f = N.GgufFile()
        check(N.lib().af_gguf_info(self._h, ctypes.byref(f)))
        m = ModelInfo(int(f.version), int(f.file_bytes), int(f.data_offset))
        key = ctypes.c_char_p()
        v = N.GgufValue()
        for i in range(f.metadata):
            check(N.lib().af_gguf_meta_at(self._h, i, ctypes.byref(key), ctypes.byref(v)))
            k = key.value.decode()
            m.metadata[k] = self.meta(k)
        t = N.GgufTensor()
        for i in range(f.tensors):
            check(N.lib().af_gguf_tensor_at(self._h, i, ctypes.byref(key), ctypes.byref(t)))
            m.tensors.append(TensorInfo(key.value.decode(), [int(t.dims[d]) for d in range(t.n_dims)],
                                        TYPE_NAMES[t.type], int(t.offset), int(t.bytes)))
        return m

    def tensor(self, name) -> TensorInfo:
        t = N.GgufTensor()
        check(N.lib().af_gguf_tensor(self._h, name.encode(), ctypes.byref(t)))
        return TensorInfo(name, [int(t.dims[d]) for d in range(t.n_dims)], TYPE_NAMES[t.type], int(t.offset),
                          int(t.bytes))

    def read(self, name, offset=0, length=None) -> np.ndarray:
        t = self.tensor(name)
        n = t.byte_length - offset if length is None else length
        out = np.empty(n, np.uint8)
        check(N.lib().af_gguf_read(self._h, name.encode(), offset, out.ctypes.data, n))
        return out

    def close(self):
        if self._h:
            N.lib().af_gguf_close(self._h)
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


def _require(cond, message):
    if not cond:
        raise AfError(N.AF_ERR_INVALID, message)


class GgufInspector:
    """ModelInspector over GGUF files (crates/model-formats/src/gguf.rs:44-413)."""

    def inspect(self, path) -> ModelInfo:
        with GgufFile(path) as g:
            return g.info()

    def read_q4_matrix(self, path, name) -> Q4Matrix:
        with GgufFile(path) as g:
            t = g.tensor(name)
            _require(t.weight_type == "Q4_0" and len(t.dimensions) == 2, "a rank-2 Q4_0 matrix is required")
            _require(t.byte_length <= 256 << 20, "matrix above the 256 MiB diagnostic limit")
            return Q4Matrix(t.dimensions[0], t.dimensions[1], g.read(name))

    def read_q6_matrix(self, path, name) -> Q6Matrix:
        with GgufFile(path) as g:
            t = g.tensor(name)
            _require(t.weight_type == "Q6K" and len(t.dimensions) == 2, "a rank-2 Q6_K matrix is required")
            _require(t.dimensions[0] <= 65536 and t.dimensions[1] <= 1000000, "Q6_K matrix too large")
            return Q6Matrix(t.dimensions[0], t.dimensions[1], g.read(name))

    def read_f32_vector(self, path, name) -> np.ndarray:
        with GgufFile(path) as g:
            t = g.tensor(name)
            _require(t.weight_type == "F32" and len(t.dimensions) == 1 and t.dimensions[0] <= 65536,
                     "an F32 vector of at most 65536 elements is required")
            v = g.read(name).view(np.float32).copy()
            _require(bool(np.isfinite(v).all()), "non-finite F32 value")
            return v

    def read_rms_norm(self, path, name) -> RmsNorm:
        with GgufFile(path) as g:
            _require(g.meta("general.architecture") == "gemma4", "the model RMSNorm diagnostic targets Gemma 4")
            eps = g.meta("gemma4.attention.layer_norm_rms_epsilon")
            _require(isinstance(eps, float), "RMSNorm epsilon missing or invalid")
            t = g.tensor(name)
            _require(t.weight_type == "F32" and len(t.dimensions) == 1 and t.dimensions[0] <= 65536,
                     "RMSNorm expects an F32 vector of 1 to 65536 elements")
            return RmsNorm(g.read(name).view(np.float32).copy(), float(np.float32(eps)))

    def read_embeddings(self, path, ids: Sequence[int]):
        """Rows `ids` of the Q6_K token_embd table (gguf.rs:199-260): (width, vocabulary, ids, bytes)."""
        with GgufFile(path) as g:
            _require(g.meta("general.architecture") == "gemma4", "embeddings: a Gemma 4 model is required")
            t = g.tensor("token_embd.weight")
            _require(t.weight_type == "Q6K" and len(t.dimensions) == 2, "embeddings: a rank-2 Q6_K table is required")
            width, vocabulary = t.dimensions
            ids = list(ids) or [0, 1, 2, 255, 256, 1023, vocabulary - 1, 1]
            _require(len(ids) <= 256 and all(0 <= i < vocabulary for i in ids),
                     "token id outside the vocabulary or more than 256 ids")
            row = t.byte_length // vocabulary
            data = np.concatenate([g.read("token_embd.weight", i * row, row) for i in ids])
            return width, vocabulary, ids, data

    def open_session(self, path, capacity) -> HipGenerationSession:
        """GpuDiagnostics::open_session on the model of a Gemma 4 file (af_gguf_session_open)."""
        with GgufFile(path) as g:
            vocabulary = g.tensor("token_embd.weight").dimensions[1]
            hidden = g.tensor("token_embd.weight").dimensions[0]
            layers = g.meta("gemma4.block_count")
            h = N.P()
            check(N.lib().af_gguf_session_open(g._h, int(capacity), ctypes.byref(h)))
        return HipGenerationSession(h.value, None, vocabulary, hidden, layers)
