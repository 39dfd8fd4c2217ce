"""ctypes bindings of the C ABI in include/af.h (adaforge_amd/libadaforge.so).

Loading fails loudly when the library is missing: there is no CPU fallback.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libadaforge.so")

AF_OK = 0
AF_ERR_INVALID = 1
AF_ERR_DEVICE = 2
AF_ERR_NONFINITE = 3
AF_ERR_POISONED = 4
AF_ERR_NO_DEVICE = 5
AF_MAX_CONTEXT = 32768
AF_MAX_NEW_TOKENS = 128
AF_LAYER_V_NORM = 1

P = ctypes.c_void_p
u8p = ctypes.POINTER(ctypes.c_uint8)
f32p = ctypes.POINTER(ctypes.c_float)
u32p = ctypes.POINTER(ctypes.c_uint32)
u16p = ctypes.POINTER(ctypes.c_uint16)
u32, u64, i32, f32, f64, sz = (ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int32, ctypes.c_float, ctypes.c_double,
                               ctypes.c_size_t)


class AfError(RuntimeError):
    """DiagnosticError (crates/application/src/lib.rs:17-25) with the ABI status code."""

    def __init__(self, code, message):
        super().__init__(f"[{code}] {message}")
        self.code = code
        self.message = message


class DeviceInfo(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 256), ("arch", ctypes.c_char * 64), ("compute_units", i32),
                ("free_memory_bytes", u64), ("total_memory_bytes", u64)]


class RmsNormDesc(ctypes.Structure):
    _fields_ = [("weights", f32p), ("len", u32), ("epsilon", f32)]


class MatrixDesc(ctypes.Structure):
    _fields_ = [("bytes", u8p), ("len", sz), ("columns", u32), ("rows", u32)]


class RopeDesc(ctypes.Structure):
    _fields_ = [("width", u32), ("base", f64), ("factors", f32p), ("context", u32)]


class AttentionConfigDesc(ctypes.Structure):
    _fields_ = [("q_heads", u32), ("kv_heads", u32), ("width", u32), ("window", u32), ("scale", f32)]


class FfnDesc(ctypes.Structure):
    _fields_ = [("pre", RmsNormDesc), ("gate", MatrixDesc), ("up", MatrixDesc), ("down", MatrixDesc),
                ("post", RmsNormDesc), ("layer_scale", f32)]


class AttentionArgs(ctypes.Structure):
    _fields_ = [("q", P), ("k", P), ("v", P), ("q_norm", P), ("k_norm", P), ("q_eps", f32), ("k_eps", f32),
                ("v_eps", f32), ("v_norm", i32), ("rope", RopeDesc), ("config", AttentionConfigDesc),
                ("k_cache", P), ("v_cache", P), ("ring", u32), ("position", u32), ("out", P)]


class LayerDesc(ctypes.Structure):
    _fields_ = [("input_norm", RmsNormDesc), ("matrices", MatrixDesc * 3), ("head_norms", RmsNormDesc * 2),
                ("rope", RopeDesc), ("attention", AttentionConfigDesc), ("output", MatrixDesc),
                ("output_norm", RmsNormDesc), ("ffn", FfnDesc), ("flags", u32)]


class HeadDesc(ctypes.Structure):
    _fields_ = [("norm", RmsNormDesc), ("matrix", MatrixDesc), ("cap", f32)]


class GenerationStats(ctypes.Structure):
    _fields_ = [("prompt_tokens", u64), ("cached_tokens", u64), ("prefill_ms", f64), ("first_token_ms", f64),
                ("has_first_token", i32), ("decode_tokens", u64), ("decode_ms", f64), ("total_ms", f64)]


class KernelTiming(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 32), ("launches", u64), ("total_ms", f64), ("bytes_per_launch", f64)]


class GgufFile(ctypes.Structure):
    _fields_ = [("version", u32), ("tensors", u64), ("metadata", u64), ("data_offset", u64), ("file_bytes", u64)]


class GgufTensor(ctypes.Structure):
    _fields_ = [("type", u32), ("n_dims", u32), ("dims", u64 * 4), ("offset", u64), ("bytes", u64)]


class GgufValue(ctypes.Structure):
    _fields_ = [("kind", i32), ("u", u64), ("i", ctypes.c_int64), ("f", f64), ("text", ctypes.c_void_p),
                ("length", u64), ("element_type", u32)]


AF_GGUF_WHOLE = 0xFFFFFFFFFFFFFFFF
GGUF_UNSIGNED, GGUF_SIGNED, GGUF_FLOAT, GGUF_BOOL, GGUF_TEXT, GGUF_ARRAY, GGUF_ARRAY_SUMMARY = range(7)
GGUF_F32, GGUF_F16, GGUF_Q4_0, GGUF_Q8_0, GGUF_Q6_K, GGUF_BF16 = 0, 1, 2, 8, 14, 30

TOKEN_FN = ctypes.CFUNCTYPE(None, P, u32)

# name -> (restype, argtypes): every function include/af.h declares.
SIGNATURES = {
    "af_last_error": (ctypes.c_char_p, []),
    "af_device_query": (i32, [ctypes.POINTER(DeviceInfo)]),
    "af_matvec_run": (i32, [u8p, sz, u32, u32, f32p, u32, u32, f32p, f32p]),
    "af_rmsnorm_run": (i32, [f32p, u32, f32, f32p, u32, u32, f32p, f32p]),
    "af_q4_upload": (i32, [u8p, sz, u32, u32, ctypes.POINTER(P)]),
    "af_q4_free": (None, [P]),
    "af_q4_gemv": (i32, [P, P, P, P]),
    "af_q4_gemm": (i32, [P, P, u32, P, P]),
    "af_q6_upload": (i32, [u8p, sz, u32, u32, ctypes.POINTER(P)]),
    "af_q6_free": (None, [P]),
    "af_q6_gemv_argmax": (i32, [P, P, P, P, P]),
    "af_q6_gemv_argmax_noalloc": (i32, [P, P, P, P, P]),
    "af_rmsnorm": (i32, [P, P, P, u32, u32, f32, P]),
    "af_softcap": (i32, [P, P, sz, f32, P]),
    "af_ffn_create": (i32, [ctypes.POINTER(FfnDesc), ctypes.POINTER(P)]),
    "af_ffn_free": (None, [P]),
    "af_ffn_run": (i32, [P, P, P, P]),
    "af_attention_decode": (i32, [ctypes.POINTER(AttentionArgs), P]),
    "af_session_open": (i32, [ctypes.POINTER(LayerDesc), u32, ctypes.POINTER(HeadDesc), u32, ctypes.POINTER(P)]),
    "af_session_generate": (i32, [P, u32p, sz, u32p, sz, u32, TOKEN_FN, P, u32p, ctypes.POINTER(sz),
                                  ctypes.POINTER(i32), ctypes.POINTER(GenerationStats)]),
    "af_session_reset": (i32, [P]),
    "af_session_speculation": (i32, [P, ctypes.POINTER(u64), ctypes.POINTER(u64), ctypes.POINTER(u64)]),
    "af_session_close": (None, [P]),
    "af_generate": (i32, [ctypes.POINTER(LayerDesc), u32, ctypes.POINTER(HeadDesc), u32p, sz, u32p, sz, u32, u32p,
                          ctypes.POINTER(sz), ctypes.POINTER(i32), ctypes.POINTER(GenerationStats)]),
    "af_session_trace": (i32, [P, u32p, sz, f32p, u16p, f32p, f32p]),
    "af_session_profile": (i32, [P, u32p, sz, u32, u32p, ctypes.POINTER(sz), ctypes.POINTER(KernelTiming), sz,
                                 ctypes.POINTER(sz)]),
    "af_gguf_open": (i32, [ctypes.c_char_p, ctypes.POINTER(P)]),
    "af_gguf_close": (None, [P]),
    "af_gguf_info": (i32, [P, ctypes.POINTER(GgufFile)]),
    "af_gguf_tensor_at": (i32, [P, u64, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(GgufTensor)]),
    "af_gguf_tensor": (i32, [P, ctypes.c_char_p, ctypes.POINTER(GgufTensor)]),
    "af_gguf_read": (i32, [P, ctypes.c_char_p, u64, P, u64]),
    "af_gguf_meta_at": (i32, [P, u64, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(GgufValue)]),
    "af_gguf_meta": (i32, [P, ctypes.c_char_p, u64, ctypes.POINTER(GgufValue)]),
    "af_gguf_session_open": (i32, [P, u32, ctypes.POINTER(P)]),
}

_lib = None


def lib():
    """The loaded C-ABI library; raises if it has not been built (no fallback exists)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: run __graft_entry__.build() (the HIP path is required)")
        lib_ = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_GLOBAL)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib_, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib_
    return _lib


def check(rc):
    if rc != AF_OK:
        raise AfError(rc, lib().af_last_error().decode(errors="replace"))
    return rc
