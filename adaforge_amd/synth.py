"""Seeded synthetic workloads for the batch-1 decode path.

Host-side only: every tensor comes from libafsynth.so (adaforge_amd/csrc/synth.h),
a pure function of (base seed, tensor name, element index), so the GPU box and
this container produce identical bytes.  Quantised matrices are GGUF blocks
(Q4_0: 18 B / 32 weights; Q6_K: 210 B / 256 weights), exactly what the
reference's GGUF reader hands to the backend (crates/model-formats/src/gguf.rs).
"""
import ctypes
import os
from dataclasses import dataclass, field
from typing import List, Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libafsynth.so")
BASE_SEED = 0x4D49333535
THREADS = max(1, min(16, os.cpu_count() or 1))

_lib = None


def _synth():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"{_LIB_PATH} is missing: run __graft_entry__.build()")
        lib = ctypes.CDLL(_LIB_PATH)
        P, u32, u64, f64, i32 = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_double, ctypes.c_int
        lib.synth_tensor_seed.restype = u64
        lib.synth_tensor_seed.argtypes = [u64, ctypes.c_char_p]
        lib.synth_q4.argtypes = [u64, u32, u32, f64, f64, P, i32]
        lib.synth_q4_signed.argtypes = [u64, u32, u32, f64, f64, P, i32]
        lib.synth_q6.argtypes = [u64, u32, u32, f64, f64, P, i32]
        lib.synth_normal_vec.argtypes = [u64, u64, f64, f64, P, i32]
        lib.synth_half.restype = ctypes.c_uint16
        lib.synth_half.argtypes = [ctypes.c_float]
        _lib = lib
    return _lib


def seed(name: str, base: int = BASE_SEED) -> int:
    return _synth().synth_tensor_seed(base, name.encode())


def q4(name, columns, rows, dlo=1e-3, dhi=2e-2, base=BASE_SEED, signed=False):
    """rows x columns Q4_0 (GGUF bytes): d ~ U[dlo, dhi] as fp16, uniform nibbles; with `signed`,
    |d| ~ U[dlo, dhi] with a random sign (GGUF's quantiser stores d = max / -8, so real scales
    take both signs)."""
    out = np.empty(rows * (columns // 32) * 18, dtype=np.uint8)
    fn = _synth().synth_q4_signed if signed else _synth().synth_q4
    fn(seed(name, base), columns, rows, dlo, dhi, out.ctypes.data, THREADS)
    return out


def q6(name, columns, rows, dlo=1e-4, dhi=5e-3, base=BASE_SEED):
    """rows x columns Q6_K (GGUF bytes): uniform 6-bit codes, int8 sub-scales U[-32, 31], d ~ U[dlo, dhi]."""
    out = np.empty(rows * (columns // 256) * 210, dtype=np.uint8)
    _synth().synth_q6(seed(name, base), columns, rows, dlo, dhi, out.ctypes.data, THREADS)
    return out


def normal(name, n, mean=0.0, std=1.0, base=BASE_SEED):
    out = np.empty(n, dtype=np.float32)
    _synth().synth_normal_vec(seed(name, base), n, mean, std, out.ctypes.data, THREADS)
    return out


def half(value) -> int:
    return _synth().synth_half(float(value))


def ramp(n):
    """The reference's structured input (i % 97) / 48 - 1 (crates/cuda-backend/src/matvec.rs:58), in f32."""
    i = np.arange(n, dtype=np.uint32)
    return ((i % 97).astype(np.float32) / np.float32(48.0) - np.float32(1.0)).astype(np.float32)


def xorshift_vector(n, amplitude=0.125, state=0x4090):
    """The reference's seeded input (matvec.rs:59-64): xorshift32 from 0x4090, ((s & 65535)/32768 - 1) * a."""
    out = np.empty(n, dtype=np.float32)
    s = state
    for i in range(n):
        s ^= (s << 13) & 0xFFFFFFFF
        s ^= s >> 17
        s ^= (s << 5) & 0xFFFFFFFF
        out[i] = (np.float32(s & 65535) / np.float32(32768.0) - np.float32(1.0)) * np.float32(amplitude)
    return out


# ---- decode-model description ----------------------------------------------------------------


@dataclass
class SynthLayer:
    """Host weights of one block, mirroring the reference's LayerWeights (crates/application/src/lib.rs:919-927)."""
    input_norm: np.ndarray
    q: np.ndarray
    k: np.ndarray
    v: Optional[np.ndarray]          # None: V shares K's weights (stack.rs:172 pointer equality)
    q_norm: np.ndarray
    k_norm: np.ndarray
    rope_base: float
    rope_factors: np.ndarray
    rope_context: int
    q_heads: int
    kv_heads: int
    head_width: int
    window: Optional[int]
    scale: float
    o: np.ndarray
    post_attn_norm: np.ndarray
    ffn_norm: np.ndarray
    gate: np.ndarray
    up: np.ndarray
    down: np.ndarray
    post_ffn_norm: np.ndarray
    layer_scale: float = 1.0
    eps: float = 1e-6
    v_norm: bool = False


@dataclass
class SynthModel:
    hidden: int
    intermediate: int
    vocabulary: int
    table: np.ndarray                 # tied Q6_K embedding / lm-head
    final_norm: np.ndarray
    final_eps: float
    layers: List[SynthLayer] = field(default_factory=list)
    cap: float = 30.0


def model(name="gemma3-12b", layers=48, hidden=3840, intermediate=15360, q_heads=16, kv_heads=8, head_width=256,
          vocabulary=262144, window=1024, local_theta=1e4, global_theta=1e6, global_every=6, scale=None,
          table_d=(1e-7, 1e-6), v_norm=False, rope_context=131072, base=BASE_SEED, signed_q4=True, final_scale=100.0):
    """Gemma-3-12B-shaped decode model with seeded random weights (BASELINE config 4 at the defaults).

    Layer i is global iff i % global_every == global_every - 1 (layers 5, 11, ..., 47); the others
    use a sliding window.  Norm weights are 1 + N(0, 0.1) (eps 1e-6), projections Q4_0 with
    |d| ~ U[1e-3, 2e-2].  The attention scale defaults to 1/sqrt(head_width).

    Two choices keep the greedy path of this random model varied and context-dependent:
    * Q4_0 scales carry a random sign (`signed_q4`, as GGUF's quantiser's d = max / -8 does).  With
      d > 0 every weight (n - 8) d of a uniform nibble n has mean -d / 2, so all rows of a matrix
      share one positive bias direction and every token is driven to the same output (the greedy
      run then repeats one id whatever the context).
    * The tied Q6_K table uses d ~ U[table_d].  The sqrt(hidden)-scaled embedding of the input
      token adds about 770 sigma_w / rms(h) times the typical winning logit to that token's own
      logit (sigma_w: the table's weight scale, h: the final residual), while the top two of
      262144 logits lie a few per cent apart: at config 2's [1e-4, 5e-3] the model only repeats
      its input, at [1e-6, 1e-5] (a bonus of about 0.15) an emitted token still tends to repeat
      (21 distinct ids in 256 greedy steps), and at the default [1e-7, 1e-6] (about 0.015) the
      run has 47 distinct ids.
    * The final norm weights are final_scale (1 + N(0, 0.1)).  The logits scale with them and the
      residual stream does not, so the default 100 lifts every top-2 logit margin of the 256-step
      run above 2.5e-3, well clear of the GPU-vs-oracle tolerance."""
    if scale is None:
        scale = 1.0 / float(np.sqrt(head_width))
    p = f"{name}."

    def nw(tag, n):
        return normal(p + tag, n, 1.0, 0.1, base)

    layer_list = []
    for i in range(layers):
        is_global = (i % global_every) == global_every - 1
        L = f"blk.{i}."
        layer_list.append(SynthLayer(
            input_norm=nw(L + "attn_norm", hidden),
            q=q4(p + L + "attn_q", hidden, q_heads * head_width, base=base, signed=signed_q4),
            k=q4(p + L + "attn_k", hidden, kv_heads * head_width, base=base, signed=signed_q4),
            v=q4(p + L + "attn_v", hidden, kv_heads * head_width, base=base, signed=signed_q4),
            q_norm=nw(L + "attn_q_norm", head_width),
            k_norm=nw(L + "attn_k_norm", head_width),
            rope_base=global_theta if is_global else local_theta,
            rope_factors=np.ones(head_width // 2, dtype=np.float32),
            rope_context=rope_context,
            q_heads=q_heads, kv_heads=kv_heads, head_width=head_width,
            window=None if is_global else window,
            scale=scale,
            o=q4(p + L + "attn_output", q_heads * head_width, hidden, base=base, signed=signed_q4),
            post_attn_norm=nw(L + "post_attention_norm", hidden),
            ffn_norm=nw(L + "ffn_norm", hidden),
            gate=q4(p + L + "ffn_gate", hidden, intermediate, base=base, signed=signed_q4),
            up=q4(p + L + "ffn_up", hidden, intermediate, base=base, signed=signed_q4),
            down=q4(p + L + "ffn_down", intermediate, hidden, base=base, signed=signed_q4),
            post_ffn_norm=nw(L + "post_ffw_norm", hidden),
            v_norm=v_norm,
        ))
    return SynthModel(hidden=hidden, intermediate=intermediate, vocabulary=vocabulary,
                      table=q6(p + "token_embd", hidden, vocabulary, table_d[0], table_d[1], base=base),
                      final_norm=(nw("output_norm", hidden) * np.float32(final_scale)).astype(np.float32), final_eps=1e-6,
                      layers=layer_list)


def gemma4_rope_factors(width, rotating=64):
    """Gemma 4's proportional RoPE on its global layers (README.md:150, rope_freqs.weight): the first
    `rotating` pairs turn with factor 1, the other width / 2 - rotating pairs carry a factor of 1e30,
    which all but stops their rotation."""
    f = np.full(width // 2, 1e30, dtype=np.float32)
    f[:rotating] = 1.0
    return f


def gemma4_model(name="gemma4", layers=6, hidden=1024, intermediate=2048, local_q=(4, 2, 256), global_q=(4, 1, 512),
                 vocabulary=2048, window=16, global_every=6, table_d=(1e-7, 1e-6), final_scale=100.0,
                 base=BASE_SEED):
    """A Gemma-4-shaped model (the reference's own model family, README.md:135-150,
    crates/application/src/stack.rs:26-107): local layers of local_q = (query heads, KV heads,
    width) with a sliding window and RoPE base 1e4; every `global_every`-th layer global, with
    global_q's geometry (one KV head of width 512 at full size), V computed with K's weights (no V
    tensor), RoPE base 1e6 with gemma4_rope_factors; attention scale 1.0 and unit-weight V RMSNorm
    on every layer; final logit softcap 30.  The full-size model is gemma4_model(layers=48,
    hidden=3840, intermediate=15360, local_q=(16, 8, 256), global_q=(16, 1, 512), vocabulary=262144,
    window=1024)."""
    p = f"{name}."

    def nw(tag, n):
        return normal(p + tag, n, 1.0, 0.1, base)

    out = []
    for i in range(layers):
        is_global = (i % global_every) == global_every - 1
        qh, kvh, hw = global_q if is_global else local_q
        L = f"blk.{i}."
        out.append(SynthLayer(
            input_norm=nw(L + "attn_norm", hidden),
            q=q4(p + L + "attn_q", hidden, qh * hw, base=base, signed=True),
            k=q4(p + L + "attn_k", hidden, kvh * hw, base=base, signed=True),
            v=None if is_global else q4(p + L + "attn_v", hidden, kvh * hw, base=base, signed=True),
            q_norm=nw(L + "attn_q_norm", hw),
            k_norm=nw(L + "attn_k_norm", hw),
            rope_base=1e6 if is_global else 1e4,
            rope_factors=gemma4_rope_factors(hw) if is_global else np.ones(hw // 2, dtype=np.float32),
            rope_context=131072,
            q_heads=qh, kv_heads=kvh, head_width=hw,
            window=None if is_global else window,
            scale=1.0,
            o=q4(p + L + "attn_output", qh * hw, hidden, base=base, signed=True),
            post_attn_norm=nw(L + "post_attention_norm", hidden),
            ffn_norm=nw(L + "ffn_norm", hidden),
            gate=q4(p + L + "ffn_gate", hidden, intermediate, base=base, signed=True),
            up=q4(p + L + "ffn_up", hidden, intermediate, base=base, signed=True),
            down=q4(p + L + "ffn_down", intermediate, hidden, base=base, signed=True),
            post_ffn_norm=nw(L + "post_ffw_norm", hidden),
            v_norm=True,
        ))
    return SynthModel(hidden=hidden, intermediate=intermediate, vocabulary=vocabulary,
                      table=q6(p + "token_embd", hidden, vocabulary, table_d[0], table_d[1], base=base),
                      final_norm=(nw("output_norm", hidden) * np.float32(final_scale)).astype(np.float32), final_eps=1e-6,
                      layers=out, cap=30.0)


def tiny_model(layers=3, hidden=512, intermediate=1024, q_heads=2, kv_heads=1, head_width=256, vocabulary=1024,
               window=4, name="tiny", **kw):
    """A few-layer model with the same code paths (local and global layers) for oracle-checked tests."""
    return model(name=name, layers=layers, hidden=hidden, intermediate=intermediate, q_heads=q_heads,
                 kv_heads=kv_heads, head_width=head_width, vocabulary=vocabulary, window=window,
                 global_every=kw.pop("global_every", 2), **kw)


def prompt_ids(n, vocabulary, name="prompt", base=BASE_SEED):
    """n seeded random token ids in [0, vocabulary)."""
    s = seed(name, base)
    out = np.empty(n, dtype=np.uint32)
    for i in range(n):
        z = _mix(s + (i + 1) * 0x9E3779B97F4A7C15 & 0xFFFFFFFFFFFFFFFF)
        out[i] = z % vocabulary
    return out


def _mix(z):
    M = 0xFFFFFFFFFFFFFFFF
    z &= M
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M
    return z ^ (z >> 31)
