"""Independent numpy restatements used to pin the C oracle (tests only).

These are written from the data-format definitions (GGUF Q4_0 / Q6_K block
layouts, the closed-form RMSNorm, NeoX RoPE as a complex rotation, softmax
attention), vectorised and structured differently from the oracle's loops, so
that a dropped term, a wrong index or a swapped nibble in either one shows up
as a disagreement.
"""
import numpy as np


def f16_to_f32(bits):
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


def q4_dequant(data, columns, rows):
    """GGUF Q4_0 -> float32 [rows, columns]: w = d * (nibble - 8), low nibbles first then high."""
    blocks = np.asarray(data, dtype=np.uint8).reshape(rows, columns // 32, 18)
    d = f16_to_f32(blocks[:, :, 0].astype(np.uint16) | (blocks[:, :, 1].astype(np.uint16) << 8))
    q = blocks[:, :, 2:]
    lo = (q & 15).astype(np.int32) - 8
    hi = (q >> 4).astype(np.int32) - 8
    codes = np.concatenate([lo, hi], axis=2).astype(np.float32)     # [rows, blocks, 32]
    return (codes * d[:, :, None]).reshape(rows, columns).astype(np.float32)


def q6_unpack(data, columns, rows):
    """GGUF Q6_K -> (codes int [rows, columns] in 0..63, sub-scale per weight int8, d per weight f32).

    Element e of a 256-block: half h = e // 128, r = e % 128, quarter = r // 32, lane = r % 32;
    the low 4 bits come from ql[64h + lane + 32*(quarter & 1)] (low nibble for quarters 0,1, high
    nibble for 2,3), the high 2 bits from qh[32h + lane] bits 2*quarter..2*quarter+1; the
    sub-scale is scales[16-element group of e] = scales[e // 16]."""
    b = np.asarray(data, dtype=np.uint8).reshape(rows, columns // 256, 210)
    e = np.arange(256)
    h, r = e // 128, e % 128
    quarter, lane = r // 32, r % 32
    ql_idx = 64 * h + lane + 32 * (quarter & 1)
    qh_idx = 128 + 32 * h + lane
    ql = b[:, :, ql_idx]
    low = np.where(quarter < 2, ql & 15, ql >> 4)
    high = (b[:, :, qh_idx] >> (2 * quarter)) & 3
    codes = (low | (high << 4)).astype(np.int32)
    scales = b[:, :, 192 + e // 16].view(np.int8).astype(np.int32)
    d = f16_to_f32(b[:, :, 208].astype(np.uint16) | (b[:, :, 209].astype(np.uint16) << 8))
    d = np.repeat(d[:, :, None], 256, axis=2)
    return codes.reshape(rows, columns), scales.reshape(rows, columns), d.reshape(rows, columns)


def q6_dequant(data, columns, rows):
    codes, scales, d = q6_unpack(data, columns, rows)
    return ((d * scales.astype(np.float32)).astype(np.float32) * (codes - 32).astype(np.float32)).astype(np.float32)


def rmsnorm(w, eps, x):
    x = np.asarray(x, dtype=np.float64).reshape(-1, len(w))
    r = 1.0 / np.sqrt((x * x).mean(axis=1, keepdims=True) + float(np.float32(eps)))
    return (x * r * np.asarray(w, dtype=np.float64)).ravel()


def rope(width, base, factors, x, position):
    """NeoX rotation as a complex multiply of (x[i] + j x[i+half]) by exp(j * angle_i)."""
    x = np.asarray(x, dtype=np.float64).reshape(-1, width)
    half = width // 2
    i = np.arange(half, dtype=np.float64)
    angle = position * base ** (-2.0 * i / width) / np.asarray(factors, dtype=np.float64)
    z = (x[:, :half] + 1j * x[:, half:]) * np.exp(1j * angle)
    return np.concatenate([z.real, z.imag], axis=1).ravel()


def attention(q_heads, kv_heads, width, window, scale, q, keys, values, tokens, position):
    q = np.asarray(q, dtype=np.float64).reshape(q_heads, width)
    k = np.asarray(keys, dtype=np.float64).reshape(tokens, kv_heads, width)
    v = np.asarray(values, dtype=np.float64).reshape(tokens, kv_heads, width)
    end = position + 1
    start = max(0, end - window) if window else 0
    out = np.zeros((q_heads, width))
    group = q_heads // kv_heads
    for h in range(q_heads):
        s = k[start:end, h // group, :] @ q[h] * scale
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ v[start:end, h // group, :]
    return out.ravel()


def gelu_tanh(x):
    return 0.5 * x * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (x + 0.044715 * x ** 3)))
