"""The int8 digit image of a GEMV input (adaforge_amd/csrc/device.h: digit_words, and the block
table block_tab in step.hip): the bound on its rounding, checked on the CPU.

The matrix-core GEMV writes each 32-element block x of its fp32 input as
    x_j ~ s (q0 + q1 2^-7 + q2 2^-14 + q3 2^-21),  s = 2^(e - 5),  e = ilogb(max |x|),
from U_j = rint(x_j 2^(26 - e)) split into signed 7-bit fields.  This file restates those integer
steps in numpy and checks what the design relies on:
  * every digit fits int8 (q1..q3 in [-64, 63], q0 in [-64, 64]) and the digits rebuild U exactly;
  * elements with |x_j| >= 2^(e - 3) (within a factor of 8 of the block maximum's binade) are
    represented exactly; every other element is rounded to the grid 2^(e - 26), an error of at most
    2^(e - 27) <= 2^-27 max |x|;
  * the integer fold 2^14 D0 + 2^7 D1 + D2 of the MFMA digit sums stays inside int32 for any Q4_0
    nibbles (|D_t| <= 32 * 15 * 64) and any Q6_K codes (16-element groups: 16 * 63 * 64).
The same device code's results are compared with the FP64 oracle through the GEMV on the GPU
(tests/test_gpu_matvec.py, including blocks of wide dynamic range)."""
import numpy as np
import pytest


def ilogb(m):
    return np.frexp(np.float32(m))[1].astype(np.int64) - 1 if m > 0 else 0


def digits(block):
    """Digits q[4][n] of one block, as device.h:digit_words computes them."""
    x = np.asarray(block, np.float32)
    m = np.float32(np.max(np.abs(x)))
    if m == 0:
        return np.zeros((4, x.size), np.int64), 0
    e = int(ilogb(m))
    U = np.rint(np.ldexp(x.astype(np.float64), 26 - e)).astype(np.int64)  # exact: x has 24 bits
    q0 = (U + 1056832) >> 21
    q1 = ((U + 8256) >> 14 & 127) - (((U + 8256) >> 14 & 127) >= 64) * 128   # sbfe(U + 8256, 14, 7)
    q2 = ((U + 64) >> 7 & 127) - (((U + 64) >> 7 & 127) >= 64) * 128         # sbfe(U + 64, 7, 7)
    q3 = (U & 127) - ((U & 127) >= 64) * 128                                  # sbfe(U, 0, 7)
    return np.stack([q0, q1, q2, q3]), e


def rebuild(q, e):
    s = np.ldexp(1.0, e - 5)
    return s * (q[0] + np.ldexp(q[1], -7) + np.ldexp(q[2], -14) + np.ldexp(q[3], -21))


def blocks(rng):
    """Random and adversarial 32-element blocks."""
    out = [rng.standard_normal(32).astype(np.float32) * np.float32(10.0 ** rng.uniform(-8, 8)) for _ in range(300)]
    for lo, hi in ((1e4, 1e-4), (1.0, 1e-30), (3e38, 1e-38), (1.0, 2 ** -24), (-1.0, 2 ** -20)):
        b = rng.standard_normal(32).astype(np.float32) * np.float32(hi)
        b[rng.integers(32)] = np.float32(lo)
        out.append(b)
    out.append(np.full(32, np.float32(-1.0)))                       # every element the maximum
    out.append(np.array([2.0 ** k for k in range(-31, 1)], np.float32))  # one element per binade
    out.append(np.float32(1.5) * (np.arange(32) % 2 * 2 - 1).astype(np.float32))
    ties = np.zeros(32, np.float32)
    ties[0] = 1.0
    ties[1:] = np.float32(2.0 ** -27) * (2 * np.arange(1, 32) + 1)   # halfway between grid points
    out.append(ties)
    sub = np.zeros(32, np.float32)
    sub[:4] = np.float32(1e-40), np.float32(-3e-42), np.float32(1.4e-45), np.float32(1e-39)  # subnormal maxima
    out.append(sub)
    return out


@pytest.fixture(scope="module")
def cases():
    return blocks(np.random.default_rng(20260))


def test_digits_fit_int8_and_rebuild_the_integer(cases):
    for b in cases:
        q, e = digits(b)
        assert q[0].min() >= -64 and q[0].max() <= 64
        assert q[1:].min() >= -64 and q[1:].max() <= 63
        if np.max(np.abs(b)) > 0:
            U = np.rint(np.ldexp(b.astype(np.float64), 26 - e)).astype(np.int64)
            assert np.array_equal((q[0] << 21) + (q[1] << 14) + (q[2] << 7) + q[3], U)


def test_rounding_bound_and_exact_near_the_block_maximum(cases):
    for b in cases:
        q, e = digits(b)
        x = b.astype(np.float64)
        err = np.abs(rebuild(q, e) - x)
        if np.max(np.abs(b)) == 0:
            assert not err.any()
            continue
        assert err.max() <= np.ldexp(1.0, e - 27), (e, err.max())
        near = np.abs(x) >= np.ldexp(1.0, e - 3)
        assert not err[near].any()          # exact within a factor of 8 of the maximum's binade
        assert err.max() <= np.ldexp(np.max(np.abs(x)), -27)


def test_wide_range_block_small_elements_are_rounded_not_exact():
    """The claim the design makes is a bound, not exactness: an element 2^-10 of the block
    maximum, with a full 24-bit significand, loses its low bits."""
    b = np.zeros(32, np.float32)
    b[0] = 1.0
    b[1] = np.float32(2.0 ** -10 * (1 + 2.0 ** -23))
    q, e = digits(b)
    err = abs(rebuild(q, e)[1] - float(b[1]))
    assert 0 < err <= 2.0 ** -27


def test_integer_fold_stays_in_int32():
    lim = 2 ** 31
    for dmax in (32 * 15 * 64, 16 * 63 * 64):  # Q4_0 nibbles x digits; Q6_K codes x digits
        assert (2 ** 14 + 2 ** 7 + 1) * dmax < lim
