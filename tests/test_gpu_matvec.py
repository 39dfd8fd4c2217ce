"""Q4_0 GEMV on the GPU through the C ABI against the CPU oracle (BASELINE config 0 and the
reference's GPU tests crates/cuda-backend/src/matvec.rs:349-413, half_conversion.rs:8-76).
Tolerance: |gpu - ref| <= 1e-4 + 1e-4 |ref| on every row, non-finite fails (matvec.rs:175-193)."""
import ctypes

import numpy as np
import pytest

import oracle
from adaforge_amd import synth
from adaforge_amd import _native as N
from adaforge_amd import hip
from adaforge_amd.backend import HipDiagnostics, Q4Matrix

pytestmark = pytest.mark.gpu


def gemv(data, columns, rows, xs):
    out, _ = HipDiagnostics().matvec_run(Q4Matrix(columns, rows, data), np.stack(xs), 0)
    return out


def test_config0_q4_gemv_4096x3840_three_inputs():
    cols, rows = 3840, 4096
    w = synth.q4("config0.W", cols, rows)
    xs = [np.zeros(cols, np.float32), synth.ramp(cols), synth.normal("config0.x", cols)]
    out = gemv(w, cols, rows, xs)
    assert np.all(out[0] == 0.0)
    for x, y in zip(xs, out):
        e, r = oracle.compare(oracle.q4_matvec(w, cols, rows, x), y)
        assert r <= 1.0


def test_check_matvec_port_reports_within_tolerance():
    cols, rows = 3840, 4096
    m = Q4Matrix(cols, rows, synth.q4("config0.W", cols, rows))
    rep = HipDiagnostics(domain=oracle).check_matvec(m)
    assert rep.checked_vectors == 3 and rep.repetitions == 10
    assert rep.max_tolerance_ratio <= 1.0 and rep.median_kernel_ms > 0.0


def test_partial_warp_group_and_multiple_blocks_matvec_rs_349():
    data = []
    for i in range(5 * 3):
        scale = 0x3800 if i % 2 == 0 else 0xBC00
        data += [scale & 0xFF, scale >> 8]
        data += [((j + i) % 16) | (((15 - j + i) % 16) << 4) for j in range(16)]
    m = Q4Matrix(96, 5, np.array(data, np.uint8))
    rep = HipDiagnostics(domain=oracle).check_matvec(m)
    assert rep.max_tolerance_ratio <= 1.0


@pytest.mark.parametrize("columns", [32, 96, 384, 3840, 4096, 8192, 15360])
def test_short_uneven_and_long_inputs_matvec_rs_361(columns):
    rows = 5
    blocks = rows * columns // 32
    data = np.empty((blocks, 18), np.uint8)
    for b in range(blocks):
        scale = [0x3800, 0xBC00, 1, 0][b % 4]
        data[b, 0], data[b, 1] = scale & 0xFF, scale >> 8
        data[b, 2:] = [(i * 37 + b * 11) & 0xFF for i in range(16)]
    data = data.ravel()
    xs = [((np.arange(columns) * 17 % 97).astype(np.float32) / np.float32(48) - np.float32(1)) * np.float32(a)
          for a in (0.0, 0.125, 1.0)]
    out = gemv(data, columns, rows, xs)
    for x, y in zip(xs, out):
        oracle.compare(oracle.q4_matvec(data, columns, rows, x), y)


@pytest.mark.parametrize("columns,rows", [(3840, 8192 + 4), (15360, 3840 + 3), (4096, 3840 + 1), (640, 77)])
def test_random_shapes_with_ragged_rows(columns, rows):
    w = synth.q4(f"rag{columns}x{rows}", columns, rows)
    x = synth.normal(f"ragx{columns}", columns)
    out = gemv(w, columns, rows, [x])
    oracle.compare(oracle.q4_matvec(w, columns, rows, x), out[0])


def test_every_finite_half_scale_converts_exactly_half_conversion_rs_8():
    halves = np.arange(65536, dtype=np.uint32)
    halves = halves[(halves & 0x7C00) != 0x7C00].astype(np.uint16)
    assert halves.size == 63488
    data = np.zeros((halves.size, 18), np.uint8)
    data[:, 0] = halves & 0xFF
    data[:, 1] = halves >> 8
    data[:, 2] = 9                     # weight 0 = 9 - 8 = 1, weight 16 = 0 - 8
    x = np.zeros(32, np.float32)
    x[0] = 1.0
    out = gemv(data.ravel(), 32, halves.size, [x])[0]
    want = halves.view(np.float16).astype(np.float32)
    # exact equality of values (the wave sum adds +0.0 lanes, so the -0.0 scale yields +0.0)
    assert np.array_equal(out, want)


def test_device_pointer_entry_point_matches_host_level_run():
    cols, rows = 3840, 4096
    w = synth.q4("config0.W", cols, rows)
    x = synth.normal("config0.x", cols)
    h = N.P()
    N.check(N.lib().af_q4_upload(w.ctypes.data_as(N.u8p), w.size, cols, rows, ctypes.byref(h)))
    try:
        xb, yb = hip.Buffer.from_numpy(x), hip.Buffer(rows)
        N.check(N.lib().af_q4_gemv(h, xb.ptr, yb.ptr, None))
        hip.synchronize()
        y = yb.numpy()
    finally:
        N.lib().af_q4_free(h)
    assert np.array_equal(y, gemv(w, cols, rows, [x])[0])


def test_wide_dynamic_range_blocks_within_tolerance():
    """Input blocks whose elements span 2^-40 .. 2^12 of one another: the digit image rounds the
    elements far below their block's maximum (to 2^-27 of it, tests/test_digits.py), and the
    outputs stay within 1e-4 + 1e-4 |ref| of the FP64 oracle on every row."""
    cols, rows = 3840, 512
    w = synth.q4("wide.W", cols, rows, signed=True)
    rng = np.random.default_rng(7)
    x = (rng.standard_normal(cols) * np.exp2(rng.integers(-40, 12, cols))).astype(np.float32)
    x[::32] = np.float32(1000.0)                       # one large element per block
    x[5::32] = np.float32(3.0e-9)
    out = gemv(w, cols, rows, [x, -x, x * np.float32(2.0 ** -30)])
    for xi, y in zip((x, -x, x * np.float32(2.0 ** -30)), out):
        oracle.compare(oracle.q4_matvec(w, cols, rows, xi), y)
