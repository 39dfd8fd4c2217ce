"""Batched Q4_0 GEMV (af_q4_gemm: up to 32 vectors per weight pass, crates/cuda-backend/src/batch.rs:113-148,
MAX_BATCH at batch.rs:10) on the GPU against the CPU oracle, every vector within the matvec tolerance
|gpu - ref| <= 1e-4 + 1e-4 |ref| (crates/cuda-backend/src/matvec.rs:175-193)."""
import ctypes

import numpy as np
import pytest

import oracle
from adaforge_amd import _native as N, hip, synth

pytestmark = pytest.mark.gpu


def gemm(w, columns, rows, xs):
    h = N.P()
    N.check(N.lib().af_q4_upload(w.ctypes.data_as(N.u8p), w.size, columns, rows, ctypes.byref(h)))
    try:
        xb, yb = hip.Buffer.from_numpy(np.ascontiguousarray(xs, np.float32)), hip.Buffer(len(xs) * rows)
        N.check(N.lib().af_q4_gemm(h, xb.ptr, len(xs), yb.ptr, None))
        hip.synchronize()
        return yb.numpy().reshape(len(xs), rows)
    finally:
        N.lib().af_q4_free(h)


@pytest.mark.parametrize("tokens", [1, 3, 4, 5, 17, 32])
def test_batched_gemv_matches_oracle_per_vector(tokens):
    cols, rows = 3840, 4096
    w = synth.q4("config0.W", cols, rows)
    rng = np.random.default_rng(tokens)
    xs = rng.standard_normal((tokens, cols)).astype(np.float32)
    xs[0] *= np.float32(0.0) if tokens > 1 else np.float32(1.0)
    y = gemm(w, cols, rows, xs)
    for t in range(tokens):
        oracle.compare(oracle.q4_matvec(w, cols, rows, xs[t]), y[t])
    if tokens > 1:
        assert np.all(y[0] == 0.0)


@pytest.mark.parametrize("columns,rows,tokens", [(32, 5, 7), (96, 77, 32), (640, 77, 9), (15360, 3843, 6),
                                                 (2560, 10240 + 16, 32)])
def test_batched_gemv_ragged_shapes(columns, rows, tokens):
    w = synth.q4(f"bg{columns}x{rows}", columns, rows, signed=True)
    rng = np.random.default_rng(columns + rows)
    xs = (rng.standard_normal((tokens, columns)) * np.exp2(rng.integers(-20, 8, (tokens, columns)))).astype(np.float32)
    y = gemm(w, columns, rows, xs)
    for t in range(tokens):
        oracle.compare(oracle.q4_matvec(w, columns, rows, xs[t]), y[t])


def test_batched_gemv_rejects_empty_and_oversized_batches():
    cols, rows = 64, 16
    w = synth.q4("bgrej", cols, rows)
    h = N.P()
    N.check(N.lib().af_q4_upload(w.ctypes.data_as(N.u8p), w.size, cols, rows, ctypes.byref(h)))
    try:
        xb, yb = hip.Buffer(33 * cols), hip.Buffer(33 * rows)
        for tokens in (0, 33):
            with pytest.raises(N.AfError):
                N.check(N.lib().af_q4_gemm(h, xb.ptr, tokens, yb.ptr, None))
    finally:
        N.lib().af_q4_free(h)
