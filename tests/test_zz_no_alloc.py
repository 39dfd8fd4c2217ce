"""af_q6_gemv_argmax_noalloc (no counterpart in the reference: the head for callers that cannot
allocate) against the allocating entry point af_q6_gemv_argmax on the same inputs: identical
logits (bit for bit: the same kernel and summation order) and identical [id, non-finite flag],
over calls in a row whose second input is smaller, so the shared scratch array's leftover
contents from a larger call must not leak into a smaller one.  The allocation-free variant runs
first, so its device-address lookup happens on its first call in this process."""
import ctypes

import numpy as np
import pytest

import oracle
from adaforge_amd import _native as N
from adaforge_amd import hip, synth

pytestmark = pytest.mark.gpu
L = N.lib


def upload(data, cols, rows):
    h = N.P()
    d = np.ascontiguousarray(data, np.uint8)
    N.check(L().af_q6_upload(d.ctypes.data_as(N.u8p), d.size, cols, rows, ctypes.byref(h)))
    return h


def head(fn, h, x, rows):
    xb, lb, rb = hip.Buffer.from_numpy(np.asarray(x, np.float32)), hip.Buffer(rows), hip.Buffer(2, np.uint32)
    N.check(fn(h, xb.ptr, lb.ptr, rb.ptr, None))
    hip.synchronize()
    return lb.numpy(), rb.numpy()


def test_noalloc_head_matches_allocating_entry_point_on_consecutive_calls():
    cases = [("config2.head", 3840, 262144, "config2.x"),   # 256 workgroups: the largest scratch
             ("noalloc.small", 512, 1000, "noalloc.x"),      # 8 workgroups
             ("noalloc.mid", 1024, 40000, "noalloc.x2")]     # 256 workgroups again
    for name, cols, rows, xname in cases:
        data = synth.q6(name, cols, rows)
        x = synth.normal(xname, cols)
        h = upload(data, cols, rows)
        try:
            lg_free, res_free = head(L().af_q6_gemv_argmax_noalloc, h, x, rows)
            lg_alloc, res_alloc = head(L().af_q6_gemv_argmax, h, x, rows)
        finally:
            L().af_q6_free(h)
        assert np.array_equal(lg_free.view(np.uint32), lg_alloc.view(np.uint32)), name
        assert np.array_equal(res_free, res_alloc), (name, res_free, res_alloc)
        assert res_free[1] == 0 and res_free[0] == oracle.greedy(lg_free), name
        print(f"{name}: {rows} x {cols}, id {res_free[0]}", flush=True)


def test_noalloc_head_rejects_invalid_arguments_before_any_gpu_work():
    rc = L().af_q6_gemv_argmax_noalloc(None, None, None, None, None)
    assert rc == N.AF_ERR_INVALID
